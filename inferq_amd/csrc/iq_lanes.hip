// iq_lanes.hip -- quantised matrix x activation rows, in the reference's
// exact f32 order (src/qgemm.rs:175-397; src/gguf.rs:608-690).
//
// Work mapping.  A wave owns 8 output rows; lane (slot = lane/8, k = lane%8)
// owns lane k of output row `slot`: the same lane k as the reference's AVX2
// accumulator, i.e. bytes 4k..4k+3 of every 32-value chunk of every block.
// The lane walks the blocks in order, forming the exact i32 lane sum with
// v_dot4 and advancing its f32 accumulator with one FMA per block, then the
// 8 lanes of the row combine with the hsum_f32_8 tree (xor 4, 2, 1) -- plus
// hsum_f32_4 over lanes 0..3 for the Q4_K mins.  The result therefore
// equals the reference bit for bit, for every input row count.
//
// Memory.  Weights stream once from HBM in their native GGUF block layout;
// each lane's bytes of a block are 32-byte-strided dwords that 8 lanes read
// as whole 32-byte segments.  All weight loads of a chunk of BC blocks are
// issued before any arithmetic so a wave keeps BC * 8 rows' worth of blocks
// in flight.  Activations (a few KiB) are L2/L1 resident.
#include "iq_device.h"
#include "iq_internal.h"

namespace iq {

namespace {

struct MMArgs {
    const uint8_t* w;
    int64_t n, row_bytes;
    int nbw;  // weight blocks per row (Q8_0: K/32)
    ActView a;
    int m;
    float* y;
    int64_t ldy;
    int32_t* isum;  // optional per-block lane integers
    int32_t* msum;
};

// Six-bit scales and mins of a Q4_K block from its 12 packed bytes
// (u0 = bytes 0..3, u1 = 4..7, u2 = 8..11): scale s is byte s of (lo, hi).
struct Q4Scales {
    uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
};
__device__ __forceinline__ Q4Scales q4_scales(uint32_t u0, uint32_t u1, uint32_t u2) {
    Q4Scales s;
    s.sc_lo = u0 & 0x3f3f3f3fu;
    s.sc_hi = (u2 & 0x0f0f0f0fu) | ((u0 >> 2) & 0x30303030u);
    s.mn_lo = u1 & 0x3f3f3f3fu;
    s.mn_hi = ((u2 >> 4) & 0x0f0f0f0fu) | ((u1 >> 2) & 0x30303030u);
    return s;
}
__device__ __forceinline__ int byte_of(uint32_t v, int i) { return (int)((v >> (8 * i)) & 0xffu); }

struct Q4W {
    u32x4a16 hdr;   // d, dmin, scales[12]
    uint32_t q[4];  // qs dwords 32j + 4k
};
struct Q6W {
    uint32_t ql[4];  // ql windows 32i + 4k
    uint32_t qh[2];  // qh windows 32j + 4k
    uint32_t sc[4];  // scales[16]
    uint32_t d;
};
struct Q8W {
    uint32_t q[8];  // qs window 2 + 4k of the 8 blocks of a group
    uint32_t d[8];
};

__device__ __forceinline__ void load_q4(const uint8_t* blk, int k, Q4W& w) {
    w.hdr = *(const u32x4a16*)blk;
#pragma unroll
    for (int j = 0; j < 4; j++) w.q[j] = ld32(blk + 16 + 32 * j + 4 * k);
}

__device__ __forceinline__ void load_q6(const uint8_t* blk, int k, Q6W& w) {
    if (((uintptr_t)blk & 3u) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) w.ql[i] = ld32(blk + 32 * i + 4 * k);
#pragma unroll
        for (int j = 0; j < 2; j++) w.qh[j] = ld32(blk + 128 + 32 * j + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) w.sc[t] = ld32(blk + 192 + 4 * t);
    } else {
        // A block at 2 (mod 4) always follows another block of the same
        // (4-byte aligned) matrix, so the two bytes before it are readable;
        // every window here ends at least 2 bytes before the block's end.
#pragma unroll
        for (int i = 0; i < 4; i++) w.ql[i] = ld32_m2(blk + 32 * i + 4 * k);
#pragma unroll
        for (int j = 0; j < 2; j++) w.qh[j] = ld32_m2(blk + 128 + 32 * j + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) w.sc[t] = ld32_m2(blk + 192 + 4 * t);
    }
    w.d = ld16(blk + 208);
}

__device__ __forceinline__ void load_q8(const uint8_t* row, int64_t b0, int nbw, int k, Q8W& w) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
        if (b0 + c < nbw) {  // uniform
            const uint8_t* blk = row + (b0 + c) * 34;
            w.q[c] = ld32_a2(blk + 2 + 4 * k);
            w.d[c] = ld16(blk);
        } else {
            w.q[c] = 0;
            w.d[c] = 0;
        }
    }
}

template <int FMT>
struct WT;
template <>
struct WT<kQ4_K> {
    using T = Q4W;
};
template <>
struct WT<kQ6_K> {
    using T = Q6W;
};
template <>
struct WT<kQ8_0> {
    using T = Q8W;
};

// FMT: weight format.  MT: input rows per launch tile (compile-time max).
// BC: 256-value groups whose weight loads are issued together.
template <int FMT, int MT, int BC, bool DBG>
__global__ __launch_bounds__(256) void k_mm_lanes(MMArgs a) {
    using W = typename WT<FMT>::T;
    const int lane = threadIdx.x & 63;
    const int k = lane & 7, slot = lane >> 3;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t row = wave * 8 + slot;
    const bool ok = row < a.n;
    const int m0 = blockIdx.y * MT;
    const int mc = min(MT, a.m - m0);
    const int ng = a.a.ng;
    const uint8_t* wrow = a.w + (ok ? row : 0) * a.row_bytes;

    float acc[MT], accm[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = accm[i] = 0.f;

    for (int g0 = 0; g0 < ng; g0 += BC) {
        W w[BC];
#pragma unroll
        for (int bi = 0; bi < BC; bi++) {
            const int g = g0 + bi;
            if (g < ng && ok) {
                if constexpr (FMT == kQ4_K) load_q4(wrow + (int64_t)g * 144, k, w[bi]);
                else if constexpr (FMT == kQ6_K) load_q6(wrow + (int64_t)g * 210, k, w[bi]);
                else load_q8(wrow, (int64_t)g * 8, a.nbw, k, w[bi]);
            } else {
                w[bi] = W{};
            }
        }
#pragma unroll
        for (int bi = 0; bi < BC; bi++) {
            const int g = g0 + bi;
            if (g >= ng) break;  // uniform
            const W& wb = w[bi];
            if constexpr (FMT == kQ4_K) {
                const Q4Scales s = q4_scales(wb.hdr.y, wb.hdr.z, wb.hdr.w);
                const float xd = f16_to_f32(wb.hdr.x), xdmin = f16_to_f32(wb.hdr.x >> 16);
                int sc[8];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    sc[t] = byte_of(s.sc_lo, t);
                    sc[t + 4] = byte_of(s.sc_hi, t);
                }
                // mins 2k and 2k+1 for lanes k < 4 (lanes 4..7 compute an
                // unused copy)
                const uint32_t mw = (k & 2) ? s.mn_hi : s.mn_lo;
                const int mA = byte_of(mw, 2 * (k & 1)), mB = byte_of(mw, 2 * (k & 1) + 1);
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    lo[j] = wb.q[j] & 0x0f0f0f0fu;
                    hi[j] = (wb.q[j] >> 4) & 0x0f0f0f0fu;
                }
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc) {
                        const int64_t r = m0 + mi;
                        const uint8_t* ap = (const uint8_t*)a.a.q + r * a.a.ldq + (int64_t)g * 256 + 32 * k;
                        const u32x4a16 a0 = *(const u32x4a16*)ap, a1 = *(const u32x4a16*)(ap + 16);
                        const uint32_t av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                        const float yd = a.a.d[r * a.a.ldd + g];
                        const uint32_t q8s = *(const uint32_t*)(a.a.s8 + (r * ng + g) * 8 + 2 * (k & 3));
                        int32_t isum = 0;
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            isum += sc[2 * j] * sdot4(lo[j], av[2 * j], 0) + sc[2 * j + 1] * sdot4(hi[j], av[2 * j + 1], 0);
                        const int32_t msum = mA * (int32_t)(int16_t)(q8s & 0xffffu) + mB * (int32_t)(int16_t)(q8s >> 16);
                        acc[mi] = __builtin_fmaf(yd * xd, (float)isum, acc[mi]);
                        accm[mi] = __builtin_fmaf(-yd * xdmin, (float)msum, accm[mi]);
                        if constexpr (DBG) {
                            if (ok) {
                                a.isum[((r * a.n + row) * a.nbw + g) * 8 + k] = isum;
                                if (k < 4) a.msum[((r * a.n + row) * a.nbw + g) * 4 + k] = msum;
                            }
                        }
                    }
                }
            } else if constexpr (FMT == kQ6_K) {
                const float xd = f16_to_f32(wb.d);
                const int hk = k >= 4;
                uint32_t v[8];
                int sc[8];
#pragma unroll
                for (int j = 0; j < 2; j++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t l = wb.ql[2 * j + (i & 1)];
                        const uint32_t lo = i < 2 ? (l & 0x0f0f0f0fu) : ((l >> 4) & 0x0f0f0f0fu);
                        const uint32_t hi = ((wb.qh[j] >> (2 * i)) & 0x03030303u) << 4;
                        // bytes q6 - 32: q6 + 0x60 never carries, and the xor
                        // with 0x80 maps it to the two's complement of q6-32
                        v[4 * j + i] = ((lo | hi) + 0x60606060u) ^ 0x80808080u;
                        const int t = 8 * j + 2 * i + hk;  // scale index of this lane
                        sc[4 * j + i] = (int)(int8_t)(uint8_t)(wb.sc[t >> 2] >> (8 * (t & 3)));
                    }
                }
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc) {
                        const int64_t r = m0 + mi;
                        const uint8_t* ap = (const uint8_t*)a.a.q + r * a.a.ldq + (int64_t)g * 256 + 32 * k;
                        const u32x4a16 a0 = *(const u32x4a16*)ap, a1 = *(const u32x4a16*)(ap + 16);
                        const uint32_t av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                        const float yd = a.a.d[r * a.a.ldd + g];
                        int32_t isum = 0;
#pragma unroll
                        for (int c = 0; c < 8; c++) isum += sc[c] * sdot4(v[c], av[c], 0);
                        acc[mi] = __builtin_fmaf(yd * xd, (float)isum, acc[mi]);
                        if constexpr (DBG) {
                            if (ok) a.isum[((r * a.n + row) * a.nbw + g) * 8 + k] = isum;
                        }
                    }
                }
            } else {  // Q8_0: a group is 8 consecutive 32-value blocks
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc) {
                        const int64_t r = m0 + mi;
                        const uint8_t* ap = (const uint8_t*)a.a.q + r * a.a.ldq + (int64_t)g * 256 + 32 * k;
                        const u32x4a16 a0 = *(const u32x4a16*)ap, a1 = *(const u32x4a16*)(ap + 16);
                        const uint32_t av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                        const float* dp = a.a.d + r * a.a.ldd + (int64_t)g * 8;
                        const f32x4 d0 = *(const f32x4*)dp, d1 = *(const f32x4*)(dp + 4);
                        const float yd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                        for (int c = 0; c < 8; c++) {
                            if ((int64_t)g * 8 + c < a.nbw) {  // uniform
                                const int32_t dot = sdot4(wb.q[c], av[c], 0);
                                acc[mi] = __builtin_fmaf(f16_to_f32(wb.d[c]) * yd[c], (float)dot, acc[mi]);
                                if constexpr (DBG) {
                                    if (ok) a.isum[((r * a.n + row) * a.nbw + (int64_t)g * 8 + c) * 8 + k] = dot;
                                }
                            }
                        }
                    }
                }
            }
        }
    }

#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        float v = hsum8(acc[mi]);
        if constexpr (FMT == kQ4_K) v = v + hsum4(accm[mi]);
        if (k == 0 && ok && mi < mc) a.y[(int64_t)(m0 + mi) * a.ldy + row] = v;
    }
}

template <int FMT, int MT, int BC>
hipError_t launch_t(const MMArgs& args, bool dbg, hipStream_t s) {
    const int64_t waves = (args.n + 7) / 8;
    dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((args.m + MT - 1) / MT));
    if (dbg) hipLaunchKernelGGL((k_mm_lanes<FMT, MT, BC, true>), grid, dim3(256), 0, s, args);
    else hipLaunchKernelGGL((k_mm_lanes<FMT, MT, BC, false>), grid, dim3(256), 0, s, args);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_fmt(const MMArgs& args, bool dbg, hipStream_t s) {
    constexpr int BC1 = FMT == kQ8_0 ? 4 : 8;
    constexpr int BCn = FMT == kQ8_0 ? 2 : 4;
    if (args.m <= 1) return launch_t<FMT, 1, BC1>(args, dbg, s);
    if (args.m <= 2) return launch_t<FMT, 2, BCn>(args, dbg, s);
    if (args.m <= 4) return launch_t<FMT, 4, BCn>(args, dbg, s);
    if (args.m <= 8) return launch_t<FMT, 8, BCn>(args, dbg, s);
    return launch_t<FMT, 16, BCn>(args, dbg, s);
}

}  // namespace

hipError_t launch_matmul_lanes(const WeightView& w, const ActView& a, float* y, int64_t ldy, int32_t* isum,
                               int32_t* msum, hipStream_t s) {
    MMArgs args;
    args.w = w.w;
    args.n = w.rows;
    args.row_bytes = w.row_bytes;
    args.nbw = (int)(w.dtype == kQ8_0 ? w.cols / 32 : w.cols / 256);
    args.a = a;
    args.m = a.m;
    args.y = y;
    args.ldy = ldy;
    args.isum = isum;
    args.msum = msum;
    if (args.n == 0 || args.m == 0) return hipSuccess;
    const bool dbg = isum != nullptr;
    switch (w.dtype) {
    case kQ4_K: return launch_fmt<kQ4_K>(args, dbg, s);
    case kQ6_K: return launch_fmt<kQ6_K>(args, dbg, s);
    case kQ8_0: return launch_fmt<kQ8_0>(args, dbg, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace iq
