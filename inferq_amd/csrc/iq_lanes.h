// iq_lanes.h -- the exact-order dequant-dot core shared by every kernel.
//
// A wave computes 8 output rows; lane (slot = lane/8, k = lane%8) owns lane
// k of row `slot`, the same lane k as the reference's AVX2 accumulator
// (src/qgemm.rs:175-397): bytes 4k..4k+3 of every 32-value chunk of every
// block.  For each block the lane forms the exact i32 lane sum with v_dot4
// and advances its f32 accumulator with one FMA; the 8 lanes of a row then
// combine with the hsum_f32_8 tree (plus hsum_f32_4 over lanes 0..3 for the
// Q4_K mins).  The result is the reference's, bit for bit, whatever the
// number of input rows.
//
// `lanes_dot` handles R weight rows per lane ("jobs"), each against its own
// list of up to MT activation rows.  All weight loads of a chunk of BC
// blocks of all R jobs are issued before any arithmetic, so one wave keeps
// R * BC * 8 blocks in flight.
#pragma once

#include "iq_device.h"

namespace iq {

struct Q4Scales {
    uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
};
// Six-bit scales and mins of a Q4_K block from its 12 packed bytes
// (u0 = bytes 0..3, u1 = 4..7, u2 = 8..11): scale s is byte s of (sc_lo,
// sc_hi), min s is byte s of (mn_lo, mn_hi).
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

template <int FMT>
struct WT;
template <>
struct WT<kQ4_K> {
    using T = Q4W;
    static constexpr int kBlockBytes = 144;
};
template <>
struct WT<kQ6_K> {
    using T = Q6W;
    static constexpr int kBlockBytes = 210;
};
template <>
struct WT<kQ8_0> {
    using T = Q8W;
    static constexpr int kBlockBytes = 34;
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
        // 4-byte aligned matrix, so the two bytes before it are readable,
        // and every window here ends at least 2 bytes before the block end.
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

// Eight activation dwords of lane k for group g of activation row r.
__device__ __forceinline__ void load_act(const ActView& a, int64_t r, int g, int k, uint32_t av[8]) {
    const uint8_t* ap = (const uint8_t*)a.q + r * a.ldq + (int64_t)g * 256 + 32 * k;
    const u32x4a16 a0 = *(const u32x4a16*)ap, a1 = *(const u32x4a16*)(ap + 16);
    av[0] = a0.x; av[1] = a0.y; av[2] = a0.z; av[3] = a0.w;
    av[4] = a1.x; av[5] = a1.y; av[6] = a1.z; av[7] = a1.w;
}

// Optional per-block lane integers (parity hook).
struct DbgOut {
    int32_t* isum = nullptr;
    int32_t* msum = nullptr;
    int64_t n = 0, row = 0;
    int nbw = 0;
};

// R jobs of one lane: weight row base (nullptr when the row is outside the
// matrix), activation rows arow[r][0..mc[r]) with mc[r] wave-uniform.
// On return out[r][i] holds the product in lane k == 0 of each 8-lane group.
template <int FMT, int MT, int R, int BC, bool DBG = false>
__device__ __forceinline__ void lanes_dot(const uint8_t* const (&wrow)[R], int nbw, const ActView& a,
                                          const int64_t (&arow)[R][MT], const int (&mc)[R], int k,
                                          float (&out)[R][MT], const DbgOut& dbg = DbgOut{}) {
    using W = typename WT<FMT>::T;
    const int ng = a.ng;
    float acc[R][MT], accm[R][MT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < MT; i++) acc[r][i] = accm[r][i] = 0.f;

    for (int g0 = 0; g0 < ng; g0 += BC) {
        W w[R][BC];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int bi = 0; bi < BC; bi++) {
                const int g = g0 + bi;
                if (g < ng && wrow[r] != nullptr) {
                    if constexpr (FMT == kQ4_K) load_q4(wrow[r] + (int64_t)g * 144, k, w[r][bi]);
                    else if constexpr (FMT == kQ6_K) load_q6(wrow[r] + (int64_t)g * 210, k, w[r][bi]);
                    else load_q8(wrow[r], (int64_t)g * 8, nbw, k, w[r][bi]);
                } else {
                    w[r][bi] = W{};
                }
            }
        }
#pragma unroll
        for (int bi = 0; bi < BC; bi++) {
            const int g = g0 + bi;
            if (g >= ng) break;  // uniform
#pragma unroll
            for (int r = 0; r < R; r++) {
                const W& wb = w[r][bi];
                if constexpr (FMT == kQ4_K) {
                    const Q4Scales s = q4_scales(wb.hdr.y, wb.hdr.z, wb.hdr.w);
                    const float xd = f16_to_f32(wb.hdr.x), xdmin = f16_to_f32(wb.hdr.x >> 16);
                    int sc[8];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        sc[t] = byte_of(s.sc_lo, t);
                        sc[t + 4] = byte_of(s.sc_hi, t);
                    }
                    // mins 2k and 2k+1 for lanes k < 4 (lanes 4..7 hold an
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
                        if (mi < mc[r]) {
                            const int64_t ar = arow[r][mi];
                            uint32_t av[8];
                            load_act(a, ar, g, k, av);
                            const float yd = a.d[ar * a.ldd + g];
                            const uint32_t q8s = *(const uint32_t*)(a.s8 + (ar * ng + g) * 8 + 2 * (k & 3));
                            int32_t isum = 0;
#pragma unroll
                            for (int j = 0; j < 4; j++)
                                isum += sc[2 * j] * sdot4(lo[j], av[2 * j], 0) +
                                        sc[2 * j + 1] * sdot4(hi[j], av[2 * j + 1], 0);
                            const int32_t msum =
                                mA * (int32_t)(int16_t)(q8s & 0xffffu) + mB * (int32_t)(int16_t)(q8s >> 16);
                            acc[r][mi] = __builtin_fmaf(yd * xd, (float)isum, acc[r][mi]);
                            accm[r][mi] = __builtin_fmaf(-yd * xdmin, (float)msum, accm[r][mi]);
                            if constexpr (DBG) {
                                if (wrow[r]) {
                                    const int64_t base = ((ar * dbg.n + dbg.row) * dbg.nbw + g);
                                    dbg.isum[base * 8 + k] = isum;
                                    if (k < 4) dbg.msum[base * 4 + k] = msum;
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
                            // bytes q6 - 32: q6 + 0x60 never carries out of a
                            // byte, and xor 0x80 maps it to two's complement
                            v[4 * j + i] = ((lo | hi) + 0x60606060u) ^ 0x80808080u;
                            const int t = 8 * j + 2 * i + hk;  // this lane's scale
                            sc[4 * j + i] = (int)(int8_t)(uint8_t)(wb.sc[t >> 2] >> (8 * (t & 3)));
                        }
                    }
#pragma unroll
                    for (int mi = 0; mi < MT; mi++) {
                        if (mi < mc[r]) {
                            const int64_t ar = arow[r][mi];
                            uint32_t av[8];
                            load_act(a, ar, g, k, av);
                            const float yd = a.d[ar * a.ldd + g];
                            int32_t isum = 0;
#pragma unroll
                            for (int c = 0; c < 8; c++) isum += sc[c] * sdot4(v[c], av[c], 0);
                            acc[r][mi] = __builtin_fmaf(yd * xd, (float)isum, acc[r][mi]);
                            if constexpr (DBG) {
                                if (wrow[r]) dbg.isum[((ar * dbg.n + dbg.row) * dbg.nbw + g) * 8 + k] = isum;
                            }
                        }
                    }
                } else {  // Q8_0: a group is 8 consecutive 32-value blocks
#pragma unroll
                    for (int mi = 0; mi < MT; mi++) {
                        if (mi < mc[r]) {
                            const int64_t ar = arow[r][mi];
                            uint32_t av[8];
                            load_act(a, ar, g, k, av);
                            const float* dp = a.d + ar * a.ldd + (int64_t)g * 8;
                            const f32x4 d0 = *(const f32x4*)dp, d1 = *(const f32x4*)(dp + 4);
                            const float yd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                            for (int c = 0; c < 8; c++) {
                                if ((int64_t)g * 8 + c < nbw) {  // uniform
                                    const int32_t dot = sdot4(wb.q[c], av[c], 0);
                                    acc[r][mi] = __builtin_fmaf(f16_to_f32(wb.d[c]) * yd[c], (float)dot, acc[r][mi]);
                                    if constexpr (DBG) {
                                        if (wrow[r])
                                            dbg.isum[((ar * dbg.n + dbg.row) * dbg.nbw + (int64_t)g * 8 + c) * 8 + k] =
                                                dot;
                                    }
                                }
                            }
                        }
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            float v = hsum8(acc[r][mi]);
            if constexpr (FMT == kQ4_K) v = v + hsum4(accm[r][mi]);
            out[r][mi] = v;
        }
    }
}

}  // namespace iq
