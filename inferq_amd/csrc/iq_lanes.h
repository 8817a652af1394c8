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
// Q5_K: the Q4_K header and nibbles plus the lane's dword of qh (bit 2j of
// byte l is the fifth bit of weight 64j + l, bit 2j + 1 that of 64j + 32 + l).
struct Q5W {
    u32x4a16 hdr;   // d, dmin, scales[12]
    uint32_t qh;    // qh dword 4k
    uint32_t q[4];  // qs dwords 32j + 4k
};
// Q6_K lane data.  A block at 2 (mod 4) is loaded as aligned dword pairs
// whose byte funnel shift (by `sh` bytes) is applied at use, so that a burst
// of loads is never interrupted by waits for earlier ones.
struct Q6W {
    u32x2 ql[4];  // ql windows 32i + 4k
    u32x2 qh[2];  // qh windows 32j + 4k
    u32x2 sc[4];  // scales[16]
    uint32_t d;
    uint32_t sh;
};
__device__ __forceinline__ uint32_t q6win(u32x2 v, uint32_t sh) { return __builtin_amdgcn_alignbyte(v.y, v.x, sh); }
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
struct WT<kQ5_K> {
    using T = Q5W;
    static constexpr int kBlockBytes = 176;
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

// 176-byte blocks keep the 16-byte alignment of the row.
__device__ __forceinline__ void load_q5(const uint8_t* blk, int k, Q5W& w) {
    w.hdr = *(const u32x4a16*)blk;
    w.qh = ld32(blk + 16 + 4 * k);
#pragma unroll
    for (int j = 0; j < 4; j++) w.q[j] = ld32(blk + 48 + 32 * j + 4 * k);
}

// Q6_K block known to start at 0 (mod 4): exact dword loads.
__device__ __forceinline__ void load_q6_a0(const uint8_t* blk, int k, Q6W& w) {
#pragma unroll
    for (int i = 0; i < 4; i++) w.ql[i] = u32x2{ld32(blk + 32 * i + 4 * k), 0u};
#pragma unroll
    for (int j = 0; j < 2; j++) w.qh[j] = u32x2{ld32(blk + 128 + 32 * j + 4 * k), 0u};
    const u32x4 sc = *(const u32x4*)(blk + 192);
    w.sc[0] = u32x2{sc.x, 0u};
    w.sc[1] = u32x2{sc.y, 0u};
    w.sc[2] = u32x2{sc.z, 0u};
    w.sc[3] = u32x2{sc.w, 0u};
    w.d = ld16(blk + 208);
    w.sh = 0;
}
// Q6_K block known to start at 2 (mod 4): each window is the aligned dword
// pair around it.  The two bytes before the block belong to the previous
// block of the same row, and every window ends at least 2 bytes before the
// block's end, so nothing outside the matrix is read.
__device__ __forceinline__ void load_q6_a2(const uint8_t* blk, int k, Q6W& w) {
#pragma unroll
    for (int i = 0; i < 4; i++) w.ql[i] = *(const u32x2*)(blk + 32 * i + 4 * k - 2);
#pragma unroll
    for (int j = 0; j < 2; j++) w.qh[j] = *(const u32x2*)(blk + 128 + 32 * j + 4 * k - 2);
#pragma unroll
    for (int t = 0; t < 4; t++) w.sc[t] = *(const u32x2*)(blk + 192 + 4 * t - 2);
    w.d = ld16(blk + 208);
    w.sh = 2;
}

__device__ __forceinline__ void load_q6(const uint8_t* blk, int k, Q6W& w) {
    if (((uintptr_t)blk & 3u) == 0) load_q6_a0(blk, k, w);
    else load_q6_a2(blk, k, w);
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

// ---- one block of one row for lane k, split into a per-row decode (shared
// by every input row) and a per-input dot.  Term values are exactly the
// reference's: isum/msum the i32 lanes, d = y.d * xd, dmin = -y.d * xdmin.
struct Q4Dec {
    uint32_t lo[4], hi[4];
    int sc[8];
    int mA, mB;
    float xd, xdmin;
};
__device__ __forceinline__ Q4Dec q4_decode(const Q4W& wb, int k) {
    Q4Dec r;
    const Q4Scales s = q4_scales(wb.hdr.y, wb.hdr.z, wb.hdr.w);
    r.xd = f16_to_f32(wb.hdr.x);
    r.xdmin = f16_to_f32(wb.hdr.x >> 16);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        r.sc[t] = byte_of(s.sc_lo, t);
        r.sc[t + 4] = byte_of(s.sc_hi, t);
    }
    // mins 2k and 2k+1 for lanes k < 4 (lanes 4..7 hold an unused copy)
    const uint32_t mw = (k & 2) ? s.mn_hi : s.mn_lo;
    r.mA = byte_of(mw, 2 * (k & 1));
    r.mB = byte_of(mw, 2 * (k & 1) + 1);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r.lo[j] = wb.q[j] & 0x0f0f0f0fu;
        r.hi[j] = (wb.q[j] >> 4) & 0x0f0f0f0fu;
    }
    return r;
}
// Q5_K decodes into the Q4_K form: the 5-bit weights (0..31) go where the
// nibbles were, so q4_dot gives the lane integers of ggml's
// vec_dot_q5_K_q8_K (the same maddubs/madd lane structure as Q4_K).
__device__ __forceinline__ Q4Dec q5_decode(const Q5W& wb, int k) {
    Q4W as4;
    as4.hdr = wb.hdr;
#pragma unroll
    for (int j = 0; j < 4; j++) as4.q[j] = wb.q[j];
    Q4Dec r = q4_decode(as4, k);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r.lo[j] |= ((wb.qh >> (2 * j)) & 0x01010101u) << 4;
        r.hi[j] |= ((wb.qh >> (2 * j + 1)) & 0x01010101u) << 4;
    }
    return r;
}

// Sum of an int over lanes 0..3 of each group of 8 (lanes 4..7 hold copies
// of lanes 0..3), in every lane: (l0 + l1) + (l2 + l3), exact.
__device__ __forceinline__ int32_t isum_quad(int32_t v) {
    v = v + __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    v = v + __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    return v;
}

__device__ __forceinline__ void q4_dot(const Q4Dec& r, const uint32_t (&av)[8], float yd, uint32_t q8s, int32_t& isum,
                                       int32_t& msum, float& d, float& dmin) {
    isum = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        isum = imad24(r.sc[2 * j], sdot4(r.lo[j], av[2 * j], 0), isum);
        isum = imad24(r.sc[2 * j + 1], sdot4(r.hi[j], av[2 * j + 1], 0), isum);
    }
    msum = imad24(r.mA, (int32_t)(int16_t)(q8s & 0xffffu), imad24(r.mB, (int32_t)(int16_t)(q8s >> 16), 0));
    d = yd * r.xd;
    dmin = -yd * r.xdmin;
}

struct Q6Dec {
    uint32_t v[8];
    int sc[8];
    float xd;
};
__device__ __forceinline__ Q6Dec q6_decode(const Q6W& wb, int k) {
    Q6Dec r;
    r.xd = f16_to_f32(wb.d);
    const int hk = k >= 4;
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l = q6win(wb.ql[2 * j + (i & 1)], wb.sh);
            const uint32_t lo = i < 2 ? (l & 0x0f0f0f0fu) : ((l >> 4) & 0x0f0f0f0fu);
            const uint32_t hi = ((q6win(wb.qh[j], wb.sh) >> (2 * i)) & 0x03030303u) << 4;
            // bytes q6 - 32: q6 + 0x60 never carries out of a byte, and xor
            // 0x80 maps it to two's complement
            r.v[4 * j + i] = ((lo | hi) + 0x60606060u) ^ 0x80808080u;
            const int t = 8 * j + 2 * i + hk;  // this lane's scale
            r.sc[4 * j + i] = (int)(int8_t)(uint8_t)(q6win(wb.sc[t >> 2], wb.sh) >> (8 * (t & 3)));
        }
    }
    return r;
}
__device__ __forceinline__ void q6_dot(const Q6Dec& r, const uint32_t (&av)[8], float yd, int32_t& isum, float& d) {
    isum = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) isum = imad24(r.sc[c], sdot4(r.v[c], av[c], 0), isum);
    d = yd * r.xd;
}

// Optional per-block lane integers (parity hook).
struct DbgOut {
    int32_t* isum = nullptr;
    int32_t* msum = nullptr;
    int64_t n = 0, row = 0;
    int nbw = 0;
};

// Issue the weight loads of blocks [g0, g0+BC) of R rows (nullptr rows and
// blocks past ng load nothing and decode as zero).
template <int FMT, int R, int BC>
__device__ __forceinline__ void lanes_load(const uint8_t* const (&wrow)[R], int g0, int ng, int nbw, int k,
                                           typename WT<FMT>::T (&w)[R][BC]) {
    using W = typename WT<FMT>::T;
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int bi = 0; bi < BC; bi++) {
            const int g = g0 + bi;
            if (g < ng && wrow[r] != nullptr) {
                if constexpr (FMT == kQ4_K) load_q4(wrow[r] + (int64_t)g * 144, k, w[r][bi]);
                else if constexpr (FMT == kQ5_K) load_q5(wrow[r] + (int64_t)g * 176, k, w[r][bi]);
                else if constexpr (FMT == kQ6_K) load_q6(wrow[r] + (int64_t)g * 210, k, w[r][bi]);
                else load_q8(wrow[r], (int64_t)g * 8, nbw, k, w[r][bi]);
            } else {
                w[r][bi] = W{};
            }
        }
    }
}

// lanes_load for exactly NG blocks per row with no control flow at all, so
// the whole burst issues back to back: every wrow[r] must be a readable row
// (callers point unused jobs at a used row and discard the results).
template <int FMT, int R, int NG>
__device__ __forceinline__ void lanes_load_exact(const uint8_t* const (&wrow)[R], int k,
                                                 typename WT<FMT>::T (&w)[R][NG]) {
    static_assert(FMT != kQ8_0, "lanes_load_exact covers the K-quants");
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int g = 0; g < NG; g++) {
            if constexpr (FMT == kQ4_K) {
                load_q4(wrow[r] + (int64_t)g * 144, k, w[r][g]);
            } else if constexpr (FMT == kQ5_K) {
                load_q5(wrow[r] + (int64_t)g * 176, k, w[r][g]);
            } else if constexpr (NG % 2 == 0) {
                // rows of an even number of 210-byte blocks are 4-byte
                // aligned, so block g starts at 2g (mod 4)
                if (g % 2 == 0) load_q6_a0(wrow[r] + (int64_t)g * 210, k, w[r][g]);
                else load_q6_a2(wrow[r] + (int64_t)g * 210, k, w[r][g]);
            } else {
                load_q6(wrow[r] + (int64_t)g * 210, k, w[r][g]);
            }
        }
    }
    // keep every consumer of the loaded data below the whole burst, so no
    // register of the burst is recycled (and waited for) mid-burst
    __builtin_amdgcn_sched_barrier(0);
}

// Advance the lane accumulators over blocks [g0, g0+BC) (see lanes_dot).
template <int FMT, int MT, int R, int BC, bool DBG = false>
__device__ __forceinline__ void lanes_accumulate(const typename WT<FMT>::T (&w)[R][BC], const uint8_t* const (&wrow)[R],
                                                 int g0, int ng, int nbw, const ActView& a,
                                                 const int64_t (&arow)[R][MT], const int (&mc)[R], int k,
                                                 float (&acc)[R][MT], float (&accm)[R][MT],
                                                 const DbgOut& dbg = DbgOut{}) {
    using W = typename WT<FMT>::T;
#pragma unroll
    for (int bi = 0; bi < BC; bi++) {
        const int g = g0 + bi;
        if (g >= ng) break;  // uniform
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (mc[r] <= 0) continue;  // uniform: a job with no rows reads nothing
            const W& wb = w[r][bi];
            if constexpr (FMT == kQ4_K) {
                const Q4Dec dec = q4_decode(wb, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc[r]) {
                        const int64_t ar = arow[r][mi];
                        uint32_t av[8];
                        load_act(a, ar, g, k, av);
                        const float yd = a.d[ar * a.ldd + g];
                        const uint32_t q8s = *(const uint32_t*)(a.s8 + (ar * a.ng + g) * 8 + 2 * (k & 3));
                        int32_t isum, msum;
                        float d, dmin;
                        q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
                        acc[r][mi] = __builtin_fmaf(d, (float)isum, acc[r][mi]);
                        accm[r][mi] = __builtin_fmaf(dmin, (float)msum, accm[r][mi]);
                        if constexpr (DBG) {
                            if (wrow[r]) {
                                const int64_t base = ((ar * dbg.n + dbg.row) * dbg.nbw + g);
                                dbg.isum[base * 8 + k] = isum;
                                if (k < 4) dbg.msum[base * 4 + k] = msum;
                            }
                        }
                    }
                }
            } else if constexpr (FMT == kQ5_K) {
                // lanes as Q4_K; the mins join one f32 scalar per row,
                // summs = summs + dmin * (m . q8s), multiply then add
                const Q4Dec dec = q5_decode(wb, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc[r]) {
                        const int64_t ar = arow[r][mi];
                        uint32_t av[8];
                        load_act(a, ar, g, k, av);
                        const float yd = a.d[ar * a.ldd + g];
                        const uint32_t q8s = *(const uint32_t*)(a.s8 + (ar * a.ng + g) * 8 + 2 * (k & 3));
                        int32_t isum, msum;
                        float d, dmin;
                        q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
                        acc[r][mi] = __builtin_fmaf(d, (float)isum, acc[r][mi]);
                        const int32_t mtot = isum_quad(msum);
                        accm[r][mi] = accm[r][mi] + dmin * (float)mtot;
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
                const Q6Dec dec = q6_decode(wb, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (mi < mc[r]) {
                        const int64_t ar = arow[r][mi];
                        uint32_t av[8];
                        load_act(a, ar, g, k, av);
                        const float yd = a.d[ar * a.ldd + g];
                        int32_t isum;
                        float d;
                        q6_dot(dec, av, yd, isum, d);
                        acc[r][mi] = __builtin_fmaf(d, (float)isum, acc[r][mi]);
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
                                        dbg.isum[((ar * dbg.n + dbg.row) * dbg.nbw + (int64_t)g * 8 + c) * 8 + k] = dot;
                                }
                            }
                        }
                    }
                }
            }
        }
    }
}

// The 8 lanes of each row combine: hsum_f32_8 (+ hsum_f32_4 of the Q4_K
// mins, + the Q5_K mins scalar).  out[r][i] is valid in lane k == 0 of each group.
template <int FMT, int MT, int R>
__device__ __forceinline__ void lanes_finish(const float (&acc)[R][MT], const float (&accm)[R][MT],
                                             float (&out)[R][MT]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            float v = hsum8(acc[r][mi]);
            if constexpr (FMT == kQ4_K) v = v + hsum4(accm[r][mi]);
            if constexpr (FMT == kQ5_K) v = v + accm[r][mi];  // every lane holds summs
            out[r][mi] = v;
        }
    }
}

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
        lanes_load<FMT, R, BC>(wrow, g0, ng, nbw, k, w);
        lanes_accumulate<FMT, MT, R, BC, DBG>(w, wrow, g0, ng, nbw, a, arow, mc, k, acc, accm, dbg);
    }
    lanes_finish<FMT, MT, R>(acc, accm, out);
}

}  // namespace iq
