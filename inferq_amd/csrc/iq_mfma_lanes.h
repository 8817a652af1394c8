// iq_mfma_lanes.h -- the reference's exact per-lane products on int8 MFMA
// (Q4_K or Q6_K weights), shared by the grouped MoE kernels and the dense
// multi-row kernels, in three forms:
//   ml_product     up to 16 RT activation rows x 64 weight rows;
//   ml_product_pk  up to 8 activation rows x 64 weight rows, two reference
//                  lanes per v_mfma_i32_16x16x64_i8;
//   ml_product_sk  up to 8 activation rows x 16 weight rows, the blocks
//                  split over the waves and the f32 chains handed on.
//
// The reference's lane k (src/qgemm.rs:175-346) owns bytes 4k..4k+3 of every
// 32-value chunk c of a block: isum_k = sum_c sc_c * dot4(w[c][k], a[c][k])
// with one scale per dword, and it advances acc_k = fma(y.d * x.d, isum_k,
// acc_k) once per block; the eight lanes meet in hsum_f32_8 (Q4_K mins: four
// lanes, hsum_f32_4).  Int8 MFMAs whose K index runs over (c, e) for one
// fixed k yield isum_k for a whole 16 x 16 tile: A holds the activation
// dwords (c, k), c = 0..7, which the activation layout keeps contiguous
// (dword 8k + c), and B the weight dwords (c, k) with each dword's scale
// folded in.  Scaled weights exceed int8, so each is split into two int8
// streams whose integer sums recombine exactly: Q4_K sc*q = 8 (sc >> 3) q +
// (sc & 7) q; Q6_K sc*(q - 32) = 256 hi + lo with hi in -16..16 and lo in
// -128..127; Q5_K (q = nibble + 16 bit) into three, 8 (sc >> 3) nibble +
// (sc & 7) nibble + 16 sc bit.  Q5_K's mins join one f32 scalar per row
// and block, summs = summs + dmin * (m . s) (ggml's vec_dot_q5_K_q8_K), the
// integer m . s from one f16 MFMA (exact: integers below 2^24).  The Q4_K mins msum_k = m_2k s_2k + m_2k+1 s_2k+1 (s = 32-value
// activation sums) come from an f16 MFMA over the 16-value sums (integers
// below 2^24: exact).  A lane keeps the f32 chains of all eight reference
// lanes for its outputs and joins them at the end in the hsum trees' order,
// ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) plus (m0+m2) + (m1+m3).
#pragma once

#include <type_traits>

#include "iq_lanes.h"

namespace iq {

typedef int v4i_ml __attribute__((ext_vector_type(4)));
typedef float v4f_ml __attribute__((ext_vector_type(4)));
typedef _Float16 v4h_ml __attribute__((ext_vector_type(4)));
typedef short s16x2_ml __attribute__((ext_vector_type(2)));

constexpr int kMlCols = 64;  // weight rows per tile (16 per wave)
constexpr int kMlAS = 272;   // LDS stride of an activation row (256 + pad)

template <int FMT>
struct MlFmt;
template <>
struct MlFmt<kQ4_K> {
    static constexpr int BB = 144;  // block bytes
    static constexpr int BS = 144;  // LDS bytes per staged row-block
    static constexpr int NL = 9;    // staging loads per row-block (16 bytes each)
    static constexpr bool kMins = true;
};
// Q5_K (ml_product only): the Q4_K header, qh at 16..47, qs at 48..175;
// 176-byte columns (11 groups of 16 bytes, coprime with the 16 bank groups)
template <>
struct MlFmt<kQ5_K> {
    static constexpr int BB = 176;
    static constexpr int BS = 176;
    static constexpr int NL = 11;
    static constexpr bool kMins = true;
};
template <>
struct MlFmt<kQ6_K> {
    static constexpr int BB = 210;
    // the block's 212-byte dword window, padded to 60 dwords: the 16
    // columns of a fragment read dwords 60 j + o, 16 distinct banks
    static constexpr int BS = 240;
    static constexpr int NL = 14;   // staging loads per row-block (16 bytes each)
    static constexpr bool kMins = false;
};

// LDS stage of RT 16-row tiles: A int8 [16 RT][kMlAS], B [64][BS], D f32
// [16 RT], H f16 [16 RT][16].
template <int FMT, int RT>
struct MlStage {
    static constexpr int R = 16 * RT;
    static constexpr int A = 0;
    static constexpr int B = A + R * kMlAS;
    static constexpr int D = B + kMlCols * MlFmt<FMT>::BS;
    static constexpr int H = D + R * 4;
    static constexpr int END = H + (MlFmt<FMT>::kMins ? R * 32 : 0);
};


// Four unsigned six-bit values u (bytes) times a signed scale sc, minus
// 32 sc: p = sc * (u - 32) in -4064..4096, split p = 256 hi + lo with hi in
// -16..16 and lo in -128..127 (byte order kept).  P = p + 128 is formed in
// 16-bit lanes (bytes 0, 2 and bytes 1, 3 of u); as a 16-bit two's
// complement value its high byte is floor(P / 256) = hi and its low byte
// is lo + 128, so both streams are byte picks of P.
__device__ __forceinline__ void ml_q6_scaled_split(uint32_t u, int sc, uint32_t& lo, uint32_t& hi) {
    const s16x2_ml s2 = {(short)sc, (short)sc}, c2 = {(short)(128 - 32 * sc), (short)(128 - 32 * sc)};
    const s16x2_ml u02 = __builtin_bit_cast(s16x2_ml, u & 0x00ff00ffu);                         // bytes 0, 2
    const s16x2_ml u13 = __builtin_bit_cast(s16x2_ml, __builtin_amdgcn_perm(0u, u, 0x0c030c01u));  // bytes 1, 3
    const uint32_t p02 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u02 * s2 + c2));
    const uint32_t p13 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u13 * s2 + c2));
    hi = __builtin_amdgcn_perm(p13, p02, 0x07030501u);                // high bytes, interleaved
    lo = __builtin_amdgcn_perm(p13, p02, 0x06020400u) ^ 0x80808080u;  // low bytes - 128
}

// The 4 bytes at byte offset o of a block staged with a dword shift of sh
// (0 or 2) bytes.
__device__ __forceinline__ uint32_t ml_lds_win(const uint8_t* row, int sh, int o) {
    const uint32_t w0 = *(const uint32_t*)(row + o), w1 = *(const uint32_t*)(row + o + 4);
    return __builtin_amdgcn_alignbyte(w1, w0, (uint32_t)sh);
}

// N consecutive windows of ml_lds_win: out[i] = the 4 bytes at byte offset
// o + 4 i (o 16-byte aligned) of a block staged with shift sh, from N + 1
// dwords read as 16-byte (and one 4-byte) LDS accesses, which spread the
// lanes of a fragment over the banks where per-window 4-byte reads would
// pile up to four lanes on a bank.
template <int N>
__device__ __forceinline__ void ml_lds_span(const uint8_t* row, int sh, int o, uint32_t (&out)[N]) {
    static_assert(N % 4 == 0, "span of whole 16-byte groups");
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
        const u32x4a16 v = *(const u32x4a16*)(row + o + 16 * i);
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
    w[N] = *(const uint32_t*)(row + o + 4 * N);
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], (uint32_t)sh);
}

// The same reads for a shift known at compile time (a Q6_K block's shift is
// 2 (b & 1) in rows whose byte length is a multiple of 4): at shift 0 the
// window is the bytes themselves, with no realignment and no extra dword.
template <int S>
using MlShift = std::integral_constant<int, S>;
template <int S>
__device__ __forceinline__ uint32_t ml_lds_win(const uint8_t* row, MlShift<S>, int o) {
    if constexpr (S == 0) return *(const uint32_t*)(row + o);
    else return ml_lds_win(row, S, o);
}
template <int N, int S>
__device__ __forceinline__ void ml_lds_span(const uint8_t* row, MlShift<S>, int o, uint32_t (&out)[N]) {
    if constexpr (S == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; i++) {
            const u32x4a16 v = *(const u32x4a16*)(row + o + 16 * i);
            out[4 * i] = v.x;
            out[4 * i + 1] = v.y;
            out[4 * i + 2] = v.z;
            out[4 * i + 3] = v.w;
        }
    } else {
        ml_lds_span<N>(row, S, o, out);
    }
}

// Operands of one tile.  Activation row rr (0 .. 16 RT - 1) of the tile is
// row arow(rr) of aq (Q8K in the lane-transposed layout, ldq bytes a row),
// ad (block scales, ldd a row) and hs ([row][nb][16] f16 16-value sums,
// Q4_K only).  Weight row c (0..63) of the tile is row brow(c) of the
// matrix at b0 (c < bsplit) or b1 (c >= bsplit), brow_bytes a row, nb blocks
// along K.  All byte offsets within a matrix fit 32 bits.
struct MlOperands {
    const int8_t* aq;
    int64_t ldq;
    const float* ad;
    int64_t ldd;
    const _Float16* hs;
    const uint8_t* b0;
    const uint8_t* b1;
    int bsplit;
    int64_t brow_bytes;
    int nb;
};

// The tile's products on a 256-thread workgroup: lane (q = l / 16, j = l % 16)
// of wave w ends with v[r] = output (row 16 (r / 4) + 4 q + r % 4, weight
// row 16 w + j), r < 4 RT.  `st` is the caller's LDS (2 stages).
//
// Fragments of v_mfma_i32_16x16x32_i8 for lane l (q = l / 16, j = l % 16):
// A row j, K 8q..8q+7; B column j, the same K; the result holds rows
// 4q..4q+3 of column j.  For lane k of the reference, K 8q..8q+7 are the
// dwords (c, k) with c = 2q, 2q+1.
template <int FMT, int RT, class ARow, class BRow>
__device__ __forceinline__ void ml_product(const MlOperands& op, ARow arow, BRow brow, uint8_t (*st)[MlStage<FMT, RT>::END],
                                           float (&v)[4 * RT]) {
    using F = MlFmt<FMT>;
    using L = MlStage<FMT, RT>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int nb = op.nb;

    // ---- staging: every thread owns fixed slots, the same for every block.
    // Sources are a wave-uniform base plus a 32-bit offset.
    constexpr int kA = L::R * 16;              // 16-byte A chunks
    constexpr int kB = kMlCols * F::NL;        // 16-byte B chunks
    constexpr int kAPer = (kA + 255) / 256;    // 1 or 2
    constexpr int kBPer = (kB + 255) / 256;    // Q4_K 3, Q6_K 4
    uint32_t a_src[kAPer];
    int a_off[kAPer];
#pragma unroll
    for (int i = 0; i < kAPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kA - 1);
        const int rr = t >> 4, part = t & 15;
        a_src[i] = (uint32_t)(arow(rr) * op.ldq + 16 * part);
        a_off[i] = (int)threadIdx.x + 256 * i < kA ? L::A + rr * kMlAS + 16 * part : -1;
    }
    // B chunk t: column t / NL, part t % NL; columns past bsplit come from
    // the second matrix.  Q6_K: the block's dword window (it starts 0 or 2
    // bytes before the block) as 13 chunks plus one ending at its last byte.
    uint32_t b_src[kBPer];
    int b_off[kBPer];
    bool b_hi[kBPer];
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kB - 1);
        const int c2 = t / F::NL, part = t - c2 * F::NL;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        b_hi[i] = c2 >= op.bsplit;
        b_src[i] = (uint32_t)(brow(c2) * op.brow_bytes + po);
        b_off[i] = (int)threadIdx.x + 256 * i < kB ? L::B + c2 * F::BS + po : -1;
    }
    // D (row scales) on threads 0 .. R-1, H (16-value sums, Q4_K) on 64 .. 64 + 2R - 1
    static_assert((L::R & (L::R - 1)) == 0, "tile rows");
    const int tD = threadIdx.x, tH = threadIdx.x - 64;
    const int64_t d_row = arow(tD & (L::R - 1));
    const int64_t h_row = arow((tH >> 1) & (L::R - 1));  // in range for idle threads too

    v4i_ml sa[kAPer];
    u32x4 sb[kBPer];
    float sd = 0.f;
    v4i_ml sh16 = {};
    auto issue = [&](int b) {
        const int8_t* abase = op.aq + (int64_t)b * 256;
#pragma unroll
        for (int i = 0; i < kAPer; i++) sa[i] = *(const v4i_ml*)(abase + a_src[i]);
        const int64_t boff = FMT == kQ6_K ? ((int64_t)b * F::BB) & ~(int64_t)3 : (int64_t)b * F::BB;
#pragma unroll
        for (int i = 0; i < kBPer; i++) sb[i] = *(const u32x4*)((b_hi[i] ? op.b1 : op.b0) + boff + b_src[i]);
        if (tD < L::R) sd = op.ad[d_row * op.ldd + b];
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 2 * L::R) sh16 = *(const v4i_ml*)(op.hs + (h_row * nb + b) * 16 + 8 * (tH & 1));
    };
    auto park = [&](uint8_t* s) {
#pragma unroll
        for (int i = 0; i < kAPer; i++)
            if (a_off[i] >= 0) *(v4i_ml*)(s + a_off[i]) = sa[i];
#pragma unroll
        for (int i = 0; i < kBPer; i++)
            if (b_off[i] >= 0) *(u32x4*)(s + b_off[i]) = sb[i];
        if (tD < L::R) *(float*)(s + L::D + 4 * tD) = sd;
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 2 * L::R) *(v4i_ml*)(s + L::H + 32 * (tH >> 1) + 16 * (tH & 1)) = sh16;
    };

    const int col = 16 * wave + jj;  // this lane's staged weight row
    // output r of the lane: tile r / 4, row 16 (r / 4) + 4 q + r % 4;
    // acc[k]: the f32 chain of reference lane k, accm[k] of mins lane k
    float acc[8][4 * RT], accm[4][4 * RT];
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
        for (int r = 0; r < 4 * RT; r++) acc[k][r] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int r = 0; r < 4 * RT; r++) accm[k][r] = 0.f;
    issue(0);
    park(st[0]);
    lds_barrier();
    for (int b = 0; b < nb; b++) {
        const uint8_t* S = st[b & 1];
        if (b + 1 < nb) issue(b + 1);
        const int sh = FMT == kQ6_K ? (int)(((int64_t)b * F::BB) & 3) : 0;
        const uint8_t* bcol = S + L::B + col * F::BS;
        float dd[4 * RT], dm[4 * RT];
        float xd, xdm = 0.f;
        uint32_t s6a = 0, s6b = 0;  // Q4_K: six-bit scales of sub-blocks 2q, 2q+1
        uint32_t q6s = 0;           // Q6_K: scale bytes 4q..4q+3
        Q4Scales sc{};
        // Q4_K: the lane's qs bytes 32q .. 32q + 31 (dword k for reference
        // lane k), read as two 16-byte LDS accesses per block: the
        // columns' 144-byte stride puts 16 lanes' 16-byte groups on 16
        // distinct bank groups, where eight 4-byte reads per block would
        // put four lanes on each bank
        u32x4a16 qs4[2] = {};
        u32x4a16 qh4[2] = {};  // Q5_K: qh bytes 0..31 (dword k: the fifth bits of lane k)
        // Q6_K: the lane's ql and qh windows for reference lanes k = 0..7
        uint32_t l0s[8] = {}, l1s[8] = {}, qhs[8] = {};
        if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
            constexpr int QO = FMT == kQ5_K ? 48 : 16;  // offset of qs
            const u32x4a16 hdr = *(const u32x4a16*)bcol;
            xd = f16_to_f32(hdr.x);
            xdm = f16_to_f32(hdr.x >> 16);
            sc = q4_scales(hdr.y, hdr.z, hdr.w);
            const uint32_t sw = q < 2 ? sc.sc_lo : sc.sc_hi;
            s6a = byte_of(sw, 2 * (q & 1));
            s6b = byte_of(sw, 2 * (q & 1) + 1);
            qs4[0] = *(const u32x4a16*)(bcol + QO + 32 * q);
            qs4[1] = *(const u32x4a16*)(bcol + QO + 16 + 32 * q);
            if constexpr (FMT == kQ5_K) {
                qh4[0] = *(const u32x4a16*)(bcol + 16);
                qh4[1] = *(const u32x4a16*)(bcol + 32);
            }
        } else {
            xd = f16_to_f32(ml_lds_win(bcol, sh, 208) & 0xffffu);
            q6s = ml_lds_win(bcol, sh, 192 + 4 * q);
            ml_lds_span<8>(bcol, sh, 64 * (q >> 1), l0s);
            ml_lds_span<8>(bcol, sh, 64 * (q >> 1) + 32, l1s);
            ml_lds_span<8>(bcol, sh, 128 + 32 * (q >> 1), qhs);
        }
#pragma unroll
        for (int r = 0; r < 4 * RT; r++) {
            const float yd = *(const float*)(S + L::D + 4 * (16 * (r >> 2) + 4 * q + (r & 3)));
            dd[r] = yd * xd;
            if constexpr (F::kMins) dm[r] = -yd * xdm;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t w1[2], w2[2], w3[2] = {0u, 0u};
            int mul;  // isum = mul * (stream 1) + (stream 2) (+ 16 * (stream 3), Q5_K)
            if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
                const uint32_t qd = qs4[k >> 2][k & 3];
                const uint32_t lo = qd & 0x0f0f0f0fu, hi = (qd >> 4) & 0x0f0f0f0fu;
                w1[0] = bytes_mul_small(lo, s6a >> 3);
                w1[1] = bytes_mul_small(hi, s6b >> 3);
                w2[0] = bytes_mul_small(lo, s6a & 7u);
                w2[1] = bytes_mul_small(hi, s6b & 7u);
                if constexpr (FMT == kQ5_K) {
                    // fifth bits of chunks 2q, 2q + 1 (bits 2q, 2q + 1 of
                    // qh bytes 4k .. 4k + 3), each byte 0 or the scale
                    const uint32_t qhd = qh4[k >> 2][k & 3];
                    w3[0] = bytes_mul_small((qhd >> (2 * q)) & 0x01010101u, s6a);
                    w3[1] = bytes_mul_small((qhd >> (2 * q + 1)) & 0x01010101u, s6b);
                }
                mul = 8;
            } else {
                const int hk = k >= 4;
                const uint32_t l0 = l0s[k], l1 = l1s[k], qh = qhs[k];
#pragma unroll
                for (int cc = 0; cc < 2; cc++) {
                    const uint32_t l = cc ? l1 : l0;
                    const uint32_t lo4 = (q & 1) ? ((l >> 4) & 0x0f0f0f0fu) : (l & 0x0f0f0f0fu);
                    const uint32_t u = lo4 | (((qh >> (2 * (2 * (q & 1) + cc))) & 0x03030303u) << 4);
                    const int scv = (int)(int8_t)(uint8_t)(q6s >> (8 * (2 * cc + hk)));
                    ml_q6_scaled_split(u, scv, w2[cc], w1[cc]);
                }
                mul = 256;
            }
            const long b1 = (long)(((uint64_t)w1[1] << 32) | w1[0]);
            const long b2 = (long)(((uint64_t)w2[1] << 32) | w2[0]);
            const long b3 = (long)(((uint64_t)w3[1] << 32) | w3[0]);
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const long a = *(const long*)(S + L::A + (16 * t + jj) * kMlAS + 32 * k + 8 * q);
                const v4i_ml z = {};
                const v4i_ml i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, z, 0, 0, 0);
                const v4i_ml i2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b2, z, 0, 0, 0);
                v4i_ml i3 = z;
                if constexpr (FMT == kQ5_K) i3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b3, z, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    int32_t isum = i1[r] * mul + i2[r];
                    if constexpr (FMT == kQ5_K) isum += 16 * i3[r];
                    acc[k][4 * t + r] = __builtin_fmaf(dd[4 * t + r], (float)isum, acc[k][4 * t + r]);
                }
            }
            // one lane's products at a time: the chains are advanced here
            // (not sunk to the end of the block), which bounds the live
            // MFMA results
#pragma unroll
            for (int r = 0; r < 4 * RT; r++) asm volatile("" : "+v"(acc[k][r]));
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (FMT == kQ5_K) {
            // m . s over the whole block in one f16 MFMA (lane group q
            // supplies mins 2q, 2q + 1 against 16-value sums 4q .. 4q + 3),
            // then summs = summs + dmin * (m . s) per row, held in accm[0]
            const uint32_t mwd = q < 2 ? sc.mn_lo : sc.mn_hi;
            const _Float16 mA = (_Float16)(float)byte_of(mwd, 2 * (q & 1));
            const _Float16 mB = (_Float16)(float)byte_of(mwd, 2 * (q & 1) + 1);
            const v4h_ml bm = {mA, mA, mB, mB};
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const v4h_ml am = *(const v4h_ml*)(S + L::H + (16 * t + jj) * 32 + 8 * q);
                const v4f_ml z = {};
                const v4f_ml ms = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, z, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) accm[0][4 * t + r] = accm[0][4 * t + r] + dm[4 * t + r] * ms[r];
            }
#pragma unroll
            for (int r = 0; r < 4 * RT; r++) asm volatile("" : "+v"(accm[0][r]));
            __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (F::kMins) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t mwd = k < 2 ? sc.mn_lo : sc.mn_hi;
                const _Float16 mA = (_Float16)(float)byte_of(mwd, 2 * (k & 1));
                const _Float16 mB = (_Float16)(float)byte_of(mwd, 2 * (k & 1) + 1);
                // B[kappa][col], kappa = 4 q + e: nonzero for q == k
                const _Float16 zh = (_Float16)0.f;
                const v4h_ml bm = q == k ? v4h_ml{mA, mA, mB, mB} : v4h_ml{zh, zh, zh, zh};
#pragma unroll
                for (int t = 0; t < RT; t++) {
                    const v4h_ml am = *(const v4h_ml*)(S + L::H + (16 * t + jj) * 32 + 8 * q);
                    const v4f_ml z = {};
                    const v4f_ml ms = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) accm[k][4 * t + r] = __builtin_fmaf(dm[4 * t + r], ms[r], accm[k][4 * t + r]);
                }
#pragma unroll
                for (int r = 0; r < 4 * RT; r++) asm volatile("" : "+v"(accm[k][r]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (b + 1 < nb) park(st[(b + 1) & 1]);
        lds_barrier();
    }
    // hsum_f32_8 and hsum_f32_4 over the lane chains
#pragma unroll
    for (int r = 0; r < 4 * RT; r++) {
        v[r] = ((acc[0][r] + acc[4][r]) + (acc[2][r] + acc[6][r])) + ((acc[1][r] + acc[5][r]) + (acc[3][r] + acc[7][r]));
        if constexpr (FMT == kQ5_K) v[r] = v[r] + accm[0][r];  // the mins scalar
        else if constexpr (F::kMins) v[r] = v[r] + ((accm[0][r] + accm[2][r]) + (accm[1][r] + accm[3][r]));
    }
}

// ---- up to 8 activation rows: two reference lanes per MFMA ------------------
//
// With at most 8 rows a 16-row tile would be half padding.  Instead one
// v_mfma_i32_16x16x64_i8 computes two reference lanes: K 16q..16q+15 of lane
// group q holds the dwords (c, kq), c = 4 (q & 1) .. +3, of reference lane
// kq = p + 4 (q >= 2) (pair p = 0..3).  A row i < 8 carries activation row i
// in the groups q < 2 and zeros in q >= 2; row 8 + i carries activation row i
// in q >= 2 and zeros in q < 2.  So output rows 0..7 are isum_p and rows
// 8..15 isum_{p+4} of the same activation rows: lane (q, j) holds
// activation rows 4 (q & 1) + r of column j for reference lane kq, and the
// lane 32 apart holds the partner lane (kq +- 4) of the same outputs, which
// is the pairing of the first level of hsum_f32_8.

// One block of a pair-lane tile for lane (q, j), all operands in LDS:
//   bcol  this lane's weight row (column j of the tile), staged as in
//         ml_product (Q6_K: the dword window at shift sh);
//   arow  this lane's A row: activation row j (q < 2) or j - 8 (q >= 2) of
//         the block's 256 int8 values, or 256 zero bytes where the lane
//         carries padding;
//   D     the block scales of activation rows 0..7; H their 16-value sums
//         (Q4_K), row r at H + 32 r.
// Returns the lane's isum[p][r] (reference lane p + 4 (q >= 2), activation
// row 4 (q & 1) + r), dd[r] = y.d * x.d, and for Q4_K the mins ms[k][r]
// (mins lane k) with dm[r] = -y.d * x.dmin.
template <int FMT>
struct MlPkBlock {
    int32_t isum[4][4];
    float dd[4];
    float ms[4][4];
    float dm[4];
};
template <int FMT, class SHT>
__device__ __forceinline__ void ml_pk_block(const uint8_t* bcol, SHT sh, const uint8_t* arow, const float* D,
                                            const uint8_t* H, int q, int jj, MlPkBlock<FMT>& o) {
    const int h = q & 1, upper = q >> 1;
    float xd, xdm = 0.f;
    Q4Scales sc{};
    uint32_t s6w = 0;         // Q4_K: six-bit scales of sub-blocks 4h .. 4h+3
    s16x2_ml q6m[4], q6c[4];  // Q6_K: (sc, sc), (128 - 32 sc, ...) of chunks 4h + cc
    // Q4_K: the lane's qs dwords 4 upper + p (p = 0..3) of the 32-byte rows
    // 2h and 2h + 1, as two 16-byte LDS reads per block (conflict-free over
    // the 144-byte column stride; four-byte reads put four lanes per bank)
    u32x4a16 qp[2] = {};
    // Q6_K: the lane's ql (rows 64 h, 64 h + 32) and qh windows, p = 0..3
    uint32_t las[4] = {}, lbs[4] = {}, qhs[4] = {};
    if constexpr (FMT == kQ4_K) {
        const u32x4a16 hdr = *(const u32x4a16*)bcol;
        xd = f16_to_f32(hdr.x);
        xdm = f16_to_f32(hdr.x >> 16);
        sc = q4_scales(hdr.y, hdr.z, hdr.w);
        s6w = h ? sc.sc_hi : sc.sc_lo;
        qp[0] = *(const u32x4a16*)(bcol + 16 + 64 * h + 16 * upper);
        qp[1] = *(const u32x4a16*)(bcol + 16 + 64 * h + 32 + 16 * upper);
    } else {
        xd = f16_to_f32(ml_lds_win(bcol, sh, 208) & 0xffffu);
        ml_lds_span<4>(bcol, sh, 64 * h + 16 * upper, las);
        ml_lds_span<4>(bcol, sh, 64 * h + 32 + 16 * upper, lbs);
        ml_lds_span<4>(bcol, sh, 128 + 32 * h + 16 * upper, qhs);
        // scales 2c + upper of chunks c = 4h + cc: bytes upper, 2 + upper of two dwords
        const uint32_t w0 = ml_lds_win(bcol, sh, 192 + 8 * h) >> (8 * upper);
        const uint32_t w1 = ml_lds_win(bcol, sh, 196 + 8 * h) >> (8 * upper);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const int scv = (int)(int8_t)(uint8_t)((cc < 2 ? w0 : w1) >> (16 * (cc & 1)));
            q6m[cc] = s16x2_ml{(short)scv, (short)scv};
            q6c[cc] = s16x2_ml{(short)(128 - 32 * scv), (short)(128 - 32 * scv)};
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float yd = D[4 * h + r];
        o.dd[r] = yd * xd;
        if constexpr (FMT == kQ4_K) o.dm[r] = -yd * xdm;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int kq = p + 4 * upper;
        uint32_t w1[4], w2[4];
        int mul;  // isum = mul * (stream 1) + (stream 2)
        if constexpr (FMT == kQ4_K) {
            // sub-blocks 4h + cc: qs dword at 16 + 32 (2h + cc / 2) + 4 kq, nibble cc % 2
            const uint32_t qd0 = qp[0][p], qd1 = qp[1][p];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const uint32_t qd = cc < 2 ? qd0 : qd1;
                const uint32_t nib = (cc & 1) ? ((qd >> 4) & 0x0f0f0f0fu) : (qd & 0x0f0f0f0fu);
                const uint32_t s6 = byte_of(s6w, cc);
                w1[cc] = bytes_mul_small(nib, s6 >> 3);
                w2[cc] = bytes_mul_small(nib, s6 & 7u);
            }
            mul = 8;
        } else {
            // chunk c = 4h + cc: ql dword at 64 h + 32 (cc % 2) + 4 kq, the high
            // nibbles for cc >= 2; qh dword at 128 + 32 h + 4 kq, bits 2 cc
            const uint32_t la = las[p], lb = lbs[p], qh = qhs[p];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const uint32_t l = (cc & 1) ? lb : la;
                const uint32_t lo4 = (cc & 2) ? ((l >> 4) & 0x0f0f0f0fu) : (l & 0x0f0f0f0fu);
                const uint32_t u = lo4 | (((qh >> (2 * cc)) & 0x03030303u) << 4);
                const s16x2_ml u02 = __builtin_bit_cast(s16x2_ml, u & 0x00ff00ffu);
                const s16x2_ml u13 = __builtin_bit_cast(s16x2_ml, __builtin_amdgcn_perm(0u, u, 0x0c030c01u));
                const uint32_t p02 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u02 * q6m[cc] + q6c[cc]));
                const uint32_t p13 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u13 * q6m[cc] + q6c[cc]));
                w1[cc] = __builtin_amdgcn_perm(p13, p02, 0x07030501u);
                w2[cc] = __builtin_amdgcn_perm(p13, p02, 0x06020400u) ^ 0x80808080u;
            }
            mul = 256;
        }
        const v4i_ml a = *(const v4i_ml*)(arow + 32 * kq);
        const v4i_ml b1 = {(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
        const v4i_ml b2 = {(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
        const v4i_ml z = {};
        const v4i_ml i1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b1, z, 0, 0, 0);
        const v4i_ml i2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b2, z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) o.isum[p][r] = i1[r] * mul + i2[r];
    }
    if constexpr (FMT == kQ4_K) {
        // mins as in ml_product; rows 8..15 of the f16 MFMA repeat rows 0..7
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t mwd = k < 2 ? sc.mn_lo : sc.mn_hi;
            const _Float16 mA = (_Float16)(float)byte_of(mwd, 2 * (k & 1));
            const _Float16 mB = (_Float16)(float)byte_of(mwd, 2 * (k & 1) + 1);
            const _Float16 zh = (_Float16)0.f;
            const v4h_ml bm = q == k ? v4h_ml{mA, mA, mB, mB} : v4h_ml{zh, zh, zh, zh};
            const v4h_ml am = *(const v4h_ml*)(H + (jj & 7) * 32 + 8 * q);
            const v4f_ml zf = {};
            const v4f_ml m4 = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, zf, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) o.ms[k][r] = m4[r];
        }
    }
}

// The chains of one block: acc[p][r] of reference lane p + 4 (q >= 2),
// accm[k][r] of mins lane k.
template <int FMT>
__device__ __forceinline__ void ml_pk_chain(const MlPkBlock<FMT>& o, float (&acc)[4][4], float (&accm)[4][4]) {
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[p][r] = __builtin_fmaf(o.dd[r], (float)o.isum[p][r], acc[p][r]);
    if constexpr (FMT == kQ4_K)
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int r = 0; r < 4; r++) accm[k][r] = __builtin_fmaf(o.dm[r], o.ms[k][r], accm[k][r]);
}

// hsum_f32_8 (and the mins' hsum_f32_4) of a pair-lane tile: the lane 32
// apart holds reference lanes kq +- 4 of the same outputs.
template <int FMT>
__device__ __forceinline__ void ml_pk_finish(const float (&acc)[4][4], const float (&accm)[4][4], float (&v)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float s[4];
#pragma unroll
        for (int p = 0; p < 4; p++) s[p] = acc[p][r] + __shfl_xor(acc[p][r], 32);
        v[r] = (s[0] + s[2]) + (s[1] + s[3]);
        if constexpr (FMT == kQ4_K) v[r] = v[r] + ((accm[0][r] + accm[2][r]) + (accm[1][r] + accm[3][r]));
    }
}

// LDS stage: A int8 [8][kMlAS], B [64][BS], D f32 [8], H f16 [8][16].
template <int FMT>
struct MlStagePk {
    static constexpr int A = 0;
    static constexpr int B = A + 8 * kMlAS;
    static constexpr int D = B + kMlCols * MlFmt<FMT>::BS;
    static constexpr int H = D + 32;
    static constexpr int END = H + (MlFmt<FMT>::kMins ? 8 * 32 : 0);
};

// As ml_product, for arow(rr) with rr < 8 (at most 8 activation rows); lane
// (q, j) of wave w ends with v[r] = output (activation row 4 (q & 1) + r,
// weight row 16 w + j), r < 4, in every lane group q.  `zero` is 256 bytes
// of LDS holding zeros (16-byte aligned), read by the padding lanes of A.
template <int FMT, class ARow, class BRow>
__device__ __forceinline__ void ml_product_pk(const MlOperands& op, ARow arow, BRow brow,
                                              uint8_t (*st)[MlStagePk<FMT>::END], const uint8_t* zero,
                                              float (&v)[4]) {
    using F = MlFmt<FMT>;
    using L = MlStagePk<FMT>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int h = q & 1;
    const int upper = q >> 1;
    const int nb = op.nb;

    // ---- staging, as in ml_product: A 8 rows x 16 chunks, B 64 rows x NL
    constexpr int kA = 8 * 16;
    constexpr int kB = kMlCols * F::NL;
    constexpr int kBPer = (kB + 255) / 256;
    const int ta = threadIdx.x;  // A chunk of threads 0..127
    const uint32_t a_src = (uint32_t)(arow((ta >> 4) & 7) * op.ldq + 16 * (ta & 15));
    const int a_off = ta < kA ? L::A + (ta >> 4) * kMlAS + 16 * (ta & 15) : -1;
    uint32_t b_src[kBPer];
    int b_off[kBPer];
    bool b_hi[kBPer];
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kB - 1);
        const int c2 = t / F::NL, part = t - c2 * F::NL;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        b_hi[i] = c2 >= op.bsplit;
        b_src[i] = (uint32_t)(brow(c2) * op.brow_bytes + po);
        b_off[i] = (int)threadIdx.x + 256 * i < kB ? L::B + c2 * F::BS + po : -1;
    }
    // D on threads 128..135, H (Q4_K) on 192..207
    const int tD = threadIdx.x - 128, tH = threadIdx.x - 192;
    const int64_t d_row = arow(tD & 7);
    const int64_t h_row = arow((tH >> 1) & 7);

    v4i_ml sa = {};
    u32x4 sb[kBPer];
    float sd = 0.f;
    v4i_ml sh16 = {};
    auto issue = [&](int b) {
        if (ta < kA) sa = *(const v4i_ml*)(op.aq + (int64_t)b * 256 + a_src);
        const int64_t boff = FMT == kQ6_K ? ((int64_t)b * F::BB) & ~(int64_t)3 : (int64_t)b * F::BB;
#pragma unroll
        for (int i = 0; i < kBPer; i++) sb[i] = *(const u32x4*)((b_hi[i] ? op.b1 : op.b0) + boff + b_src[i]);
        if (tD >= 0 && tD < 8) sd = op.ad[d_row * op.ldd + b];
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 16) sh16 = *(const v4i_ml*)(op.hs + (h_row * nb + b) * 16 + 8 * (tH & 1));
    };
    auto park = [&](uint8_t* s) {
        if (a_off >= 0) *(v4i_ml*)(s + a_off) = sa;
#pragma unroll
        for (int i = 0; i < kBPer; i++)
            if (b_off[i] >= 0) *(u32x4*)(s + b_off[i]) = sb[i];
        if (tD >= 0 && tD < 8) *(float*)(s + L::D + 4 * tD) = sd;
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 16) *(v4i_ml*)(s + L::H + 32 * (tH >> 1) + 16 * (tH & 1)) = sh16;
    };

    const int col = 16 * wave + jj;
    // A row of this lane: activation row j (q < 2) or j - 8 (q >= 2) where
    // that lane carries data, else the zero row
    const bool a_live = (jj < 8) == (upper == 0);
    float acc[4][4], accm[4][4];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[p][r] = accm[p][r] = 0.f;
    issue(0);
    park(st[0]);
    lds_barrier();
    for (int b = 0; b < nb; b++) {
        const uint8_t* S = st[b & 1];
        if (b + 1 < nb) issue(b + 1);
        const uint8_t* arowp = a_live ? S + L::A + (jj & 7) * kMlAS + 16 * h : zero + 16 * h;
        MlPkBlock<FMT> o;
        // Q6_K: block b of a row sits at shift 2 (b & 1) (rows of a multiple of 4 bytes)
        if (FMT == kQ6_K && (b & 1))
            ml_pk_block<FMT>(S + L::B + col * F::BS, MlShift<2>{}, arowp, (const float*)(S + L::D), S + L::H, q, jj, o);
        else
            ml_pk_block<FMT>(S + L::B + col * F::BS, MlShift<0>{}, arowp, (const float*)(S + L::D), S + L::H, q, jj, o);
        ml_pk_chain<FMT>(o, acc, accm);
        __builtin_amdgcn_sched_barrier(0);
        if (b + 1 < nb) park(st[(b + 1) & 1]);
        lds_barrier();
    }
    ml_pk_finish<FMT>(acc, accm, v);
}

// ---- split K: 16 weight rows, the blocks spread over the waves ----------
//
// For matrices whose 64-row tiles leave too few workgroups: a workgroup of
// NW waves takes 16 weight rows (columns j of the pair-lane tile) and up to
// 8 activation rows, and wave w two of the 2 NW blocks, all loaded at once;
// the waves form their blocks' exact integers in parallel (ml_pk_block),
// then the f32 chains pass from wave to wave in block order through LDS, so
// every output is the one-row kernel's bit for bit.

template <int FMT>
struct MlSkRegion {  // one block of one wave in LDS
    static constexpr int A = 0;                        // int8 [8][kMlAS]
    static constexpr int B = A + 8 * kMlAS;            // [16][BS]
    static constexpr int D = B + 16 * MlFmt<FMT>::BS;  // f32 [8]
    static constexpr int H = D + 32;                   // f16 [8][16] (Q4_K)
    static constexpr int END = H + (MlFmt<FMT>::kMins ? 8 * 32 : 0);
};
constexpr int kSkBPW = 2;  // blocks per wave

// op.nb must be 2 NW; brow(c) for c < 16 (columns at or past op.bsplit come
// from op.b1); arow(rr) for rr < 8.  `reg` is the caller's LDS
// [NW][kSkBPW][END], `zero` 256 bytes of LDS (zeroed here).  The result is
// in wave NW - 1: v[r] = output (activation row 4 (q & 1) + r, column j).
template <int FMT, int NW, class ARow, class BRow>
__device__ __forceinline__ void ml_product_sk(const MlOperands& op, ARow arow, BRow brow,
                                              uint8_t (*reg)[kSkBPW][MlSkRegion<FMT>::END], uint8_t* zero,
                                              float (&v)[4]) {
    using F = MlFmt<FMT>;
    using R = MlSkRegion<FMT>;
    constexpr int BPW = kSkBPW, NH = FMT == kQ4_K ? 32 : 16;  // handed-over floats per lane
    // the chains' hand-over [NH][64] reuses wave 0's stage: wave 0 writes it
    // after its own blocks, and the other waves' stages stay untouched
    static_assert(NH * 64 * 4 <= BPW * R::END, "hand-over fits wave 0's stage");
    // [NH / 4][64] float4: one 16-byte LDS access per four chains, lanes
    // 16 bytes apart (no bank conflicts)
    f32x4 (*hand)[64] = (f32x4 (*)[64])reg[0][0];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15, h = q & 1;
    ((uint32_t*)zero)[lane] = 0u;
    const int b0 = wave * BPW;

    // staging of this wave's blocks b0, b0 + 1: A 8 rows x 16 chunks, B 16
    // rows x NL chunks, D 8 scales, H 8 x 2 chunks (Q4_K), per block
    constexpr int kA = 8 * 16 * BPW, kB = 16 * F::NL * BPW;
    constexpr int kAPer = kA / 64, kBPer = (kB + 63) / 64;
    v4i_ml sa[kAPer];
    u32x4 sb[kBPer];
#pragma unroll
    for (int i = 0; i < kAPer; i++) {
        const int t = lane + 64 * i, bi = t >> 7, row = (t >> 4) & 7, part = t & 15;
        sa[i] = *(const v4i_ml*)(op.aq + arow(row) * op.ldq + (int64_t)(b0 + bi) * 256 + 16 * part);
    }
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min(lane + 64 * i, kB - 1);
        const int cb = t / F::NL, part = t - cb * F::NL, col = cb / BPW, bi = cb - col * BPW;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        const int64_t b = b0 + bi;
        const int64_t boff = FMT == kQ6_K ? (b * F::BB) & ~(int64_t)3 : b * F::BB;
        sb[i] = *(const u32x4*)((col >= op.bsplit ? op.b1 : op.b0) + brow(col) * op.brow_bytes + boff + po);
    }
    float sd = 0.f;
    if (lane < 8 * BPW) sd = op.ad[arow(lane & 7) * op.ldd + b0 + (lane >> 3)];
    v4i_ml sh16 = {};
    if constexpr (F::kMins)
        if (lane < 16 * BPW)
            sh16 = *(const v4i_ml*)(op.hs + (arow((lane >> 1) & 7) * op.nb + b0 + (lane >> 4)) * 16 + 8 * (lane & 1));
#pragma unroll
    for (int i = 0; i < kAPer; i++) {
        const int t = lane + 64 * i, bi = t >> 7, row = (t >> 4) & 7, part = t & 15;
        *(v4i_ml*)(reg[wave][bi] + R::A + row * kMlAS + 16 * part) = sa[i];
    }
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = lane + 64 * i;
        if (t < kB) {
            const int cb = t / F::NL, part = t - cb * F::NL, col = cb / BPW, bi = cb - col * BPW;
            const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
            *(u32x4*)(reg[wave][bi] + R::B + col * F::BS + po) = sb[i];
        }
    }
    if (lane < 8 * BPW) *(float*)(reg[wave][lane >> 3] + R::D + 4 * (lane & 7)) = sd;
    if constexpr (F::kMins)
        if (lane < 16 * BPW) *(v4i_ml*)(reg[wave][lane >> 4] + R::H + 32 * ((lane >> 1) & 7) + 16 * (lane & 1)) = sh16;
    lds_barrier();  // the zero row and every wave's stage

    // this wave's blocks: exact integers and scales
    const bool a_live = (jj < 8) == (q < 2);
    MlPkBlock<FMT> o[BPW];
#pragma unroll
    for (int bi = 0; bi < BPW; bi++) {
        const uint8_t* S = reg[wave][bi];
        const int sh = FMT == kQ6_K ? (int)(((int64_t)(b0 + bi) * F::BB) & 3) : 0;
        const uint8_t* arowp = a_live ? S + R::A + (jj & 7) * kMlAS + 16 * h : zero + 16 * h;
        ml_pk_block<FMT>(S + R::B + jj * F::BS, sh, arowp, (const float*)(S + R::D), S + R::H, q, jj, o[bi]);
    }
    // the chains, wave 0 first: each wave continues them over its blocks
    float acc[4][4], accm[4][4];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[p][r] = accm[p][r] = 0.f;
    for (int w2 = 0; w2 < NW; w2++) {
        if (wave == w2) {
            if (w2 > 0) {
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const f32x4 t = hand[p][lane];
                    acc[p][0] = t.x; acc[p][1] = t.y; acc[p][2] = t.z; acc[p][3] = t.w;
                }
                if constexpr (F::kMins)
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        const f32x4 t = hand[4 + p][lane];
                        accm[p][0] = t.x; accm[p][1] = t.y; accm[p][2] = t.z; accm[p][3] = t.w;
                    }
            }
#pragma unroll
            for (int bi = 0; bi < BPW; bi++) ml_pk_chain<FMT>(o[bi], acc, accm);
            if (w2 < NW - 1) {
#pragma unroll
                for (int p = 0; p < 4; p++) hand[p][lane] = f32x4{acc[p][0], acc[p][1], acc[p][2], acc[p][3]};
                if constexpr (F::kMins)
#pragma unroll
                    for (int p = 0; p < 4; p++) hand[4 + p][lane] = f32x4{accm[p][0], accm[p][1], accm[p][2], accm[p][3]};
            }
        }
        if (w2 < NW - 1) lds_barrier();
    }
    if (wave == NW - 1) ml_pk_finish<FMT>(acc, accm, v);
}

// ---- tile order: one f32 step per output and block ------------------------
//
// For products whose outputs are not quantised again (the grouped MoE down
// products, on request): the block's whole integer isum (the sum of the
// eight reference lanes' integers) on v_mfma_i32_16x16x64_i8, then one
// step out += y.d (x.d isum - x.dmin msum) per output and block.  The
// per-block integers are exact; the f32 order is one chain per output
// instead of eight lane chains joined by hsum_f32_8, a few ulps apart.
//
// K chunk of step p (0..3) for lane group q (h = q & 1, upper = q >> 1):
// the activation dwords (c, k), k = p + 4 upper, c = 4 h .. 4 h + 3, which
// the activation layout keeps as the 16 bytes at 32 k + 16 h; B carries the
// same four weight dwords with their scales folded in, decoded as in the
// pair-lane tile (ml_pk_block).  Over the four steps and lane groups the
// chunks cover the block once, and one decoded B fragment serves every
// 16-row tile.

// One block: o[t][r] += output (row 16 t + 4 q + r, column j) for the RT
// tiles.  Operands in LDS: A the block's activation rows at stride kMlAS,
// bcol this lane's weight row staged as in ml_product (Q6_K: the dword
// window at shift sh), D the rows' block scales, H their 16-value sums
// (Q4_K, 32 bytes a row).
template <int FMT, int RT, class SHT>
__device__ __forceinline__ void ml_tile_block(const uint8_t* A, const uint8_t* bcol, const float* D,
                                              const uint8_t* H, SHT sh, int q, int jj, float (&o)[RT][4]) {
    const int h = q & 1, upper = q >> 1;
    float xd, xdm = 0.f;
    Q4Scales sc{};
    uint32_t s6w = 0;
    s16x2_ml q6m[4], q6c[4];
    u32x4a16 qp[2] = {};
    uint32_t las[4] = {}, lbs[4] = {}, qhs[4] = {};
    if constexpr (FMT == kQ4_K) {
        const u32x4a16 hdr = *(const u32x4a16*)bcol;
        xd = f16_to_f32(hdr.x);
        xdm = f16_to_f32(hdr.x >> 16);
        sc = q4_scales(hdr.y, hdr.z, hdr.w);
        s6w = h ? sc.sc_hi : sc.sc_lo;
        qp[0] = *(const u32x4a16*)(bcol + 16 + 64 * h + 16 * upper);
        qp[1] = *(const u32x4a16*)(bcol + 16 + 64 * h + 32 + 16 * upper);
    } else {
        xd = f16_to_f32(ml_lds_win(bcol, sh, 208) & 0xffffu);
        ml_lds_span<4>(bcol, sh, 64 * h + 16 * upper, las);
        ml_lds_span<4>(bcol, sh, 64 * h + 32 + 16 * upper, lbs);
        ml_lds_span<4>(bcol, sh, 128 + 32 * h + 16 * upper, qhs);
        const uint32_t w0 = ml_lds_win(bcol, sh, 192 + 8 * h) >> (8 * upper);
        const uint32_t w1 = ml_lds_win(bcol, sh, 196 + 8 * h) >> (8 * upper);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const int scv = (int)(int8_t)(uint8_t)((cc < 2 ? w0 : w1) >> (16 * (cc & 1)));
            q6m[cc] = s16x2_ml{(short)scv, (short)scv};
            q6c[cc] = s16x2_ml{(short)(128 - 32 * scv), (short)(128 - 32 * scv)};
        }
    }
    v4i_ml i1[RT], i2[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) i1[t] = i2[t] = v4i_ml{0, 0, 0, 0};
    constexpr int mul = FMT == kQ4_K ? 8 : 256;  // isum = mul * (stream 1) + (stream 2)
#pragma unroll
    for (int p = 0; p < 4; p++) {
        uint32_t w1[4], w2[4];
        if constexpr (FMT == kQ4_K) {
            const uint32_t qd0 = qp[0][p], qd1 = qp[1][p];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const uint32_t qd = cc < 2 ? qd0 : qd1;
                const uint32_t nib = (cc & 1) ? ((qd >> 4) & 0x0f0f0f0fu) : (qd & 0x0f0f0f0fu);
                const uint32_t s6 = byte_of(s6w, cc);
                w1[cc] = bytes_mul_small(nib, s6 >> 3);
                w2[cc] = bytes_mul_small(nib, s6 & 7u);
            }
        } else {
            const uint32_t la = las[p], lb = lbs[p], qh = qhs[p];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const uint32_t l = (cc & 1) ? lb : la;
                const uint32_t lo4 = (cc & 2) ? ((l >> 4) & 0x0f0f0f0fu) : (l & 0x0f0f0f0fu);
                const uint32_t u = lo4 | (((qh >> (2 * cc)) & 0x03030303u) << 4);
                const s16x2_ml u02 = __builtin_bit_cast(s16x2_ml, u & 0x00ff00ffu);
                const s16x2_ml u13 = __builtin_bit_cast(s16x2_ml, __builtin_amdgcn_perm(0u, u, 0x0c030c01u));
                const uint32_t p02 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u02 * q6m[cc] + q6c[cc]));
                const uint32_t p13 = __builtin_bit_cast(uint32_t, (s16x2_ml)(u13 * q6m[cc] + q6c[cc]));
                w1[cc] = __builtin_amdgcn_perm(p13, p02, 0x07030501u);
                w2[cc] = __builtin_amdgcn_perm(p13, p02, 0x06020400u) ^ 0x80808080u;
            }
        }
        const v4i_ml b1 = {(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
        const v4i_ml b2 = {(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const v4i_ml a = *(const v4i_ml*)(A + (16 * t + jj) * kMlAS + 32 * (p + 4 * upper) + 16 * h);
            i1[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b1, i1[t], 0, 0, 0);
            i2[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b2, i2[t], 0, 0, 0);
        }
    }
    // Q4_K mins: msum = sum over the 16-value sums s of m_{s/2} bsum16_s
    // (lane group q: sums 4 q .. 4 q + 3, mins m_2q, m_2q+1), integers
    // below 2^24 in the f16 MFMA's f32 result
    v4h_ml bm = {};
    if constexpr (FMT == kQ4_K) {
        const uint32_t mw = q < 2 ? sc.mn_lo : sc.mn_hi;
        const _Float16 mA = (_Float16)(float)byte_of(mw, 2 * (q & 1));
        const _Float16 mB = (_Float16)(float)byte_of(mw, 2 * (q & 1) + 1);
        bm = v4h_ml{mA, mA, mB, mB};
    }
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const f32x4 yd = *(const f32x4*)(D + 16 * t + 4 * q);
        v4f_ml ms = {};
        if constexpr (FMT == kQ4_K) {
            const v4h_ml am = *(const v4h_ml*)(H + (16 * t + jj) * 32 + 8 * q);
            ms = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, v4f_ml{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
        const float ydr[4] = {yd.x, yd.y, yd.z, yd.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float isum = (float)(i1[t][r] * mul + i2[t][r]);
            if constexpr (FMT == kQ4_K)
                o[t][r] = __builtin_fmaf(ydr[r], __builtin_fmaf(-xdm, ms[r], xd * isum), o[t][r]);
            else
                o[t][r] = __builtin_fmaf(ydr[r] * xd, isum, o[t][r]);
        }
    }
}

// NT 16-row tiles x 64 weight rows on a 256-thread workgroup, in a stage of
// RT >= NT tiles staged as in ml_product (rows past 16 NT are not loaded);
// lane (q, j) of wave w ends with v[4 t + r] = output (row 16 t + 4 q + r,
// weight row 16 w + j), t < NT.
template <int FMT, int RT, int NT, class ARow, class BRow>
__device__ __forceinline__ void ml_product_tiles(const MlOperands& op, ARow arow, BRow brow,
                                                 uint8_t (*st)[MlStage<FMT, RT>::END], float (&v)[4 * RT]) {
    using F = MlFmt<FMT>;
    using L = MlStage<FMT, RT>;
    static_assert(NT <= RT, "live tiles");
    constexpr int rt_used = NT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int nb = op.nb;
    static_assert(RT <= 4, "D and H staging threads");

    constexpr int kAPer = RT;  // 16 RT rows x 16 chunks = 256 RT
    constexpr int kB = kMlCols * F::NL;
    constexpr int kBPer = (kB + 255) / 256;
    uint32_t a_src[kAPer];
    int a_off[kAPer];
#pragma unroll
    for (int i = 0; i < kAPer; i++) {
        const int t = (int)threadIdx.x + 256 * i;
        const int rr = t >> 4, part = t & 15;
        a_src[i] = (uint32_t)(arow(rr) * op.ldq + 16 * part);
        a_off[i] = rr < 16 * rt_used ? L::A + rr * kMlAS + 16 * part : -1;
    }
    uint32_t b_src[kBPer];
    int b_off[kBPer];
    bool b_hi[kBPer];
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kB - 1);
        const int c2 = t / F::NL, part = t - c2 * F::NL;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        b_hi[i] = c2 >= op.bsplit;
        b_src[i] = (uint32_t)(brow(c2) * op.brow_bytes + po);
        b_off[i] = (int)threadIdx.x + 256 * i < kB ? L::B + c2 * F::BS + po : -1;
    }
    const int tD = threadIdx.x, tH = threadIdx.x - 64;
    const int64_t d_row = arow(tD & (L::R - 1));
    const int64_t h_row = arow((tH >> 1) & (L::R - 1));

    v4i_ml sa[kAPer];
    u32x4 sb[kBPer];
    float sd = 0.f;
    v4i_ml sh16 = {};
    auto issue = [&](int b) {
        const int8_t* abase = op.aq + (int64_t)b * 256;
#pragma unroll
        for (int i = 0; i < kAPer; i++)
            if (a_off[i] >= 0) sa[i] = *(const v4i_ml*)(abase + a_src[i]);
        const int64_t boff = FMT == kQ6_K ? ((int64_t)b * F::BB) & ~(int64_t)3 : (int64_t)b * F::BB;
#pragma unroll
        for (int i = 0; i < kBPer; i++) sb[i] = *(const u32x4*)((b_hi[i] ? op.b1 : op.b0) + boff + b_src[i]);
        if (tD < L::R) sd = op.ad[d_row * op.ldd + b];
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 2 * L::R) sh16 = *(const v4i_ml*)(op.hs + (h_row * nb + b) * 16 + 8 * (tH & 1));
    };
    auto park = [&](uint8_t* s) {
#pragma unroll
        for (int i = 0; i < kAPer; i++)
            if (a_off[i] >= 0) *(v4i_ml*)(s + a_off[i]) = sa[i];
#pragma unroll
        for (int i = 0; i < kBPer; i++)
            if (b_off[i] >= 0) *(u32x4*)(s + b_off[i]) = sb[i];
        if (tD < L::R) *(float*)(s + L::D + 4 * tD) = sd;
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 2 * L::R) *(v4i_ml*)(s + L::H + 32 * (tH >> 1) + 16 * (tH & 1)) = sh16;
    };

    const int col = 16 * wave + jj;
    float o[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) o[t][r] = 0.f;
    issue(0);
    park(st[0]);
    lds_barrier();
    for (int b = 0; b < nb; b++) {
        const uint8_t* S = st[b & 1];
        if (b + 1 < nb) issue(b + 1);
        if (FMT == kQ6_K && (b & 1))  // block b of a row sits at shift 2 (b & 1)
            ml_tile_block<FMT, NT>(S + L::A, S + L::B + col * F::BS, (const float*)(S + L::D), S + L::H, MlShift<2>{},
                                   q, jj, o);
        else
            ml_tile_block<FMT, NT>(S + L::A, S + L::B + col * F::BS, (const float*)(S + L::D), S + L::H, MlShift<0>{},
                                   q, jj, o);
        __builtin_amdgcn_sched_barrier(0);
        if (b + 1 < nb) park(st[(b + 1) & 1]);
        lds_barrier();
    }
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) v[4 * t + r] = t < NT ? o[t][r] : 0.f;
}

}  // namespace iq
