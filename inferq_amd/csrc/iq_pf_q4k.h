// iq_pf_q4k.h -- one Q4_K block of a wave's prefill tile on int8 MFMA:
// per-block integers exact, f32 combination in tile order (the dense
// prefill, iq_prefill.hip).  Not for products whose outputs are quantised
// again (the MoE gate/up, whose SwiGLU rows become Q8K for down): a last-ulp
// difference there can move a value across a rounding boundary of the
// quantiser, and one changed int8 activation shifts the down output by
// about 1e-4 of its norm.
//
// Per block of 256 weights the reference's integers are isum = sum_j sc_j *
// sum_{e in sub-block j} q_e a_e and msum = sum_j m_j * bsum32_j
// (src/qgemm.rs:175-245; sc_j, m_j six-bit, q_e four-bit, a_e the Q8K int8
// activations).  A six-bit scale times a four-bit quant does not fit int8,
// so the scale is split, sc = 8 sc_hi + sc_lo with both parts in 0..7: the
// MFMA streams w1 = sc_hi q and w2 = sc_lo q (bytes <= 105) give isum =
// 8 acc1 + acc2 exactly.  msum comes from one f16 MFMA over the block's 16
// bsums of 16 values (|bsum16| <= 2048, the mins exact in f16, products and
// sums below 2^24 in the f32 accumulator).  The tile then takes
// out += dx (dw isum - dmin msum): a different f32 order than the
// reference's per-lane chains (results within the 1e-4 normwise bar).
#pragma once

#include "iq_lanes.h"

namespace iq {

typedef int pf_v4i __attribute__((ext_vector_type(4)));
typedef float pf_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 pf_v4h __attribute__((ext_vector_type(4)));

// A wave's RT row tiles (16 rows each) times one 16-column B fragment over
// one block, all operands in LDS:
//   A     int8 activations, row r at A + r * AS, the block's 256 values in
//         natural order;
//   bcol  this lane's column: the raw 144-byte Q4_K block (16-byte aligned);
//   H     the rows' 16 bsum16 values as f16, row r at H + 32 r;
//   D     the rows' block scales dx (f32).
// Lane l (g = l / 16, j = l % 16) holds K 16g..16g+15 of each 64-value step
// for row / column j, and the results of rows 16 rt + 4g + r (r < 4) of
// column j; one K step is sub-blocks 2s and 2s+1, the low and the high
// nibbles of qs bytes 32s..32s+31.  hook(rt, r, isum, msum) sees every
// per-block integer pair (parity hooks; a no-op otherwise).
template <int RT, int AS, class Hook>
__device__ __forceinline__ void pf_q4k_block(const uint8_t* A, const uint8_t* bcol, const uint8_t* H,
                                             const float* D, int g, int jj, float (&out)[RT][4], Hook&& hook) {
    const u32x4a16 hdr = *(const u32x4a16*)bcol;
    const float dw = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
    const Q4Scales sc = q4_scales(hdr.y, hdr.z, hdr.w);
    pf_v4i acc1[RT], acc2[RT];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {  // K step: values 64 s4 .. +63
        const int shn = (g >> 1) * 4;
        // sub-block 2 s4 + (g >> 1): byte (2 s4 + (g >> 1)) & 3 of the low or high scale word
        const uint32_t s6 = byte_of(s4 < 2 ? sc.sc_lo : sc.sc_hi, (2 * s4 + (g >> 1)) & 3);
        const uint32_t hi = s6 >> 3, lo = s6 & 7u;
        const u32x4a16 raw = *(const u32x4a16*)(bcol + 16 + 32 * s4 + 16 * (g & 1));
        const uint32_t qv[4] = {(raw.x >> shn) & 0x0f0f0f0fu, (raw.y >> shn) & 0x0f0f0f0fu,
                                (raw.z >> shn) & 0x0f0f0f0fu, (raw.w >> shn) & 0x0f0f0f0fu};
        const pf_v4i w1 = {(int)bytes_mul_small(qv[0], hi), (int)bytes_mul_small(qv[1], hi),
                           (int)bytes_mul_small(qv[2], hi), (int)bytes_mul_small(qv[3], hi)};
        const pf_v4i w2 = {(int)bytes_mul_small(qv[0], lo), (int)bytes_mul_small(qv[1], lo),
                           (int)bytes_mul_small(qv[2], lo), (int)bytes_mul_small(qv[3], lo)};
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const pf_v4i a = *(const pf_v4i*)(A + (16 * rt + jj) * AS + 64 * s4 + 16 * g);
            const pf_v4i z = {};
            acc1[rt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, w1, s4 == 0 ? z : acc1[rt], 0, 0, 0);
            acc2[rt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, w2, s4 == 0 ? z : acc2[rt], 0, 0, 0);
        }
    }
    // mins: msum = sum_t m_{t/2} bsum16_t (K = 16; lane group g: t = 4g..4g+3)
    const uint32_t mw = g < 2 ? sc.mn_lo : sc.mn_hi;  // m_{2g}, m_{2g+1}: bytes 2 (g & 1) + 0, 1
    const _Float16 mA = (_Float16)(float)byte_of(mw, 2 * (g & 1));
    const _Float16 mB = (_Float16)(float)byte_of(mw, 2 * (g & 1) + 1);
    const pf_v4h bm = {mA, mA, mB, mB};
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const pf_v4h am = *(const pf_v4h*)(H + (16 * rt + jj) * 32 + 8 * g);
        const f32x4 dx = *(const f32x4*)(D + 16 * rt + 4 * g);
        const pf_v4f z = {};
        const pf_v4f msum = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int32_t isum = 8 * acc1[rt][r] + acc2[rt][r];
            const float t = __builtin_fmaf(-dmin, msum[r], dw * (float)isum);
            out[rt][r] = __builtin_fmaf(dx[r], t, out[rt][r]);
            hook(rt, r, isum, msum[r]);
        }
    }
}

}  // namespace iq
