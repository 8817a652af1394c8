/*
 * qgemm_lanes.c -- TEST INFRASTRUCTURE (parity oracle, see iq_oracle.h).
 *
 * Scalar emulation of the reference's fused kernels (src/qgemm.rs:175-397):
 * eight f32 lane accumulators per input row (plus four for the Q4_K mins),
 * each advanced once per block by a fused multiply-add of the block scale and
 * that lane's exact integer, then reduced by the fixed hsum trees
 * (src/qgemm.rs:132-148).  fmaf() is a correctly rounded FMA, the same
 * operation as vfmadd231ps, so this reproduces the AVX2 result bit for bit.
 */
#include <math.h>

#include "iq_oracle.h"

/* hsum_f32_8: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) */
static float hsum8(const float l[8]) {
    float a = l[0] + l[4], b = l[1] + l[5], c = l[2] + l[6], d = l[3] + l[7];
    return (a + c) + (b + d);
}

/* hsum_f32_4: (l0+l2) + (l1+l3) */
static float hsum4(const float l[4]) { return (l[0] + l[2]) + (l[1] + l[3]); }

void or_q4k_q8k_row_lanes(const or_q4k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out) {
    for (size_t r = 0; r < rows; r++) {
        float acc[8] = {0}, accm[4] = {0};
        for (size_t b = 0; b < nb; b++) {
            const or_q8k_block *y = &in[b * rows + r];
            int32_t isum[8], msum[4];
            or_q4k_block_lanes(&w[b], y, isum, msum);
            float xd = or_f16_to_f32(w[b].d);
            float xdmin = or_f16_to_f32(w[b].dmin);
            float d = y->d * xd;
            float dmin = -y->d * xdmin;
            for (int k = 0; k < 8; k++) acc[k] = fmaf(d, (float)isum[k], acc[k]);
            for (int k = 0; k < 4; k++) accm[k] = fmaf(dmin, (float)msum[k], accm[k]);
        }
        out[r] = hsum8(acc) + hsum4(accm);
    }
}

void or_q5k_q8k_row_lanes(const or_q5k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out) {
    for (size_t r = 0; r < rows; r++) {
        float acc[8] = {0}, summs = 0.f;
        for (size_t b = 0; b < nb; b++) {
            const or_q8k_block *y = &in[b * rows + r];
            int32_t isum[8], msum[4];
            or_q5k_block_lanes(&w[b], y, isum, msum);
            float d = y->d * or_f16_to_f32(w[b].d);
            float dmin = -y->d * or_f16_to_f32(w[b].dmin);
            for (int k = 0; k < 8; k++) acc[k] = fmaf(d, (float)isum[k], acc[k]);
            /* hadd(hadd(prod, 0), 0): (l0 + l1) + (l2 + l3), exact in i32 */
            int32_t m = (msum[0] + msum[1]) + (msum[2] + msum[3]);
            summs = summs + dmin * (float)m;
        }
        out[r] = hsum8(acc) + summs;
    }
}

void or_q6k_q8k_row_lanes(const or_q6k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out) {
    for (size_t r = 0; r < rows; r++) {
        float acc[8] = {0};
        for (size_t b = 0; b < nb; b++) {
            const or_q8k_block *y = &in[b * rows + r];
            int32_t isum[8];
            or_q6k_block_lanes(&w[b], y, isum);
            float d = y->d * or_f16_to_f32(w[b].d);
            for (int k = 0; k < 8; k++) acc[k] = fmaf(d, (float)isum[k], acc[k]);
        }
        out[r] = hsum8(acc);
    }
}

void or_q80_q80_row_lanes(const or_q80_block *w, size_t nb, const or_q80_block *in, size_t rows, float *out) {
    for (size_t r = 0; r < rows; r++) {
        float acc[8] = {0};
        for (size_t b = 0; b < nb; b++) {
            const or_q80_block *y = &in[b * rows + r];
            int32_t isum[8];
            or_q80_block_lanes(&w[b], y, isum);
            float d = or_f16_to_f32(w[b].d) * or_f16_to_f32(y->d);
            for (int k = 0; k < 8; k++) acc[k] = fmaf(d, (float)isum[k], acc[k]);
        }
        out[r] = hsum8(acc);
    }
}
