/*
 * qgemm_avx2.c -- TEST INFRASTRUCTURE (parity oracle and timed CPU baseline,
 * see iq_oracle.h).
 *
 * The reference's AVX2+FMA fused kernels (src/qgemm.rs:99-443) restated with
 * the same intrinsic sequence, so that this file reproduces the reference's
 * CPU arithmetic (and its speed class) on any x86-64 host with AVX2 and FMA.
 * A tile of T <= 8 input rows shares one decode of each weight block; a row
 * count that is not a multiple of 8 ends with one narrower tile
 * (tiled_entry!, src/qgemm.rs:399-438).
 */
#include "iq_oracle.h"

#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#include <string.h>

int or_have_avx2(void) { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }

static inline float hsum_f32_8(__m256 x) {
    __m128 res = _mm256_extractf128_ps(x, 1);
    res = _mm_add_ps(res, _mm256_castps256_ps128(x));
    res = _mm_add_ps(res, _mm_movehl_ps(res, res));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}

static inline float hsum_f32_4(__m128 x) {
    __m128 res = _mm_add_ps(x, _mm_movehl_ps(x, x));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}

/* The utmp sequence of ggml's K-quant scale unpack: dwords 0-1 hold the eight
 * scales, dwords 2-3 the eight mins, one byte each. */
static inline void utmp_unpack(const uint8_t s[12], uint32_t u[4]) {
    const uint32_t kmask1 = 0x3f3f3f3f, kmask2 = 0x0f0f0f0f, kmask3 = 0x03030303;
    memcpy(u, s, 12);
    u[3] = ((u[2] >> 4) & kmask2) | (((u[1] >> 6) & kmask3) << 4);
    uint32_t uaux = u[1] & kmask1;
    u[1] = (u[2] & kmask2) | (((u[0] >> 6) & kmask3) << 4);
    u[2] = uaux;
    u[0] &= kmask1;
}

/* Broadcast i16 element `i` of a vector across each 128-bit lane. */
static inline __m256i bcast16(int i) { return _mm256_set1_epi16((short)(((2 * i + 1) << 8) | (2 * i))); }

/* Low 8 bytes select byte 2i, high 8 bytes select byte 2i+1. */
static inline __m128i q6_pair(int i) {
    return _mm_set_epi64x((long long)(0x0101010101010101ull * (uint64_t)(2 * i + 1)),
                          (long long)(0x0101010101010101ull * (uint64_t)(2 * i)));
}

static inline __attribute__((always_inline)) void q4k_tile(const or_q4k_block *w, size_t nb, const or_q8k_block *in,
                                                           size_t rows, size_t base, float *out, const int T) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc[8];
    __m128 accm[8];
    for (int t = 0; t < T; t++) {
        acc[t] = _mm256_setzero_ps();
        accm[t] = _mm_setzero_ps();
    }
    for (size_t b = 0; b < nb; b++) {
        uint32_t u[4];
        utmp_unpack(w[b].scales, u);
        __m256i ms = _mm256_cvtepu8_epi16(_mm_set_epi32((int)u[3], (int)u[2], (int)u[1], (int)u[0]));
        __m128i sc128 = _mm256_extracti128_si256(ms, 0);
        __m128i mins128 = _mm256_extracti128_si256(ms, 1);
        __m256i scales = _mm256_set_m128i(sc128, sc128);
        float xd = or_f16_to_f32(w[b].d), xdmin = or_f16_to_f32(w[b].dmin);
        __m256i sumi[8];
        for (int t = 0; t < T; t++) sumi[t] = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i q4bits = _mm256_loadu_si256((const __m256i *)(w[b].qs + 32 * j));
            __m256i q4l = _mm256_and_si256(q4bits, m4);
            __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            __m256i sl = _mm256_shuffle_epi8(scales, bcast16(2 * j));
            __m256i sh = _mm256_shuffle_epi8(scales, bcast16(2 * j + 1));
            for (int t = 0; t < T; t++) {
                const or_q8k_block *y = &in[b * rows + base + t];
                __m256i q8l = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j));
                __m256i q8h = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j + 32));
                __m256i pl = _mm256_madd_epi16(sl, _mm256_maddubs_epi16(q4l, q8l));
                __m256i ph = _mm256_madd_epi16(sh, _mm256_maddubs_epi16(q4h, q8h));
                sumi[t] = _mm256_add_epi32(sumi[t], _mm256_add_epi32(pl, ph));
            }
        }
        for (int t = 0; t < T; t++) {
            const or_q8k_block *y = &in[b * rows + base + t];
            float d = y->d * xd;
            float dmin = -y->d * xdmin;
            acc[t] = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi[t]), acc[t]);
            __m256i q8sums = _mm256_loadu_si256((const __m256i *)y->bsums);
            __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
            __m128i prod = _mm_madd_epi16(mins128, q8s);
            accm[t] = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), accm[t]);
        }
    }
    for (int t = 0; t < T; t++) out[base + t] = hsum_f32_8(acc[t]) + hsum_f32_4(accm[t]);
}

static inline __attribute__((always_inline)) void q6k_tile(const or_q6k_block *w, size_t nb, const or_q8k_block *in,
                                                           size_t rows, size_t base, float *out, const int T) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m256i m2 = _mm256_set1_epi8(3);
    const __m256i m32s = _mm256_set1_epi8(32);
    __m256 acc[8];
    for (int t = 0; t < T; t++) acc[t] = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        float xd = or_f16_to_f32(w[b].d);
        __m128i scales = _mm_loadu_si128((const __m128i *)w[b].scales);
        __m256i sumi[8];
        for (int t = 0; t < T; t++) sumi[t] = _mm256_setzero_si256();
        for (int j = 0; j < 2; j++) {
            __m256i b1 = _mm256_loadu_si256((const __m256i *)(w[b].ql + 64 * j));
            __m256i b2 = _mm256_loadu_si256((const __m256i *)(w[b].ql + 64 * j + 32));
            __m256i bh = _mm256_loadu_si256((const __m256i *)(w[b].qh + 32 * j));
            __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(bh, m2), 4);
            __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 2), m2), 4);
            __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 4), m2), 4);
            __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 6), m2), 4);
            __m256i q0 = _mm256_or_si256(_mm256_and_si256(b1, m4), h0);
            __m256i q1 = _mm256_or_si256(_mm256_and_si256(b2, m4), h1);
            __m256i q2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b1, 4), m4), h2);
            __m256i q3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b2, 4), m4), h3);
            int is = 4 * j;
            __m256i s0 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, q6_pair(is)));
            __m256i s1 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, q6_pair(is + 1)));
            __m256i s2 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, q6_pair(is + 2)));
            __m256i s3 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, q6_pair(is + 3)));
            for (int t = 0; t < T; t++) {
                const or_q8k_block *y = &in[b * rows + base + t];
                const int8_t *p = y->qs + 128 * j;
                __m256i a0 = _mm256_loadu_si256((const __m256i *)p);
                __m256i a1 = _mm256_loadu_si256((const __m256i *)(p + 32));
                __m256i a2 = _mm256_loadu_si256((const __m256i *)(p + 64));
                __m256i a3 = _mm256_loadu_si256((const __m256i *)(p + 96));
                __m256i p0 = _mm256_sub_epi16(_mm256_maddubs_epi16(q0, a0), _mm256_maddubs_epi16(m32s, a0));
                __m256i p1 = _mm256_sub_epi16(_mm256_maddubs_epi16(q1, a1), _mm256_maddubs_epi16(m32s, a1));
                __m256i p2 = _mm256_sub_epi16(_mm256_maddubs_epi16(q2, a2), _mm256_maddubs_epi16(m32s, a2));
                __m256i p3 = _mm256_sub_epi16(_mm256_maddubs_epi16(q3, a3), _mm256_maddubs_epi16(m32s, a3));
                p0 = _mm256_madd_epi16(s0, p0);
                p1 = _mm256_madd_epi16(s1, p1);
                p2 = _mm256_madd_epi16(s2, p2);
                p3 = _mm256_madd_epi16(s3, p3);
                sumi[t] = _mm256_add_epi32(sumi[t], _mm256_add_epi32(_mm256_add_epi32(p0, p1), _mm256_add_epi32(p2, p3)));
            }
        }
        for (int t = 0; t < T; t++) {
            const or_q8k_block *y = &in[b * rows + base + t];
            acc[t] = _mm256_fmadd_ps(_mm256_set1_ps(y->d * xd), _mm256_cvtepi32_ps(sumi[t]), acc[t]);
        }
    }
    for (int t = 0; t < T; t++) out[base + t] = hsum_f32_8(acc[t]);
}

static inline __attribute__((always_inline)) void q80_tile(const or_q80_block *w, size_t nb, const or_q80_block *in,
                                                           size_t rows, size_t base, float *out, const int T) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc[8];
    for (int t = 0; t < T; t++) acc[t] = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        __m256i bx = _mm256_loadu_si256((const __m256i *)w[b].qs);
        __m256i ax = _mm256_sign_epi8(bx, bx);
        float xd = or_f16_to_f32(w[b].d);
        for (int t = 0; t < T; t++) {
            const or_q80_block *y = &in[b * rows + base + t];
            __m256i by = _mm256_loadu_si256((const __m256i *)y->qs);
            __m256i sy = _mm256_sign_epi8(by, bx);
            __m256i dot = _mm256_madd_epi16(ones, _mm256_maddubs_epi16(ax, sy));
            __m256 d = _mm256_set1_ps(xd * or_f16_to_f32(y->d));
            acc[t] = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(dot), acc[t]);
        }
    }
    for (int t = 0; t < T; t++) out[base + t] = hsum_f32_8(acc[t]);
}

#define TILED_ENTRY(NAME, TILEFN, WT, IT)                                                   \
    int NAME(const WT *w, size_t nb, const IT *in, size_t rows, float *out) {               \
        size_t base = 0;                                                                    \
        while (base + 8 <= rows) {                                                          \
            TILEFN(w, nb, in, rows, base, out, 8);                                          \
            base += 8;                                                                      \
        }                                                                                   \
        switch (rows - base) {                                                              \
        case 0: break;                                                                      \
        case 1: TILEFN(w, nb, in, rows, base, out, 1); break;                               \
        case 2: TILEFN(w, nb, in, rows, base, out, 2); break;                               \
        case 3: TILEFN(w, nb, in, rows, base, out, 3); break;                               \
        case 4: TILEFN(w, nb, in, rows, base, out, 4); break;                               \
        case 5: TILEFN(w, nb, in, rows, base, out, 5); break;                               \
        case 6: TILEFN(w, nb, in, rows, base, out, 6); break;                               \
        default: TILEFN(w, nb, in, rows, base, out, 7); break;                              \
        }                                                                                   \
        return 0;                                                                           \
    }

TILED_ENTRY(or_q4k_q8k_row_avx2, q4k_tile, or_q4k_block, or_q8k_block)
TILED_ENTRY(or_q6k_q8k_row_avx2, q6k_tile, or_q6k_block, or_q8k_block)
TILED_ENTRY(or_q80_q80_row_avx2, q80_tile, or_q80_block, or_q80_block)

#else /* no AVX2 at build time */

int or_have_avx2(void) { return 0; }
int or_q4k_q8k_row_avx2(const or_q4k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out) {
    (void)w; (void)nb; (void)in; (void)rows; (void)out;
    return -1;
}
int or_q6k_q8k_row_avx2(const or_q6k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out) {
    (void)w; (void)nb; (void)in; (void)rows; (void)out;
    return -1;
}
int or_q80_q80_row_avx2(const or_q80_block *w, size_t nb, const or_q80_block *in, size_t rows, float *out) {
    (void)w; (void)nb; (void)in; (void)rows; (void)out;
    return -1;
}
#endif
