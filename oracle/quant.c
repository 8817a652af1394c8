/*
 * quant.c -- TEST INFRASTRUCTURE (parity oracle, see iq_oracle.h).
 *
 * f16 conversions, activation quantisers (candle from_float restatements),
 * K-quant scale unpacking, the scalar lane-exact per-block integers, the
 * textbook per-block integers and GGUF dequantisation.
 */
#include <math.h>
#include <string.h>

#include "iq_oracle.h"

_Static_assert(sizeof(or_q4k_block) == 144, "Q4_K block is 144 bytes");
_Static_assert(sizeof(or_q5k_block) == 176, "Q5_K block is 176 bytes");
_Static_assert(sizeof(or_q6k_block) == 210, "Q6_K block is 210 bytes");
_Static_assert(sizeof(or_q80_block) == 34, "Q8_0 block is 34 bytes");
_Static_assert(sizeof(or_q8k_block) == 292, "Q8K block is 292 bytes");

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    float f;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24 is exact in binary32 */
        f = (float)man * 0x1p-24f;
        uint32_t bits;
        memcpy(&bits, &f, 4);
        bits |= sign;
        memcpy(&f, &bits, 4);
        return f;
    }
    uint32_t bits;
    if (exp == 31)
        bits = sign | 0x7f800000u | (man << 13);
    else
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        /* result is subnormal (or zero) in binary16: value / 2^-24, RNE */
        if (ax < 0x33000000u) /* < 2^-25: rounds to zero (2^-25 itself ties to even 0) */
            return (uint16_t)sign;
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); want units of 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u)))
            q++;
        return (uint16_t)(sign | q);
    }
    /* normal: rebias and round the 13 dropped bits to nearest even */
    uint32_t r = ax - 0x38000000u; /* exponent 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
        q++;
    return (uint16_t)(sign | q);
}

size_t or_block_bytes(int dtype) {
    switch (dtype) {
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_Q8_0: return 34;
    default: return 0;
    }
}

size_t or_block_elems(int dtype) {
    switch (dtype) {
    case OR_Q4_K:
    case OR_Q5_K:
    case OR_Q6_K: return 256;
    case OR_Q8_0: return 32;
    default: return 0;
    }
}

/* Rust `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v <= -128.f) return -128;
    if (v >= 127.f) return 127;
    return (int8_t)v;
}

int or_quantize_q8k(const float *x, size_t k, or_q8k_block *out) {
    if (k % 256) return -1;
    for (size_t i = 0; i < k / 256; i++) {
        const float *xs = x + 256 * i;
        or_q8k_block *y = out + i;
        float max = 0.f, amax = 0.f;
        for (int j = 0; j < 256; j++) {
            float ax = fabsf(xs[j]);
            if (amax < ax) { /* strict: the first element reaching |max| wins */
                amax = ax;
                max = xs[j];
            }
        }
        memset(y->bsums, 0, sizeof y->bsums);
        if (amax == 0.f) {
            y->d = 0.f;
            memset(y->qs, 0, sizeof y->qs);
            continue;
        }
        float iscale = -128.f / max;
        for (int j = 0; j < 256; j++) {
            float v = roundf(iscale * xs[j]); /* round half away from zero */
            y->qs[j] = sat_i8(v < 127.f ? v : 127.f);
        }
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int ii = 0; ii < 16; ii++) s += y->qs[16 * j + ii];
            y->bsums[j] = (int16_t)s;
        }
        y->d = 1.f / iscale;
    }
    return 0;
}

int or_quantize_q80(const float *x, size_t k, or_q80_block *out) {
    if (k % 32) return -1;
    for (size_t i = 0; i < k / 32; i++) {
        const float *xs = x + 32 * i;
        float amax = 0.f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xs[j]));
        float d = amax / 127.f;
        float id = d != 0.f ? 1.f / d : 0.f;
        out[i].d = or_f32_to_f16(d);
        for (int j = 0; j < 32; j++) out[i].qs[j] = sat_i8(roundf(xs[j] * id));
    }
    return 0;
}

void or_unpack_k_scales(const uint8_t b[12], uint8_t sc[8], uint8_t mn[8]) {
    /* Six-bit scale s and min s of a K-quant super-block.  The first four
     * of each sit in the low six bits of bytes 0..7; the last four are
     * split between a nibble of bytes 8..11 and the top two bits of
     * bytes 0..7. */
    for (int s = 0; s < 4; s++) {
        sc[s] = b[s] & 63;
        mn[s] = b[s + 4] & 63;
    }
    for (int s = 4; s < 8; s++) {
        sc[s] = (uint8_t)((b[s + 4] & 15) | ((b[s - 4] >> 6) << 4));
        mn[s] = (uint8_t)((b[s + 4] >> 4) | ((b[s] >> 6) << 4));
    }
}

/* Scalar emulation of the AVX2 lanes.  Lane k of a 256-bit i32 vector built
 * by madd(maddubs(w, x)) holds the four products of bytes 4k..4k+3 of a
 * 32-byte chunk; the chunks of one block are summed into the same lane. */
void or_q4k_block_lanes(const or_q4k_block *w, const or_q8k_block *x, int32_t isum[8], int32_t msum[4]) {
    uint8_t sc[8], mn[8];
    or_unpack_k_scales(w->scales, sc, mn);
    for (int k = 0; k < 8; k++) {
        int32_t s = 0;
        for (int j = 0; j < 4; j++) {
            int32_t lo = 0, hi = 0;
            for (int b = 4 * k; b < 4 * k + 4; b++) {
                uint8_t q = w->qs[32 * j + b];
                lo += (int32_t)(q & 15) * x->qs[64 * j + b];
                hi += (int32_t)(q >> 4) * x->qs[64 * j + 32 + b];
            }
            s += (int32_t)sc[2 * j] * lo + (int32_t)sc[2 * j + 1] * hi;
        }
        isum[k] = s;
    }
    int16_t q8s[8]; /* hadd of the sixteen bsums: one sum per 32-weight sub-block */
    for (int i = 0; i < 8; i++) q8s[i] = (int16_t)(x->bsums[2 * i] + x->bsums[2 * i + 1]);
    for (int k = 0; k < 4; k++)
        msum[k] = (int32_t)mn[2 * k] * q8s[2 * k] + (int32_t)mn[2 * k + 1] * q8s[2 * k + 1];
}

void or_q5k_block_lanes(const or_q5k_block *w, const or_q8k_block *x, int32_t isum[8], int32_t msum[4]) {
    uint8_t sc[8], mn[8];
    or_unpack_k_scales(w->scales, sc, mn);
    for (int k = 0; k < 8; k++) {
        int32_t s = 0;
        for (int j = 0; j < 4; j++) {
            int32_t lo = 0, hi = 0;
            for (int b = 4 * k; b < 4 * k + 4; b++) {
                uint8_t q = w->qs[32 * j + b];
                int32_t h0 = (w->qh[b] >> (2 * j)) & 1, h1 = (w->qh[b] >> (2 * j + 1)) & 1;
                lo += ((int32_t)(q & 15) + 16 * h0) * x->qs[64 * j + b];
                hi += ((int32_t)(q >> 4) + 16 * h1) * x->qs[64 * j + 32 + b];
            }
            s += (int32_t)sc[2 * j] * lo + (int32_t)sc[2 * j + 1] * hi;
        }
        isum[k] = s;
    }
    int16_t q8s[8];
    for (int i = 0; i < 8; i++) q8s[i] = (int16_t)(x->bsums[2 * i] + x->bsums[2 * i + 1]);
    for (int k = 0; k < 4; k++)
        msum[k] = (int32_t)mn[2 * k] * q8s[2 * k] + (int32_t)mn[2 * k + 1] * q8s[2 * k + 1];
}

void or_q6k_block_lanes(const or_q6k_block *w, const or_q8k_block *x, int32_t isum[8]) {
    for (int k = 0; k < 8; k++) {
        int32_t s = 0;
        for (int j = 0; j < 2; j++) {
            for (int i = 0; i < 4; i++) {
                int32_t sc = w->scales[8 * j + 2 * i + (k >= 4)];
                int32_t p = 0;
                for (int b = 4 * k; b < 4 * k + 4; b++) {
                    uint8_t l = w->ql[64 * j + 32 * (i & 1) + b];
                    int32_t lo = i < 2 ? (l & 15) : (l >> 4);
                    int32_t hi = (w->qh[32 * j + b] >> (2 * i)) & 3;
                    p += ((lo | (hi << 4)) - 32) * x->qs[128 * j + 32 * i + b];
                }
                s += sc * p;
            }
        }
        isum[k] = s;
    }
}

void or_q80_block_lanes(const or_q80_block *w, const or_q80_block *x, int32_t isum[8]) {
    for (int k = 0; k < 8; k++) {
        int32_t s = 0;
        for (int b = 4 * k; b < 4 * k + 4; b++) s += (int32_t)w->qs[b] * x->qs[b];
        isum[k] = s;
    }
}

/* ---- textbook forms, indexed by weight element, from the dequantisation
 * formulas (ggml dequantize_row_q4_K / q6_K / q8_0). ---- */

static int q4k_elem(const or_q4k_block *w, int e, int *sub) {
    int j = e / 64, r = e % 64;
    *sub = 2 * j + (r >= 32);
    uint8_t q = w->qs[32 * j + (r % 32)];
    return r < 32 ? (q & 15) : (q >> 4);
}

/* ggml dequantize_row_q5_K: weight 64j + l takes the low nibble of
 * qs[32j + l] and bit 2j of qh[l]; weight 64j + 32 + l the high nibble and
 * bit 2j + 1. */
static int q5k_elem(const or_q5k_block *w, int e, int *sub) {
    int j = e / 64, r = e % 64, l = r % 32;
    *sub = 2 * j + (r >= 32);
    uint8_t q = w->qs[32 * j + l];
    int lo = r < 32 ? (q & 15) : (q >> 4);
    int hi = (w->qh[l] >> (2 * j + (r >= 32))) & 1;
    return lo + 16 * hi;
}

static int q6k_elem(const or_q6k_block *w, int e) {
    int h = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
    uint8_t lq = w->ql[64 * h + 32 * (quarter & 1) + l];
    int lo = quarter < 2 ? (lq & 15) : (lq >> 4);
    int hi = (w->qh[32 * h + l] >> (2 * quarter)) & 3;
    return (lo | (hi << 4)) - 32;
}

void or_q4k_block_textbook(const or_q4k_block *w, const or_q8k_block *x, int64_t *isum, int64_t *msum) {
    uint8_t sc[8], mn[8];
    or_unpack_k_scales(w->scales, sc, mn);
    int64_t is = 0, ms = 0;
    for (int e = 0; e < 256; e++) {
        int sub;
        int q = q4k_elem(w, e, &sub);
        is += (int64_t)sc[sub] * q * x->qs[e];
        ms += (int64_t)mn[sub] * x->qs[e];
    }
    *isum = is;
    *msum = ms;
}

void or_q5k_block_textbook(const or_q5k_block *w, const or_q8k_block *x, int64_t *isum, int64_t *msum) {
    uint8_t sc[8], mn[8];
    or_unpack_k_scales(w->scales, sc, mn);
    int64_t is = 0, ms = 0;
    for (int e = 0; e < 256; e++) {
        int sub;
        int q = q5k_elem(w, e, &sub);
        is += (int64_t)sc[sub] * q * x->qs[e];
        ms += (int64_t)mn[sub] * x->qs[e];
    }
    *isum = is;
    *msum = ms;
}

void or_q6k_block_textbook(const or_q6k_block *w, const or_q8k_block *x, int64_t *isum) {
    int64_t is = 0;
    for (int e = 0; e < 256; e++) is += (int64_t)w->scales[e / 16] * q6k_elem(w, e) * x->qs[e];
    *isum = is;
}

void or_q80_block_textbook(const or_q80_block *w, const or_q80_block *x, int64_t *isum) {
    int64_t is = 0;
    for (int e = 0; e < 32; e++) is += (int64_t)w->qs[e] * x->qs[e];
    *isum = is;
}

int or_dequantize(int dtype, const void *blocks, size_t n_rows, size_t cols, float *out) {
    size_t be = or_block_elems(dtype);
    if (!be || cols % be) return -1;
    size_t nb = n_rows * (cols / be);
    for (size_t i = 0; i < nb; i++) {
        float *y = out + i * be;
        if (dtype == OR_Q4_K) {
            const or_q4k_block *w = (const or_q4k_block *)blocks + i;
            uint8_t sc[8], mn[8];
            or_unpack_k_scales(w->scales, sc, mn);
            float d = or_f16_to_f32(w->d), dmin = or_f16_to_f32(w->dmin);
            for (int e = 0; e < 256; e++) {
                int sub;
                int q = q4k_elem(w, e, &sub);
                y[e] = d * sc[sub] * q - dmin * mn[sub];
            }
        } else if (dtype == OR_Q5_K) {
            const or_q5k_block *w = (const or_q5k_block *)blocks + i;
            uint8_t sc[8], mn[8];
            or_unpack_k_scales(w->scales, sc, mn);
            float d = or_f16_to_f32(w->d), dmin = or_f16_to_f32(w->dmin);
            for (int e = 0; e < 256; e++) {
                int sub;
                int q = q5k_elem(w, e, &sub);
                y[e] = d * sc[sub] * q - dmin * mn[sub];
            }
        } else if (dtype == OR_Q6_K) {
            const or_q6k_block *w = (const or_q6k_block *)blocks + i;
            float d = or_f16_to_f32(w->d);
            for (int e = 0; e < 256; e++) y[e] = d * w->scales[e / 16] * q6k_elem(w, e);
        } else {
            const or_q80_block *w = (const or_q80_block *)blocks + i;
            float d = or_f16_to_f32(w->d);
            for (int e = 0; e < 32; e++) y[e] = d * w->qs[e];
        }
    }
    return 0;
}
