// iq_route.h -- MoE routing inside a wave (src/qwen/moe.rs:21-54).
//
// Selection.  The reference ranks experts by softmax probability with an
// unstable sort.  Probability is a non-decreasing function of the logit
// (x - max, exp and the division by one denominator are all monotone), so
// ranking by logit -- larger first, equal logits by lower index -- is one of
// the orders the reference can produce, and the only one where it leaves a
// choice (exactly equal probabilities) is fixed deterministically.  The
// oracle uses the same resolution.
//
// Weights.  p = exp(x - max) / sum_i exp(x_i - max) with the denominator
// summed sequentially in index order, then renormalised over the top k by
// a sequential sum in rank order, exactly as the reference.
#pragma once

#include "iq_device.h"

namespace iq {

// Order-preserving 64-bit key: logit (NaN ranks lowest, -0 equals +0) in
// the high word, complemented index in the low word.  0 marks "taken".
__device__ __forceinline__ uint64_t route_key(float x, int idx) {
    if (x != x) x = -INFINITY;
    if (x == 0.f) x = 0.f;
    uint32_t b = __builtin_bit_cast(uint32_t, x);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t dpp64(uint64_t v, int ctrl_sel) {
    int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    switch (ctrl_sel) {
    case 0: lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false); break;
    case 1: lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false); break;
    case 2: lo = __builtin_amdgcn_mov_dpp(lo, 0x124, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x124, 0xF, 0xF, false); break;
    default: lo = __builtin_amdgcn_mov_dpp(lo, 0x128, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x128, 0xF, 0xF, false); break;
    }
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Maximum of v over the 64 lanes of the wave (every lane gets it).
__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
    v = umax64(v, dpp64(v, 0));  // quad: xor 1
    v = umax64(v, dpp64(v, 1));  // quad: xor 2
    v = umax64(v, dpp64(v, 2));  // row: rotate 4
    v = umax64(v, dpp64(v, 3));  // row: rotate 8
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    uint64_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; row++) {
        const uint64_t rv = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 16 * row) << 32) |
                            (uint32_t)__builtin_amdgcn_readlane(lo, 16 * row);
        r = umax64(r, rv);
    }
    return r;
}

constexpr int kRoutePer = 8;  // logits per lane (E <= 512)

// Order-preserving 32-bit key of a logit (NaN lowest among logits, -0 == +0);
// 0 is below every key and marks "taken" or "absent".
__device__ __forceinline__ uint32_t route_ukey(float x) {
    if (x != x) x = -INFINITY;
    if (x == 0.f) x = 0.f;
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false));
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return max(a, b);
}

// Lane l's logits l + 64 j (-inf past E).
__device__ __forceinline__ void route_load(const float* lg, int E, float (&lv)[kRoutePer]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) {
        const int i = lane + 64 * j;
        lv[j] = i < E ? lg[i] : -INFINITY;
    }
}

// Top-`count` experts by (logit desc, index asc) from route_load's values:
// sel[0..count) wave-uniform.  PER = logits per lane actually present
// (ceil(E / 64)).  Each round takes the wave maximum of the 32-bit keys,
// then the lowest index holding it (first non-empty ballot, lowest lane).
template <int MAXK, int PER>
__device__ __forceinline__ void route_topk_vals(const float (&lv)[kRoutePer], int E, int count, int (&sel)[MAXK]) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = lane + 64 * j;
        key[j] = i < E ? route_ukey(lv[j]) : 0u;
    }
    for (int s = 0; s < count; s++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < PER; j++) m = max(m, key[j]);
        const uint32_t best = wave_max_u32(m);
        int win = -1;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const unsigned long long b = __ballot(key[j] == best);
            if (win < 0 && b) win = (__ffsll((long long)b) - 1) + 64 * j;
        }
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (win == lane + 64 * j) key[j] = 0u;
        sel[s] = win;
    }
}

template <int MAXK>
__device__ __forceinline__ void route_topk_any(const float (&lv)[kRoutePer], int E, int count, int (&sel)[MAXK]) {
    if (E <= 256) route_topk_vals<MAXK, 4>(lv, E, count, sel);
    else route_topk_vals<MAXK, kRoutePer>(lv, E, count, sel);
}

template <int MAXK>
__device__ __forceinline__ void route_topk(const float* lg, int E, int count, int (&sel)[MAXK], float (&lv)[kRoutePer]) {
    route_load(lg, E, lv);
    route_topk_any<MAXK>(lv, E, count, sel);
}

// Exact routing weights of the selected experts (one wave; `scratch` holds
// E floats of LDS).  lv are the lane's logits from route_topk.
template <int MAXK>
__device__ __forceinline__ void route_weights(const float (&lv)[kRoutePer], int E, int K, const int (&sel)[MAXK],
                                              int normalize, float* scratch, float (&w)[MAXK]) {
    const int lane = threadIdx.x & 63;
    // max over all logits, NaN ignored (fold from -inf with f32::max)
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) mx = fmaxf(mx, lv[j]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) {
        const int i = lane + 64 * j;
        if (i < E) scratch[i] = exp_f32(lv[j] - mx);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the softmax denominator: a sequential f32 sum in index order (loads
    // batched 16 at a time so the LDS latency overlaps the add chain)
    float den = 0.f;
    int i = 0;
    for (; i + 16 <= E; i += 16) {
        const f32x4 t0 = *(const f32x4*)(scratch + i), t1 = *(const f32x4*)(scratch + i + 4);
        const f32x4 t2 = *(const f32x4*)(scratch + i + 8), t3 = *(const f32x4*)(scratch + i + 12);
        den = den + t0.x; den = den + t0.y; den = den + t0.z; den = den + t0.w;
        den = den + t1.x; den = den + t1.y; den = den + t1.z; den = den + t1.w;
        den = den + t2.x; den = den + t2.y; den = den + t2.z; den = den + t2.w;
        den = den + t3.x; den = den + t3.y; den = den + t3.z; den = den + t3.w;
    }
    for (; i < E; i++) den = den + scratch[i];
    float sum = 0.f;
    for (int s = 0; s < K; s++) {
        w[s] = __fdiv_rn(scratch[sel[s]], den);
        sum = sum + w[s];
    }
    if (normalize)
        for (int s = 0; s < K; s++) w[s] = __fdiv_rn(w[s], sum);
}

}  // namespace iq

namespace iq {

// First 32 terms per lane of selector_gate (h = lane + 64 j, j < 32),
// loaded ahead of other traffic; selector_gate_vals finishes the sum in the
// same order as selector_gate.
__device__ __forceinline__ void selector_load(const float* x, const float* sel, int64_t H, float (&xv)[32],
                                              float (&sv)[32]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int64_t h = lane + 64 * j;
        xv[j] = h < H ? x[h] : 0.f;
        sv[j] = h < H ? sel[h] : 0.f;
    }
}

__device__ __forceinline__ float selector_gate_vals(const float (&xv)[32], const float (&sv)[32], const float* x,
                                                    const float* sel, int64_t H) {
    const int lane = threadIdx.x & 63;
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++)
        if (lane + 64 * j < H) part = part + xv[j] * sv[j];
    for (int64_t h = 2048 + lane; h < H; h += 64) part = part + x[h] * sel[h];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
    return __fdiv_rn(1.f, exp_f32(-part) + 1.f);
}

// sigmoid(x . selector) for the shared expert gate (one wave).  The
// reference computes x . selector with candle's f32 gemm, whose summation
// order is not visible; here each lane sums x[h] * s[h] over h = lane + 64 j
// in order of j, and the lanes meet in a fixed butterfly -- identically in
// every kernel that needs the gate.  Loads go 16 per lane at a time.
__device__ __forceinline__ float selector_gate(const float* x, const float* sel, int64_t H) {
    const int lane = threadIdx.x & 63;
    float part = 0.f;
    int64_t h0 = 0;
    for (; h0 + 64 * 16 <= H; h0 += 64 * 16) {
        float xv[16], sv[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            xv[j] = x[h0 + lane + 64 * j];
            sv[j] = sel[h0 + lane + 64 * j];
        }
#pragma unroll
        for (int j = 0; j < 16; j++) part = part + xv[j] * sv[j];
    }
    for (int64_t h = h0 + lane; h < H; h += 64) part = part + x[h] * sel[h];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
    return __fdiv_rn(1.f, exp_f32(-part) + 1.f);
}

}  // namespace iq
