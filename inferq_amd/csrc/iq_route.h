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

constexpr int kRoutePer = 8;  // logits per lane (E <= 512)

// Logits per lane: lane l holds logits per*l .. per*l + per - 1, so lane
// order is index order.
__device__ __forceinline__ int route_per(int E) { return E <= 256 ? 4 : 8; }

// Order-preserving 32-bit key of a logit (NaN lowest among logits, -0 == +0);
// 0 is below every key and marks "taken" or "absent".
__device__ __forceinline__ uint32_t route_ukey(float x) {
    if (x != x) x = -INFINITY;
    if (x == 0.f) x = 0.f;
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The lane's logits (-inf past E), 16-byte loads when E is 256 or 512 and
// the row is aligned.
__device__ __forceinline__ void route_load(const float* lg, int E, float (&lv)[kRoutePer]) {
    const int lane = threadIdx.x & 63;
    const int per = route_per(E);
    if ((E == 256 || E == 512) && ((uintptr_t)lg & 15) == 0) {
        const f32x4* v = (const f32x4*)(lg + per * lane);
        const f32x4 a = v[0];
        f32x4 b = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (E == 512) b = v[1];
        lv[0] = a.x; lv[1] = a.y; lv[2] = a.z; lv[3] = a.w;
        lv[4] = b.x; lv[5] = b.y; lv[6] = b.z; lv[7] = b.w;
        return;
    }
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) {
        const int i = per * lane + j;
        lv[j] = (j < per && i < E) ? lg[i] : -INFINITY;
    }
}

// Top-`count` experts by (logit desc, index asc) from route_load's values:
// sel[0..count) wave-uniform.  Each round takes the wave maximum of the
// lanes' largest remaining keys; the lowest lane holding it holds the lowest
// index among equal logits (lane order is index order), and within that lane
// the first position holding it is the lowest.
template <int MAXK, int PER>
__device__ __forceinline__ void route_topk_vals(const float (&lv)[kRoutePer], int E, int count, int (&sel)[MAXK]) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) key[j] = PER * lane + j < E ? route_ukey(lv[j]) : 0u;
    for (int s = 0; s < count; s++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < PER; j++) m = max(m, key[j]);
        const uint32_t best = wave_max_u32(m);
        const int L = (int)__builtin_ctzll(__ballot(m == best));
        int jf = PER - 1;
#pragma unroll
        for (int j = PER - 2; j >= 0; j--) jf = key[j] == m ? j : jf;
        const int j = __builtin_amdgcn_readlane(jf, L);
#pragma unroll
        for (int q = 0; q < PER; q++) key[q] = (lane == L && q == j) ? 0u : key[q];
        sel[s] = PER * L + j;
    }
}

// route_topk_vals with each pick handed to store(s, expert) as it is found
// (wave-uniform arguments) instead of written into an array indexed by the
// round: kernels whose register budget is tight would otherwise keep that
// array in scratch memory, on the routing's dependent chain.
template <int PER, class Store>
__device__ __forceinline__ void route_topk_each(const float (&lv)[kRoutePer], int E, int count, Store&& store) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) key[j] = PER * lane + j < E ? route_ukey(lv[j]) : 0u;
    for (int s = 0; s < count; s++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < PER; j++) m = max(m, key[j]);
        const uint32_t best = wave_max_u32(m);
        const int L = (int)__builtin_ctzll(__ballot(m == best));
        int jf = PER - 1;
#pragma unroll
        for (int j = PER - 2; j >= 0; j--) jf = key[j] == m ? j : jf;
        const int j = __builtin_amdgcn_readlane(jf, L);
#pragma unroll
        for (int q = 0; q < PER; q++) key[q] = (lane == L && q == j) ? 0u : key[q];
        store(s, PER * L + j);
    }
}

template <class Store>
__device__ __forceinline__ void route_topk_each_any(const float (&lv)[kRoutePer], int E, int count, Store&& store) {
    if (E <= 256) route_topk_each<4>(lv, E, count, store);
    else route_topk_each<kRoutePer>(lv, E, count, store);
}

// The expert at rank s (0-based) of the same order, wave-uniform, without
// the s rounds before it: a bitwise search for T, the (s+1)-th largest key
// counted with multiplicity (the largest value with at least s+1 keys at or
// above it; keys are counted by ballots, so each step is a few compares and
// scalar population counts), stopping once exactly s+1 keys lie at or above
// the candidate (T is then their minimum); the expert is then the
// (s - #{keys > T})-th lowest index among the keys equal to T.  Fewer VALU
// ops than the rounds, but a longer dependent chain: it pays where many
// workgroups share the SIMDs (several tokens), not for one token.
template <int PER>
__device__ __forceinline__ int route_rank_vals(const float (&lv)[kRoutePer], int E, int s) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) key[j] = PER * lane + j < E ? route_ukey(lv[j]) : 0u;
    uint32_t lo = 0;  // invariant: at least s+1 keys are >= lo
    bool exact = false;
    for (int b = 31; b >= 0; b--) {
        const uint32_t c = lo | (1u << b);
        int n = 0;
#pragma unroll
        for (int q = 0; q < PER; q++) n += __builtin_popcountll(__ballot(key[q] >= c));
        if (n > s) {
            lo = c;
            if (n == s + 1) {
                exact = true;
                break;
            }
        }
    }
    uint32_t T = lo;
    if (exact) {
        uint32_t mn = 0xffffffffu;
#pragma unroll
        for (int q = 0; q < PER; q++) mn = key[q] >= lo ? min(mn, key[q]) : mn;
        T = ~wave_max_u32(~mn);
    }
    int above = 0;
#pragma unroll
    for (int q = 0; q < PER; q++) above += __builtin_popcountll(__ballot(key[q] > T));
    for (int r = s - above;; r--) {  // r-th lowest index among the keys equal to T
        bool has = false;
        int jf = PER - 1;
#pragma unroll
        for (int j = PER - 1; j >= 0; j--) {
            has = has || key[j] == T;
            jf = key[j] == T ? j : jf;
        }
        const int L = (int)__builtin_ctzll(__ballot(has));
        const int j = __builtin_amdgcn_readlane(jf, L);
        if (r <= 0) return PER * L + j;
#pragma unroll
        for (int q = 0; q < PER; q++) key[q] = (lane == L && q == j) ? 0u : key[q];
    }
}

__device__ __forceinline__ int route_rank(const float (&lv)[kRoutePer], int E, int s) {
    return E <= 256 ? route_rank_vals<4>(lv, E, s) : route_rank_vals<kRoutePer>(lv, E, s);
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
    const int per = route_per(E);
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) {
        const int i = per * lane + j;
        if (j < per && i < E) scratch[i] = exp_f32(lv[j] - mx);
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

// route_weights in two parts that can run on different waves: the softmax
// denominator (exp(x - max) of every logit into `scratch`, E floats of LDS,
// and their sequential sum in index order; independent of the selection),
// then the picks' weights from it with the picks read from LDS (sel[0..K))
// and written to LDS (w[0..K), lane 0).  The same operations in the same
// order as route_weights, and no per-lane array indexed by the rank.
__device__ __forceinline__ float route_softmax_den(const float (&lv)[kRoutePer], int E, float* scratch) {
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) mx = fmaxf(mx, lv[j]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    const int per = route_per(E);
#pragma unroll
    for (int j = 0; j < kRoutePer; j++) {
        const int i = per * lane + j;
        if (j < per && i < E) scratch[i] = exp_f32(lv[j] - mx);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
    return den;
}

__device__ __forceinline__ void route_pick_weights(float den, int K, const int* sel, int normalize,
                                                   const float* scratch, float* w) {
    const int lane = threadIdx.x & 63;
    float sum = 0.f;
    for (int s = 0; s < K; s++) sum = sum + __fdiv_rn(scratch[sel[s]], den);
    for (int s = 0; s < K; s++) {
        const float ws = __fdiv_rn(scratch[sel[s]], den);
        if (lane == 0) w[s] = normalize ? __fdiv_rn(ws, sum) : ws;
    }
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
