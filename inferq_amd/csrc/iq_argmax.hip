// iq_argmax.hip -- greedy selection over logit rows (sampling::argmax,
// src/sampling.rs:104-110): the index of the largest finite value; among
// equal values the last index (Rust's Iterator::max_by keeps the later of
// two equal elements, and partial_cmp makes -0 equal to +0); non-finite
// values are skipped; -1 when a row has no finite value (the reference's
// "all logits are non-finite" error).
//
// Over logits in memory, two launches, no atomics: k_argmax_part reduces
// chunks of a row to one key each, k_argmax_final reduces a row's chunk
// keys.  A key (argmax_key) is the order-preserving image of the value in
// the high 32 bits and the index in the low 32, so the largest key is the
// largest value and, among equal values, the largest index; 0 (below every
// finite value's key) marks "no finite value".  Fused into the LM head's
// product (iq_matmul_argmax at 1..8 rows), the product kernels leave one
// (key, logit) pair per wave or workgroup as they write the logits, and
// k_argmax_final_kv joins them: one launch instead of two and no re-read of
// the logits (LM head [248320 x 2048] Q6_K, graph replays: 76.1 -> 71.3 us
// per call at one row, 106 -> 104 us at eight, against 66.7 / 96-99 us for
// the product alone).
#include "iq_device.h"
#include "iq_internal.h"

namespace iq {

namespace {

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPerThread = 16;
constexpr int64_t kArgmaxChunk = (int64_t)kArgmaxThreads * kArgmaxPerThread;

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Maximum key over the workgroup, valid in thread 0.
__device__ __forceinline__ uint64_t block_max(uint64_t key) {
    __shared__ uint64_t s_part[kArgmaxThreads / 64];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)key, off), hi = __shfl_xor((uint32_t)(key >> 32), off);
        key = max_u64(key, ((uint64_t)hi << 32) | lo);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) s_part[wave] = key;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < kArgmaxThreads / 64; w++) key = max_u64(key, s_part[w]);
    return key;
}

// Grid (chunks, m): chunk c of row r covers [c * kArgmaxChunk, ...).
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_part(const float* __restrict__ y, int64_t ldy, int64_t n,
                                                                uint64_t* __restrict__ part, int chunks) {
    const int64_t r = blockIdx.y;
    const int64_t base = (int64_t)blockIdx.x * kArgmaxChunk;
    const float* row = y + r * ldy;
    uint64_t key = 0;
#pragma unroll
    for (int j = 0; j < kArgmaxPerThread; j++) {
        const int64_t i = base + (int64_t)j * kArgmaxThreads + threadIdx.x;
        if (i < n) key = max_u64(key, argmax_key(row[i], i));
    }
    key = block_max(key);
    if (threadIdx.x == 0) part[r * chunks + blockIdx.x] = key;
}

// Grid m: the row's chunk keys to (index, value).
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_final(const float* __restrict__ y, int64_t ldy,
                                                                 const uint64_t* __restrict__ part, int chunks,
                                                                 int32_t* __restrict__ idx, float* __restrict__ val) {
    const int64_t r = blockIdx.x;
    uint64_t key = 0;
    for (int c = threadIdx.x; c < chunks; c += kArgmaxThreads) key = max_u64(key, part[r * chunks + c]);
    key = block_max(key);
    if (threadIdx.x == 0) {
        const int32_t i = key ? (int32_t)(uint32_t)key : -1;
        idx[r] = i;
        if (val) val[r] = i >= 0 ? y[r * ldy + i] : __builtin_nanf("");
    }
}

// Grid m: the n (key, value) pairs of row r of a fused product
// (launch_gemv_argmax, launch_dense_argmax), at keys / vals + r n, to the
// row's index and value.  Each thread loads its pairs kKvPer at a time, all
// in flight together, before comparing them.
constexpr int kKvThreads = 1024, kKvPer = 4;
__global__ __launch_bounds__(kKvThreads) void k_argmax_final_kv(const uint64_t* __restrict__ keys,
                                                                const float* __restrict__ vals, int n,
                                                                int32_t* __restrict__ idx, float* __restrict__ val) {
    const int64_t r = blockIdx.x;
    keys += r * n;
    vals += r * n;
    __shared__ uint64_t s_key[kKvThreads / 64];
    __shared__ float s_val[kKvThreads / 64];
    uint64_t key = 0;
    float v = 0.f;
    for (int c0 = 0; c0 < n; c0 += kKvThreads * kKvPer) {
        uint64_t kk[kKvPer];
        float vv[kKvPer];
#pragma unroll
        for (int j = 0; j < kKvPer; j++) {
            const int c = c0 + j * kKvThreads + (int)threadIdx.x;
            kk[j] = c < n ? keys[c] : 0;
            vv[j] = c < n ? vals[c] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < kKvPer; j++)
            if (kk[j] > key) {
                key = kk[j];
                v = vv[j];
            }
    }
    wave_max_kv(key, v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_key[wave] = key;
        s_val[wave] = v;
    }
    __syncthreads();
    if (wave == 0) {  // the 16 waves' pairs in lanes 0..15
        static_assert(kKvThreads / 64 == 16, "one row of 16 lanes");
        const int l = threadIdx.x & 15;
        key = s_key[l];
        v = s_val[l];
        row16_max_kv(key, v);
        if (threadIdx.x == 0) {
            const int32_t i = key ? (int32_t)(uint32_t)key : -1;
            idx[r] = i;
            if (val) val[r] = i >= 0 ? v : __builtin_nanf("");
        }
    }
}

}  // namespace

hipError_t launch_argmax_kv(const uint64_t* keys, const float* vals, int64_t m, int nparts, int32_t* idx, float* val,
                            hipStream_t s) {
    if (nparts <= 0 || m <= 0 || m > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_final_kv, dim3((unsigned)m), dim3(kKvThreads), 0, s, keys, vals, nparts, idx, val);
    return hipGetLastError();
}

size_t argmax_workspace_size(int64_t m, int64_t n) {
    const int64_t chunks = (n + kArgmaxChunk - 1) / kArgmaxChunk;
    return (size_t)(m * chunks) * sizeof(uint64_t);
}

hipError_t launch_argmax(const float* y, int64_t m, int64_t n, int64_t ldy, int32_t* idx, float* val, void* ws,
                         hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (n > INT32_MAX || m > 65535) return hipErrorInvalidValue;
    const int chunks = (int)((n + kArgmaxChunk - 1) / kArgmaxChunk);
    uint64_t* part = (uint64_t*)ws;
    hipLaunchKernelGGL(k_argmax_part, dim3((unsigned)chunks, (unsigned)m), dim3(kArgmaxThreads), 0, s, y, ldy, n,
                       part, chunks);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)m), dim3(kArgmaxThreads), 0, s, y, ldy, part, chunks, idx, val);
    return hipGetLastError();
}

}  // namespace iq
