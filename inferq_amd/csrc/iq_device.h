// iq_device.h -- device helpers shared by the gfx950 kernels.
//
// Numerics contract: every kernel here reproduces the reference CPU kernels'
// f32 arithmetic exactly (src/qgemm.rs:175-397): exact integer lane sums,
// one correctly rounded FMA per block per lane, and the fixed hsum trees.
// The library is compiled with -ffp-contract=off so that no a*b+c is fused
// unless written as __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_internal.h"

namespace iq {

// Internal activation layout.  Activations for K-quant weights are Q8K
// (256 values per block); for Q8_0 weights they are Q8_0 (32 per block).
// Either way the int8 values of each 256-value group are stored with their
// dwords transposed 8x8: dword (chunk c, lane k), which holds values
// 32c+4k .. 32c+4k+3, is stored at dword index 8k+c.  Lane k of an output
// row then reads its eight dwords (one per 32-value chunk) as 32 contiguous
// bytes.
__host__ __device__ constexpr int perm_dword(int c, int k) { return 8 * k + c; }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4), aligned(16)));
typedef float f32x4 __attribute__((ext_vector_type(4), aligned(16)));

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Bytes of q (each < 16) times s (< 8) byte by byte, as two 16-bit lanes:
// every product is below 128, so no lane carries into the next byte.
__device__ __forceinline__ uint32_t bytes_mul_small(uint32_t q, uint32_t s) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 a = __builtin_bit_cast(u16x2, q);
    const u16x2 b = {(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, a * b);
}

__device__ __forceinline__ int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Workgroup barrier ordering LDS only: global loads issued before it stay
// in flight (a full __syncthreads would also wait for them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// a * b + c for |a|, |b| < 2^23 (full-rate v_mad_i32_i24 instead of the
// quarter-rate 32-bit multiply); exact for every scale x lane-dot product here.
__device__ __forceinline__ int32_t imad24(int32_t a, int32_t b, int32_t c) { return __mul24(a, b) + c; }

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }

// Four bytes at a 2-byte aligned address, never reading outside [p, p+4).
__device__ __forceinline__ uint32_t ld32_a2(const uint8_t* p) {
    if (((uintptr_t)p & 3u) == 0) return ld32(p);
    return ld16(p) | (ld16(p + 2) << 16);
}

// Four bytes at p == 2 (mod 4) when the two bytes before p are readable:
// one aligned 8-byte load and a byte funnel shift.
__device__ __forceinline__ uint32_t ld32_m2(const uint8_t* p) {
    u32x2 v = *(const u32x2*)(p - 2);
    return __builtin_amdgcn_alignbyte(v.y, v.x, 2);
}

// Lane exchange inside groups of 8 lanes (lane ^ mask), mask in {1, 2, 4}.
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    int i = __builtin_bit_cast(int, v);
    int r;
    if constexpr (MASK == 1) {
        r = __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (MASK == 2) {
        r = __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else {
        r = __builtin_amdgcn_ds_swizzle(i, 0x101F);  // bitmode: and 0x1f, xor 4
    }
    return __builtin_bit_cast(float, r);
}

// Maximum of v over the 64 lanes, wave-uniform.  Four DPP steps inside each
// 16-lane row (lanes a step leaves out read 0, the identity), then
// row_bcast:15 and row_bcast:31 fold the rows into lane 63; every step
// issues as one v_max_u32_dpp (half the VALU ops of lane-half swaps).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true));   // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true));   // quad [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, true));  // row half mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, true));  // row mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false)); // row_bcast:15 -> rows 1, 3
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false)); // row_bcast:31 -> rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// hsum_f32_8 over the 8 lanes of a group: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)).
// Every lane of the group ends with the same value.
__device__ __forceinline__ float hsum8(float v) {
    v = v + xor_lane<4>(v);
    v = v + xor_lane<2>(v);
    v = v + xor_lane<1>(v);
    return v;
}

// hsum_f32_4 over lanes 0..3 of a group: (l0+l2) + (l1+l3), valid in lane 0.
__device__ __forceinline__ float hsum4(float v) {
    v = v + xor_lane<2>(v);
    v = v + xor_lane<1>(v);
    return v;
}

// Greedy-selection key of logit v at index i (sampling::argmax,
// src/sampling.rs:104-110): the order-preserving image of v in the high 32
// bits and the index in the low 32, so the largest key is the largest value
// and, among equal values, the largest index (the last of equal maxima);
// non-finite values map to 0, below every finite value's key; -0 ranks
// equal to +0.
__device__ __forceinline__ uint64_t argmax_key(float v, int64_t i) {
    if (!__builtin_isfinite(v)) return 0;
    if (v == 0.f) v = 0.f;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(uint32_t)i;
}

// One step of a (key, value) maximum across lanes `off` apart (keys are
// unique but for 0, whose value is never used).
__device__ __forceinline__ void max_kv_xor(uint64_t& key, float& val, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)key, off), hi = __shfl_xor((uint32_t)(key >> 32), off);
    const float ov = __shfl_xor(val, off);
    const uint64_t ok = ((uint64_t)hi << 32) | lo;
    if (ok > key) {
        key = ok;
        val = ov;
    }
}

// One step of the same maximum with the partner lane given by a DPP
// permutation within each row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ void max_kv_dpp(uint64_t& key, float& val) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)key, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(key >> 32), CTRL, 0xF, 0xF, false);
    const float ov = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, val), CTRL, 0xF, 0xF, false));
    const uint64_t ok = ((uint64_t)hi << 32) | lo;
    if (ok > key) {
        key = ok;
        val = ov;
    }
}

// The largest (key, value) pair of each row of 16 lanes, in every lane of
// the row: quad swaps, then the half-row and row mirrors.
__device__ __forceinline__ void row16_max_kv(uint64_t& key, float& val) {
    max_kv_dpp<0xB1>(key, val);   // quad_perm [1,0,3,2]
    max_kv_dpp<0x4E>(key, val);   // quad_perm [2,3,0,1]
    max_kv_dpp<0x141>(key, val);  // row_half_mirror
    max_kv_dpp<0x140>(key, val);  // row_mirror
}

// The largest (key, value) pair of the wave, in every lane.
__device__ __forceinline__ void wave_max_kv(uint64_t& key, float& val) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) max_kv_xor(key, val, off);
}

// Correctly rounded exp for f32 arguments: exp is evaluated in double and
// rounded once.  glibc's expf (what the reference's f32::exp calls) agrees
// with it except where glibc itself misrounds a near-midpoint case.
__device__ __forceinline__ float exp_f32(float x) { return (float)::exp((double)x); }

}  // namespace iq
