// iq_quant.h -- wave-level activation quantisers, bit-exact to candle
// 0.11's BlockQ8K::from_float and BlockQ8_0::from_float (called by the
// reference at src/gguf.rs:648-654).
//
// One wave quantises one 256-value group of one row.  Lane l holds values
// 4l..4l+3, i.e. chunk c = l/8 and lane-in-chunk k = l%8, and writes its
// packed dword to the lane-transposed position 8k+c of the internal layout.
#pragma once

#include "iq_device.h"

namespace iq {

__device__ __forceinline__ f32x4 load4(const float* p) {
    if (((uintptr_t)p & 15u) == 0) return *(const f32x4*)p;
    return f32x4{p[0], p[1], p[2], p[3]};
}

__device__ __forceinline__ int sat_i8(float v) {  // Rust `f32 as i8`
    if (v != v) return 0;
    v = v < -128.f ? -128.f : v;
    v = v > 127.f ? 127.f : v;
    return (int)v;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// Q8K of one 256-value group whose values 4l..4l+3 lane l already holds
// (all 64 lanes call it).  Returns lane l's four int8 packed in a dword,
// the block scale d (every lane), the sum of the lane's 16-value sub-block
// (lanes 4j..4j+3: bsums[j]) and of its 32-value sub-block (lanes
// 8c..8c+7).
struct Q8KLane {
    uint32_t packed;
    float d;
    int bsum16, sum32;
};
__device__ __forceinline__ Q8KLane quant_q8k_core(const f32x4 v) {
    // amax and the first index reaching it (the reference updates only on a
    // strictly larger |x| while scanning upwards): the lane's first largest
    // |x| (never NaN, never negative, so its bits order like the values),
    // the wave maximum of those, and the lowest lane holding it, whose
    // values come first in the block.
    float am = 0.f, mine = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float ax = fabsf(v[e]);
        if (am < ax) {
            am = ax;
            mine = v[e];
        }
    }
    const uint32_t amb = __builtin_bit_cast(uint32_t, am);
    const uint32_t top = wave_max_u32(amb);
    int q[4] = {0, 0, 0, 0};
    float dval = 0.f;
    if (top != 0u) {  // uniform
        const int first = (int)__builtin_ctzll(__ballot(amb == top));
        const float maxv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first));
        const float iscale = __fdiv_rn(-128.f, maxv);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float t = roundf(iscale * v[j]);
            q[j] = sat_i8(t < 127.f ? t : 127.f);
        }
        dval = __fdiv_rn(1.f, iscale);
    }
    Q8KLane r;
    r.packed = pack4(q[0], q[1], q[2], q[3]);
    int s = q[0] + q[1] + q[2] + q[3];
    s += __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    s += __builtin_amdgcn_mov_dpp(s, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    r.bsum16 = s;
    s += __builtin_amdgcn_ds_swizzle(s, 0x101F);  // lane ^ 4
    r.sum32 = s;
    r.d = dval;
    return r;
}

// quant_q8k_core into row `row`, group `g` of `a` and, when `ref` is not
// null, the reference 292-byte block.
__device__ __forceinline__ void quant_q8k_vals4(const f32x4 v, int64_t row, int g, const ActView& a, uint8_t* ref) {
    const int lane = threadIdx.x & 63;
    const Q8KLane r = quant_q8k_core(v);
    const int c = lane >> 3, k = lane & 7;
    uint32_t* qrow = (uint32_t*)(a.q + row * a.ldq + (int64_t)g * 256);
    qrow[perm_dword(c, k)] = r.packed;
    if (k == 0) a.s8[(row * a.ng + g) * 8 + c] = (int16_t)r.sum32;
    if (lane == 0) a.d[row * a.ldd + g] = r.d;
    if (ref) {
        if (lane == 0) *(float*)ref = r.d;
        *(uint32_t*)(ref + 4 + 4 * lane) = r.packed;
        if ((lane & 3) == 0) *(int16_t*)(ref + 260 + 2 * (lane >> 2)) = (int16_t)r.bsum16;
    }
}

// Q8K: xs points at the 256 values of group g of activation row `row`.
__device__ __forceinline__ void quant_q8k_wave(const float* xs, int64_t row, int g, const ActView& a, uint8_t* ref) {
    const int lane = threadIdx.x & 63;
    quant_q8k_vals4(load4(xs + 4 * lane), row, g, a, ref);
}

// The values lane l quantises in quant_q80_vals4: 4 values of block
// 8g + l/8 of a row of width k (zeros past the row's last block).
__device__ __forceinline__ f32x4 q80_vals4_load(const float* xrow, int64_t k, int g) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)g * 8 + (lane >> 3);
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (b < k / 32) v = load4(xrow + b * 32 + 4 * (lane & 7));
    return v;
}

// Q8_0 of the 8 blocks of group g of a row of width k (values from
// q80_vals4_load); `ref_row`, when not null, receives the row's reference
// 34-byte blocks.
__device__ __forceinline__ void quant_q80_vals4(const f32x4 v, int64_t k, int64_t row, int g, const ActView& a,
                                                uint8_t* ref_row) {
    const int lane = threadIdx.x & 63;
    const int c = lane >> 3, kk = lane & 7;
    const int64_t nb32 = k / 32;
    const int64_t b = (int64_t)g * 8 + c;  // this lane's Q8_0 block
    const bool valid = b < nb32;
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = fmaxf(am, __shfl_xor(am, 1));
    am = fmaxf(am, __shfl_xor(am, 2));
    am = fmaxf(am, __shfl_xor(am, 4));
    const float d = __fdiv_rn(am, 127.f);
    const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
    int q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) q[j] = sat_i8(roundf(v[j] * id));
    const uint32_t packed = pack4(q[0], q[1], q[2], q[3]);
    const uint16_t dh = f32_to_f16_rne(d);
    uint32_t* qrow = (uint32_t*)(a.q + row * a.ldq + (int64_t)g * 256);
    qrow[perm_dword(c, kk)] = packed;  // padding lanes store zeros
    if (valid && kk == 0) a.d[row * a.ldd + b] = f16_to_f32(dh);
    if (valid && ref_row) {
        uint8_t* blk = ref_row + b * 34;
        if (kk == 0) *(uint16_t*)blk = dh;
        *(uint16_t*)(blk + 2 + 4 * kk) = (uint16_t)(packed & 0xffffu);
        *(uint16_t*)(blk + 4 + 4 * kk) = (uint16_t)(packed >> 16);
    }
}

// Q8_0: the 8 blocks of group g of a row of width k (xrow = row start).
__device__ __forceinline__ void quant_q80_wave(const float* xrow, int64_t k, int64_t row, int g, const ActView& a,
                                               uint8_t* ref_row) {
    quant_q80_vals4(q80_vals4_load(xrow, k, g), k, row, g, a, ref_row);
}

}  // namespace iq

namespace iq {

// 64-lane DPP helpers for 8-lane groups (xor 1, xor 2 within a quad; xor 4
// by swizzle) on 32-bit payloads.
__device__ __forceinline__ int xor_lane_i(int v, int mask) {
    if (mask == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    if (mask == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    return __builtin_amdgcn_ds_swizzle(v, 0x101F);
}

// Load this lane's 32 values for quant8_q8k_vals (chunk l % 8 of the
// 256-value block at `src`; zeros when src is null).  Issued separately so
// callers can put these loads ahead of others in the memory queue.
__device__ __forceinline__ void q8k_chunk_load(const float* src, float (&v)[32]) {
    const int c = threadIdx.x & 7;
    if (src) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f32x4 t = load4(src + 32 * c + 4 * j);
            v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = 0.f;
    }
}

// One pass over up to 8 Q8K blocks: lane l quantises chunk c = l % 8 (32
// values, from q8k_chunk_load) of block l / 8 into row `row`, group `g` of
// `a` (live == false: an idle 8-lane group).  All 64 lanes must call it.
// Same arithmetic as quant_q8k_wave.
__device__ __forceinline__ void quant8_q8k_vals(const float (&v)[32], bool live, int64_t row, int g,
                                                const ActView& a, int32_t* corr = nullptr) {
    const int c = threadIdx.x & 7;
    // first index of the largest |x| in this chunk, then across the 8 chunks
    float am = 0.f, mv = 0.f;
    int idx = 1 << 20;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const float ax = fabsf(v[j]);
        if (am < ax) {
            am = ax;
            mv = v[j];
            idx = 32 * c + j;
        }
    }
#pragma unroll
    for (int mask = 1; mask <= 4; mask <<= 1) {
        const float am2 = __builtin_bit_cast(float, xor_lane_i(__builtin_bit_cast(int, am), mask));
        const float mv2 = __builtin_bit_cast(float, xor_lane_i(__builtin_bit_cast(int, mv), mask));
        const int idx2 = xor_lane_i(idx, mask);
        if (am2 > am || (am2 == am && idx2 < idx)) {
            am = am2;
            mv = mv2;
            idx = idx2;
        }
    }
    if (!live) return;
    int q[32];
    float dval = 0.f;
    if (am != 0.f) {  // uniform per 8-lane group
        const float iscale = __fdiv_rn(-128.f, mv);
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float t = roundf(iscale * v[j]);
            q[j] = sat_i8(t < 127.f ? t : 127.f);
        }
        dval = __fdiv_rn(1.f, iscale);
    } else {
#pragma unroll
        for (int j = 0; j < 32; j++) q[j] = 0;
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 32; j++) s += q[j];
    uint32_t* qrow = (uint32_t*)(a.q + row * a.ldq + (int64_t)g * 256);
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
        const uint32_t pk = pack4(q[4 * kk], q[4 * kk + 1], q[4 * kk + 2], q[4 * kk + 3]);
        qrow[perm_dword(c, kk)] = pk;
        // optional Q6_K offset term, laid out like q: -32 * (sum of the dword's four int8)
        if (corr) corr[(row * a.ng + g) * 64 + perm_dword(c, kk)] = sdot4(pk, 0xe0e0e0e0u, 0);
    }
    a.s8[(row * a.ng + g) * 8 + c] = (int16_t)s;
    if (c == 0) a.d[row * a.ldd + g] = dval;
}

__device__ __forceinline__ void quant8_q8k(const float* src, int64_t row, int g, const ActView& a) {
    float v[32];
    q8k_chunk_load(src, v);
    quant8_q8k_vals(v, src != nullptr, row, g, a);
}

// Load the 32 values of one Q8_0 block (zeros when src is null).
__device__ __forceinline__ void q80_block_load(const float* src, float (&v)[32]) {
    if (src) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f32x4 t = load4(src + 4 * j);
            v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = 0.f;
    }
}

// One pass over up to 64 Q8_0 blocks: lane l quantises one 32-value block
// (from q80_block_load) into block b of row `row` of `a`.  Same arithmetic
// as quant_q80_wave.
__device__ __forceinline__ void quant64_q80_vals(const float (&v)[32], bool live, int64_t row, int64_t b,
                                                 const ActView& a) {
    if (!live) return;
    float am = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) am = fmaxf(am, fabsf(v[j]));
    const float d = __fdiv_rn(am, 127.f);
    const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
    const int g = (int)(b / 8), c = (int)(b % 8);
    uint32_t* qrow = (uint32_t*)(a.q + row * a.ldq + (int64_t)g * 256);
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
        qrow[perm_dword(c, kk)] = pack4(sat_i8(roundf(v[4 * kk] * id)), sat_i8(roundf(v[4 * kk + 1] * id)),
                                        sat_i8(roundf(v[4 * kk + 2] * id)), sat_i8(roundf(v[4 * kk + 3] * id)));
    a.d[row * a.ldd + b] = f16_to_f32(f32_to_f16_rne(d));
}

__device__ __forceinline__ void quant64_q80(const float* src, int64_t row, int64_t b, const ActView& a) {
    float v[32];
    q80_block_load(src, v);
    quant64_q80_vals(v, src != nullptr, row, b, a);
}

}  // namespace iq

namespace iq {

// xor-exchange across lanes for any mask < 32 (DPP for 1 and 2, swizzle
// otherwise), 32-bit payload.
__device__ __forceinline__ int xor_lane_any(int v, int mask) {
    switch (mask) {
    case 1: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    case 2: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    case 4: return __builtin_amdgcn_ds_swizzle(v, 0x101F);
    case 8: return __builtin_amdgcn_ds_swizzle(v, 0x201F);
    default: return __builtin_amdgcn_ds_swizzle(v, 0x401F);
    }
}

// Q8K with VPL values per lane (8, 16 or 32): a block spans LPB = 256/VPL
// lanes and a wave covers 64/LPB blocks; lane l holds values
// VPL*(l % LPB) .. +VPL of its block.  q8k_vpl_load fetches them (zeros when
// src, the block start, is null); quant_q8k_vpl quantises the block into
// row `row`, group `g` of `a` (live == false: skip the stores).  Same
// arithmetic as quant_q8k_wave.
template <int VPL>
__device__ __forceinline__ void q8k_vpl_load(const float* src, float (&v)[VPL]) {
    constexpr int LPB = 256 / VPL;
    const int pl = (threadIdx.x & 63) % LPB;
    if (src) {
#pragma unroll
        for (int j = 0; j < VPL / 4; j++) {
            const f32x4 t = load4(src + VPL * pl + 4 * j);
            v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) v[j] = 0.f;
    }
}

template <int VPL>
__device__ __forceinline__ void quant_q8k_vpl(const float (&v)[VPL], bool live, int64_t row, int g,
                                              const ActView& a, int32_t* corr = nullptr) {
    constexpr int LPB = 256 / VPL, LPC = 32 / VPL > 0 ? 32 / VPL : 1;
    static_assert(VPL == 8 || VPL == 16 || VPL == 32, "VPL");
    const int pl = (threadIdx.x & 63) % LPB;
    float am = 0.f, mv = 0.f;
    int idx = 1 << 20;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const float ax = fabsf(v[j]);
        if (am < ax) {
            am = ax;
            mv = v[j];
            idx = VPL * pl + j;
        }
    }
#pragma unroll
    for (int mask = 1; mask < LPB; mask <<= 1) {
        const float am2 = __builtin_bit_cast(float, xor_lane_any(__builtin_bit_cast(int, am), mask));
        const float mv2 = __builtin_bit_cast(float, xor_lane_any(__builtin_bit_cast(int, mv), mask));
        const int idx2 = xor_lane_any(idx, mask);
        if (am2 > am || (am2 == am && idx2 < idx)) {
            am = am2;
            mv = mv2;
            idx = idx2;
        }
    }
    int q[VPL];
    float dval = 0.f;
    if (am != 0.f) {
        const float iscale = __fdiv_rn(-128.f, mv);
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const float t = roundf(iscale * v[j]);
            q[j] = sat_i8(t < 127.f ? t : 127.f);
        }
        dval = __fdiv_rn(1.f, iscale);
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) q[j] = 0;
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < VPL; j++) s += q[j];
#pragma unroll
    for (int mask = 1; mask < LPC; mask <<= 1) s += xor_lane_any(s, mask);
    if (!live) return;
    const int c = (VPL * pl) / 32, kk0 = ((VPL * pl) % 32) / 4;
    uint32_t* qrow = (uint32_t*)(a.q + row * a.ldq + (int64_t)g * 256);
#pragma unroll
    for (int t = 0; t < VPL / 4; t++) {
        const uint32_t pk = pack4(q[4 * t], q[4 * t + 1], q[4 * t + 2], q[4 * t + 3]);
        qrow[perm_dword(c, kk0 + t)] = pk;
        // optional Q6_K offset term, laid out like q: -32 * (sum of the dword's four int8)
        if (corr) corr[(row * a.ng + g) * 64 + perm_dword(c, kk0 + t)] = sdot4(pk, 0xe0e0e0e0u, 0);
    }
    if (pl % LPC == 0) a.s8[(row * a.ng + g) * 8 + c] = (int16_t)s;
    if (pl == 0) a.d[row * a.ldd + g] = dval;
}

}  // namespace iq
