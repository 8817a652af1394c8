// iq_gemv.hip -- y = x . W^T for many output rows and up to 8 input rows
// (decode and verify shapes: LM head, dense projections), in the reference's
// exact f32 order (src/qgemm.rs:175-397 via src/gguf.rs:608-690).
//
// Each wave owns groups of RPW consecutive weight rows.  A group is consumed
// in slices of 2048 weights (Q8_0: 1024) per row: the wave copies the slice
// bytes of its rows -- one contiguous span per row -- with 16-byte loads
// spread evenly over its 64 lanes, parks them in its own LDS region, and
// decodes from there with the same lane structure as iq_lanes.h (lane
// (slot, k) owns lane k of row `slot`).
//
// Two forms.  Tiles of several input rows take groups of 8 rows with two
// slices in flight per wave: while one is decoded, the loads of the next
// two are outstanding.  One-row tiles (k_gemv4) take groups of 4 rows:
// lanes 0-7 and 8-15 of a row's 16 form the chain steps of the first and
// the second half of the slice's units, and lanes 0-7 run the reference
// chain through both halves in order.  Half the LDS per wave and, on grids
// that fill the GPU, one slice in flight (Q6_K: 116 VGPRs) give four waves
// per SIMD instead of two, which hides the decode under the stream: the LM
// head [248320 x 2048] Q6_K 73.2 -> 67.8 us at steady clocks, [40960 x
// 2048] Q6_K 21.3 -> 16.2 us, [61440 x 2048] Q4_K 23.8 -> 17.3 us; on small
// grids the shorter items alone pay (Q8_0 [4096 x 2048] 7.25 -> 6.3 us).
//
// Every workgroup quantises the input rows itself (from_float, bit-exact to
// iq_quant.h) into LDS, after issuing its first weight loads, so a call is
// one launch and the quantisation hides under the first memory round trip.
//
// Weights are read with non-temporal loads: they stream through once, and
// keeping them out of the caches' retention lifts sustained HBM throughput.
//
// LDS rows are padded so that the rows of a wave start in different bank
// groups.  Q6_K blocks at 2 (mod 4) bytes are read as aligned dword pairs and
// funnel-shifted; the parity of every block in a slice is a compile-time
// constant because slices hold a multiple of 8 blocks.
#include <atomic>
#include <type_traits>

#include "iq_lanes.h"
#include "iq_quant.h"

namespace iq {

namespace {

template <int FMT>
struct GvFmt;
template <>
struct GvFmt<kQ4_K> {
    static constexpr int UB = 144;  // bytes per 256-value unit
    static constexpr int SU = 8;    // units per slice
    static constexpr int PAD = 32;
    static constexpr int DPU = 1;   // activation scales per unit
};
template <>
struct GvFmt<kQ6_K> {
    static constexpr int UB = 210, SU = 8, PAD = 16, DPU = 1;
};
template <>
struct GvFmt<kQ8_0> {
    static constexpr int UB = 272, SU = 4, PAD = 96, DPU = 8;  // unit = 8 blocks of 34 B
};

template <int FMT, int RPW = 8>
struct GvGeom {
    static constexpr int UB = GvFmt<FMT>::UB, SU = GvFmt<FMT>::SU, DPU = GvFmt<FMT>::DPU;
    static constexpr int SB = UB * SU;               // slice bytes per row
    static constexpr int RS = SB + GvFmt<FMT>::PAD;  // LDS row stride
    static constexpr int CPR = SB / 16;              // 16-byte chunks per row slice
    static constexpr int NL = (RPW * CPR + 63) / 64;   // chunks per lane per slice
    static constexpr int WAVE_LDS = RPW * RS;
    static_assert(SB % 16 == 0 && RS % 16 == 0, "slices must be 16-byte granular");
};

struct GemvArgs {
    const uint8_t* w;
    int64_t n, row_bytes;
    int nu;      // 256-value units per row
    int groups;  // ceil(n / 8)
    const float* x;  // f32 input rows [m][ldx]
    int64_t ldx;
    int m;
    float* y;
    int64_t ldy;
    int act_lds;  // bytes of the activation tile in LDS
    // fused greedy selection (one input row): wave w of workgroup b leaves
    // its rows' largest (argmax key, logit) at index 4 b + w
    uint64_t* amx_key = nullptr;
    float* amx_val = nullptr;
};

// Activation tile in LDS: q [MT][nu][256] (lane-transposed groups),
// d [MT][nu * DPU], s8 [MT][nu][8] (K-quants), corr [MT][nu][64] int32
// (Q6_K).  Every part starts 16-byte aligned.
template <int FMT, int MT>
__host__ __device__ constexpr int act_d_offset(int nu) { return MT * nu * 256; }
template <int FMT, int MT>
__host__ __device__ constexpr int act_s8_offset(int nu) {
    return act_d_offset<FMT, MT>(nu) + ((MT * nu * GvFmt<FMT>::DPU * 4 + 15) & ~15);
}
template <int FMT, int MT>
__host__ __device__ constexpr int act_corr_offset(int nu) {
    return act_s8_offset<FMT, MT>(nu) + (FMT == kQ8_0 ? 0 : MT * nu * 16);
}
template <int FMT, int MT>
__host__ __device__ constexpr int act_lds_bytes(int nu) {
    return act_corr_offset<FMT, MT>(nu) + (FMT == kQ6_K ? MT * nu * 256 : 0);
}

template <int FMT, int MT>
struct ActLds {
    const uint8_t* q;
    const float* d;
    const int16_t* s8;
    const uint8_t* corr;
    int nu;
    __device__ __forceinline__ ActLds(const uint8_t* base, int nu_) : nu(nu_) {
        q = base;
        d = (const float*)(base + act_d_offset<FMT, MT>(nu));
        s8 = (const int16_t*)(base + act_s8_offset<FMT, MT>(nu));
        corr = base + act_corr_offset<FMT, MT>(nu);
    }
    // Q6_K: -32 * (sum of the four int8 of dword (chunk c, lane k)), laid out
    // like q, so that the dot of (q6 - 32) is the dot of q6 started at it
    __device__ __forceinline__ void load_corr(int mi, int u, int k, int32_t (&cv)[8]) const {
        const uint8_t* p = corr + ((size_t)mi * nu + u) * 256 + 32 * k;
        const u32x4a16 a0 = *(const u32x4a16*)p, a1 = *(const u32x4a16*)(p + 16);
        cv[0] = (int32_t)a0.x; cv[1] = (int32_t)a0.y; cv[2] = (int32_t)a0.z; cv[3] = (int32_t)a0.w;
        cv[4] = (int32_t)a1.x; cv[5] = (int32_t)a1.y; cv[6] = (int32_t)a1.z; cv[7] = (int32_t)a1.w;
    }
    __device__ __forceinline__ void load_q(int mi, int u, int k, uint32_t (&av)[8]) const {
        const uint8_t* p = q + ((size_t)mi * nu + u) * 256 + 32 * k;
        const u32x4a16 a0 = *(const u32x4a16*)p, a1 = *(const u32x4a16*)(p + 16);
        av[0] = a0.x; av[1] = a0.y; av[2] = a0.z; av[3] = a0.w;
        av[4] = a1.x; av[5] = a1.y; av[6] = a1.z; av[7] = a1.w;
    }
};

// The activation tile as an ActView over LDS (rows 0..MT-1).
template <int FMT, int MT>
__device__ __forceinline__ ActView act_view_lds(uint8_t* lds, int nu) {
    ActView a;
    a.q = (int8_t*)lds;
    a.d = (float*)(lds + act_d_offset<FMT, MT>(nu));
    a.s8 = (int16_t*)(lds + act_s8_offset<FMT, MT>(nu));
    a.ldq = (int64_t)nu * 256;
    a.ldd = (int64_t)nu * GvFmt<FMT>::DPU;
    a.ng = nu;
    a.m = MT;
    return a;
}

// Input quantisation in passes of 8 groups of 256 values: in pass `ps`,
// lane l holds values 32 (l % 8) .. +31 of tile group t = 8 ps + l / 8 (row
// t / nu, group t % nu).  For Q8_0 these 32 values are exactly block
// 8 (t % nu) + l % 8 of the row, so both formats load the same way.
template <int MT>
__device__ __forceinline__ void quant_pass_load(const GemvArgs& p, int m0, int mc, int ps, float (&v)[32]) {
    const int lane = threadIdx.x & 63;
    const int t = 8 * ps + (lane >> 3);
    const int tt = min(t, MT * p.nu - 1);  // lanes past the tile re-read the last group
    const int mi = tt / p.nu, g = tt - mi * p.nu;
    const float* src = p.x + (int64_t)(m0 + min(mi, mc - 1)) * p.ldx + (int64_t)g * 256 + 32 * (lane & 7);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const f32x4 q = load4(src + 4 * j);
        v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
    }
}
template <int FMT, int MT>
__device__ __forceinline__ void quant_pass_store(const GemvArgs& p, const ActView& a, int32_t* corr, int ps,
                                                 const float (&v)[32]) {
    const int lane = threadIdx.x & 63;
    const int t = 8 * ps + (lane >> 3);
    const bool live = t < MT * p.nu;
    const int tt = min(t, MT * p.nu - 1);
    const int mi = tt / p.nu, g = tt - mi * p.nu;
    if constexpr (FMT == kQ8_0) quant64_q80_vals(v, live, mi, (int64_t)g * 8 + (lane & 7), a);
    else quant8_q8k_vals(v, live, mi, g, a, corr);
}

// ---- per-unit decode from LDS ------------------------------------------------

// Q6_K block at LDS address b; A2: b == 2 (mod 4).
template <bool A2>
__device__ __forceinline__ Q6Dec q6_decode_lds(const uint8_t* b, int k) {
    uint32_t ql[4], qh[2], sc[4];
    if constexpr (!A2) {
#pragma unroll
        for (int i = 0; i < 4; i++) ql[i] = *(const uint32_t*)(b + 32 * i + 4 * k);
#pragma unroll
        for (int j = 0; j < 2; j++) qh[j] = *(const uint32_t*)(b + 128 + 32 * j + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) sc[t] = *(const uint32_t*)(b + 192 + 4 * t);
    } else {
        const uint8_t* a = b - 2;  // 4-byte aligned
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x2 v = *(const u32x2*)(a + 32 * i + 4 * k);
            ql[i] = __builtin_amdgcn_alignbyte(v.y, v.x, 2);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const u32x2 v = *(const u32x2*)(a + 128 + 32 * j + 4 * k);
            qh[j] = __builtin_amdgcn_alignbyte(v.y, v.x, 2);
        }
        uint32_t s[5];
#pragma unroll
        for (int t = 0; t < 5; t++) s[t] = *(const uint32_t*)(a + 192 + 4 * t);
#pragma unroll
        for (int t = 0; t < 4; t++) sc[t] = __builtin_amdgcn_alignbyte(s[t + 1], s[t], 2);
    }
    Q6Dec r;
    r.xd = f16_to_f32(*(const uint16_t*)(b + 208));
    const int hk = k >= 4 ? 8 : 0;
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l = ql[2 * j + (i & 1)];
            const uint32_t lo = i < 2 ? (l & 0x0f0f0f0fu) : ((l >> 4) & 0x0f0f0f0fu);
            const uint32_t h = qh[j];
            const uint32_t hs = i == 0 ? h << 4 : i == 1 ? h << 2 : i == 2 ? h : h >> 2;
            r.v[4 * j + i] = (hs & 0x30303030u) | lo;  // bytes q6 in [0, 64); the -32 comes with the activation
            // scale 8j + 2i + (k >= 4): byte (2i & 3) + (k >= 4) of word 2j + i/2
            r.sc[4 * j + i] = __builtin_amdgcn_sbfe(sc[2 * j + (i >> 1)], 16 * (i & 1) + hk, 8);
        }
    }
    return r;
}

__device__ __forceinline__ Q4Dec q4_decode_lds(const uint8_t* b, int k) {
    Q4W w;
    w.hdr = *(const u32x4a16*)b;
#pragma unroll
    for (int j = 0; j < 4; j++) w.q[j] = *(const uint32_t*)(b + 16 + 32 * j + 4 * k);
    return q4_decode(w, k);
}

// Q8_0: the 8 blocks of a unit at LDS address b (16-byte aligned).
struct Q8Dec {
    uint32_t q[8];
    float d[8];
};
__device__ __forceinline__ Q8Dec q8_decode_lds(const uint8_t* b, int k) {
    Q8Dec r;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const uint8_t* blk = b + 34 * c;
        if (c % 2 == 0) {  // window at 2 (mod 4)
            const u32x2 v = *(const u32x2*)(blk + 4 * k);
            r.q[c] = __builtin_amdgcn_alignbyte(v.y, v.x, 2);
        } else {
            r.q[c] = *(const uint32_t*)(blk + 2 + 4 * k);
        }
        r.d[c] = f16_to_f32(*(const uint16_t*)blk);
    }
    return r;
}

// ---- the kernel ----------------------------------------------------------------

template <int FMT, int MT, int RPW, int NBUF, bool AMX = false>
__device__ __forceinline__ void gemv_run(const GemvArgs& p) {
    using G = GvGeom<FMT, RPW>;
    static_assert(RPW == 8 || (RPW == 4 && MT == 1), "four-row items: one input row");
    static_assert(!AMX || MT == 1, "fused greedy selection: one input row");
    constexpr int UPL = RPW == 8 ? G::SU : G::SU / 2;  // units of a slice per lane
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    // wave-uniform in a register the compiler knows is uniform, so that
    // every loop and branch on the item index is scalar
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int k = lane & 7, slot = RPW == 8 ? lane >> 3 : lane >> 4;
    const int half = RPW == 8 ? 0 : (lane >> 3) & 1;
    const int m0 = blockIdx.y * MT;
    const int mc = min(MT, p.m - m0);
    const int nsl = p.nu / G::SU;
    const int gstride = gridDim.x * 4;
    const int grp0 = blockIdx.x * 4 + wave;
    // this wave's items: (group grp0 + (i / nsl) * gstride, slice i % nsl)
    const int my_groups = grp0 < p.groups ? (p.groups - grp0 + gstride - 1) / gstride : 0;
    const int nitems = my_groups * nsl;

    // this lane's 16-byte chunks of a slice: global offset from the slice
    // base, and LDS offset (-1: no chunk)
    uint32_t goff[G::NL];
    int loff[G::NL];
#pragma unroll
    for (int i = 0; i < G::NL; i++) {
        int q = i * 64 + lane;
        const bool ok = q < RPW * G::CPR;
        if (!ok) q = RPW * G::CPR - 1;
        const int r = q / G::CPR, cq = q - r * G::CPR;
        goff[i] = (uint32_t)(r * p.row_bytes + cq * 16);
        loff[i] = ok ? r * G::RS + cq * 16 : -1;
    }
    // Loads are issued unconditionally (past the last item, the last item
    // again: its lines are still in L2), so that the same number of loads is
    // outstanding on every path and the compiler's vmcnt waits stay exact:
    // parking one buffer waits only for that buffer's loads.  A wave with
    // no items reads group 0, which always exists.
    const int gbase = nitems > 0 ? grp0 : 0;
    const int ilast = nitems > 0 ? nitems - 1 : 0;
    // fused greedy selection: the largest key among this lane's rows, and
    // its logit; every wave leaves its pair (key 0 when it had no rows)
    uint64_t bk = 0;
    float bv = 0.f;
    auto amx_finish = [&]() {
        if constexpr (AMX) {
            wave_max_kv(bk, bv);
            if (lane == 0) {
                const int64_t wi = (int64_t)blockIdx.x * 4 + wave;
                p.amx_key[wi] = bk;
                p.amx_val[wi] = bv;
            }
        }
    };
    auto issue = [&](u32x4a16 (&st)[G::NL], int it_) {
        const int it = min(it_, ilast);
        const int g8 = gbase + (it / nsl) * gstride, sl = it - (it / nsl) * nsl;
        const uint8_t* base = p.w + (int64_t)g8 * RPW * p.row_bytes + (int64_t)sl * G::SB;
        if ((int64_t)g8 * RPW + RPW <= p.n) {  // uniform: a full group
#pragma unroll
            for (int i = 0; i < G::NL; i++) st[i] = __builtin_nontemporal_load((const u32x4a16*)(base + goff[i]));
        } else {  // the last group: rows past the end re-read the last row
            const int last = (int)(p.n - (int64_t)g8 * RPW) - 1;
#pragma unroll
            for (int i = 0; i < G::NL; i++) {
                const int q = min(i * 64 + lane, RPW * G::CPR - 1);
                const int r = q / G::CPR, cq = q - r * G::CPR;
                st[i] = __builtin_nontemporal_load((const u32x4a16*)(base + (int64_t)min(r, last) * p.row_bytes + cq * 16));
            }
        }
    };
    auto park = [&](const u32x4a16 (&st)[G::NL], uint8_t* wl) {
#pragma unroll
        for (int i = 0; i < G::NL; i++)
            if (loff[i] >= 0) *(u32x4a16*)(wl + loff[i]) = st[i];
    };

    // Quantise the input tile into LDS.  Where every input load of a wave
    // fits in its registers, the first two weight slices go out between
    // loading and quantising, so the quantisation runs under their memory
    // latency; larger tiles quantise first, then issue (an input load issued
    // after the weight loads could only be waited for together with them).
    constexpr bool kEarly = MT == 1;
    const int npass = (MT * p.nu + 7) / 8;
    u32x4a16 stA[G::NL], stB[G::NL];
    const ActView al = act_view_lds<FMT, MT>(smem, p.nu);
    int32_t* corr = FMT == kQ6_K ? (int32_t*)(smem + act_corr_offset<FMT, MT>(p.nu)) : nullptr;
    if constexpr (kEarly && FMT != kQ8_0) {
        // K-quants at one input row (nu = 8 or 16 groups): wave w quantises
        // groups nu/4 * w .. +nu/4, nu values per lane
        auto early = [&](auto vpl) {
            constexpr int VPL = decltype(vpl)::value, LPB = 256 / VPL;
            const int gq = (VPL / 4) * wave + lane / LPB;
            float xv[VPL];
            q8k_vpl_load<VPL>(p.x + (int64_t)m0 * p.ldx + (int64_t)gq * 256, xv);
            issue(stA, 0);
            if constexpr (NBUF == 2) issue(stB, 1);
            quant_q8k_vpl<VPL>(xv, true, 0, gq, al, corr);
        };
        if (p.nu == 8) early(std::integral_constant<int, 8>{});
        else early(std::integral_constant<int, 16>{});
    } else if constexpr (kEarly) {
        float xv[32];
        if (wave < npass) quant_pass_load<MT>(p, m0, mc, wave, xv);
        issue(stA, 0);
        if constexpr (NBUF == 2) issue(stB, 1);
        if (wave < npass) quant_pass_store<FMT, MT>(p, al, corr, wave, xv);
    } else if (npass <= 8) {
        // up to two passes per wave: the wave's input loads, then the first
        // weight loads, then the quantisation, which runs under their
        // latency (the input loads, issued first, are waited for alone)
        float xv[2][32];
#pragma unroll
        for (int i = 0; i < 2; i++)
            if (wave + 4 * i < npass) quant_pass_load<MT>(p, m0, mc, wave + 4 * i, xv[i]);
        issue(stA, 0);
        if constexpr (NBUF == 2) issue(stB, 1);
#pragma unroll
        for (int i = 0; i < 2; i++)
            if (wave + 4 * i < npass) quant_pass_store<FMT, MT>(p, al, corr, wave + 4 * i, xv[i]);
    } else {
        for (int ps = wave; ps < npass; ps += 4) {
            float xv[32];
            quant_pass_load<MT>(p, m0, mc, ps, xv);
            quant_pass_store<FMT, MT>(p, al, corr, ps, xv);
        }
        issue(stA, 0);
        if constexpr (NBUF == 2) issue(stB, 1);
    }
    lds_barrier();
    if (nitems == 0) {  // uniform per wave; no barrier follows
        amx_finish();
        return;
    }

    const ActLds<FMT, MT> act(smem, p.nu);
    uint8_t* wl = smem + p.act_lds + wave * G::WAVE_LDS;
    const uint8_t* rowl = wl + slot * G::RS + half * UPL * G::UB;
    float acc[MT], accm[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = accm[i] = 0.f;

    auto compute = [&](int it) {
        const int g8 = grp0 + (it / nsl) * gstride, sl = it - (it / nsl) * nsl;
        // LDS operations of one wave complete in order: the stores that
        // parked this slice are visible to the loads below; keep the
        // compiler from moving the loads above them.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (RPW == 4) {
            // lanes of half h form the chain steps of units UPL h ..
            // UPL h + UPL - 1 of the slice (one step per unit, Q8_0 one per
            // 32-value block); half 0 then runs the chain through its own
            // steps and the other half's (lane ^ 8), in order
            constexpr int SPU = FMT == kQ8_0 ? 8 : 1, NS = UPL * SPU;
            int32_t is[NS], ms[NS];
            float dd[NS], dm[NS];
#pragma unroll
            for (int j = 0; j < UPL; j++) {
                const int ug = sl * G::SU + half * UPL + j;
                const uint8_t* b = rowl + j * G::UB;
                uint32_t av[8];
                act.load_q(0, ug, k, av);
                if constexpr (FMT == kQ8_0) {
                    const Q8Dec dec = q8_decode_lds(b, k);
                    const float* dp = act.d + (size_t)ug * 8;
                    const f32x4 d0 = *(const f32x4*)dp, d1 = *(const f32x4*)(dp + 4);
                    const float yd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        is[8 * j + c] = sdot4(dec.q[c], av[c], 0);
                        dd[8 * j + c] = dec.d[c] * yd[c];
                    }
                    continue;
                }
                const float yd = act.d[ug];
                if constexpr (FMT == kQ4_K) {
                    const Q4Dec dec = q4_decode_lds(b, k);
                    const uint32_t q8s = *(const uint32_t*)(act.s8 + (size_t)ug * 8 + 2 * (k & 3));
                    q4_dot(dec, av, yd, q8s, is[j], ms[j], dd[j], dm[j]);
                } else {
                    // unit 4h + j sits at 2j (mod 4)
                    const Q6Dec dec = (j & 1) ? q6_decode_lds<true>(b, k) : q6_decode_lds<false>(b, k);
                    int32_t cv[8];
                    act.load_corr(0, ug, k, cv);
                    int32_t isum = 0;
#pragma unroll
                    for (int c = 0; c < 8; c++) isum = imad24(dec.sc[c], sdot4(dec.v[c], av[c], cv[c]), isum);
                    is[j] = isum;
                    dd[j] = yd * dec.xd;
                }
            }
#pragma unroll
            for (int j = 0; j < NS; j++) {
                acc[0] = __builtin_fmaf(dd[j], (float)is[j], acc[0]);
                if constexpr (FMT == kQ4_K) accm[0] = __builtin_fmaf(dm[j], (float)ms[j], accm[0]);
            }
#pragma unroll
            for (int j = 0; j < NS; j++) {
                const int pi = __builtin_amdgcn_mov_dpp(is[j], 0x128, 0xF, 0xF, false);  // row_ror:8
                const float pd = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, dd[j]), 0x128, 0xF, 0xF, false));
                acc[0] = __builtin_fmaf(pd, (float)pi, acc[0]);
                if constexpr (FMT == kQ4_K) {
                    const int pm = __builtin_amdgcn_mov_dpp(ms[j], 0x128, 0xF, 0xF, false);
                    const float pdm = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, dm[j]), 0x128, 0xF, 0xF, false));
                    accm[0] = __builtin_fmaf(pdm, (float)pm, accm[0]);
                }
            }
        } else
#pragma unroll
        for (int u = 0; u < G::SU; u++) {
            const int ug = sl * G::SU + u;
            const uint8_t* b = rowl + u * G::UB;
            if constexpr (FMT == kQ4_K) {
                const Q4Dec dec = q4_decode_lds(b, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (MT == 1 || mi < mc) {
                        uint32_t av[8];
                        act.load_q(mi, ug, k, av);
                        const float yd = act.d[mi * p.nu + ug];
                        const uint32_t q8s = *(const uint32_t*)(act.s8 + ((size_t)mi * p.nu + ug) * 8 + 2 * (k & 3));
                        int32_t isum, msum;
                        float d, dmin;
                        q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
                        acc[mi] = __builtin_fmaf(d, (float)isum, acc[mi]);
                        accm[mi] = __builtin_fmaf(dmin, (float)msum, accm[mi]);
                    }
                }
            } else if constexpr (FMT == kQ6_K) {
                // block u of a slice sits at 2u (mod 4); u is a constant once unrolled
                const Q6Dec dec = (u & 1) ? q6_decode_lds<true>(b, k) : q6_decode_lds<false>(b, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (MT == 1 || mi < mc) {
                        uint32_t av[8];
                        int32_t cv[8];
                        act.load_q(mi, ug, k, av);
                        act.load_corr(mi, ug, k, cv);
                        const float yd = act.d[mi * p.nu + ug];
                        int32_t isum = 0;
#pragma unroll
                        for (int c = 0; c < 8; c++) isum = imad24(dec.sc[c], sdot4(dec.v[c], av[c], cv[c]), isum);
                        acc[mi] = __builtin_fmaf(yd * dec.xd, (float)isum, acc[mi]);
                    }
                }
            } else {
                const Q8Dec dec = q8_decode_lds(b, k);
#pragma unroll
                for (int mi = 0; mi < MT; mi++) {
                    if (MT == 1 || mi < mc) {
                        uint32_t av[8];
                        act.load_q(mi, ug, k, av);
                        const float* dp = act.d + ((size_t)mi * p.nu + ug) * 8;
                        const f32x4 d0 = *(const f32x4*)dp, d1 = *(const f32x4*)(dp + 4);
                        const float yd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                        for (int c = 0; c < 8; c++)
                            acc[mi] = __builtin_fmaf(dec.d[c] * yd[c], (float)sdot4(dec.q[c], av[c], 0), acc[mi]);
                    }
                }
            }
        }
        if (sl == nsl - 1) {
            const int64_t row = (int64_t)g8 * RPW + slot;
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                float v = hsum8(acc[mi]);
                if constexpr (FMT == kQ4_K) v = v + hsum4(accm[mi]);
                if (k == 0 && half == 0 && row < p.n && (MT == 1 || mi < mc)) {
                    p.y[(int64_t)(m0 + mi) * p.ldy + row] = v;
                    if constexpr (AMX) {
                        const uint64_t key = argmax_key(v, row);
                        if (key > bk) {
                            bk = key;
                            bv = v;
                        }
                    }
                }
                acc[mi] = accm[mi] = 0.f;
            }
        }
    };

    if constexpr (NBUF == 1) {
        // one slice in flight while the parked one is decoded.  With one
        // buffer every park waits for all outstanding loads anyway, so the
        // last item is not issued again (non-temporal lines are gone from
        // L2 by then: a re-issue read 5.7% more HBM bytes on the LM head)
        for (int it = 0; it < nitems; it++) {
            park(stA, wl);
            if (it + 1 < nitems) issue(stA, it + 1);
            compute(it);
        }
        amx_finish();
        return;
    }
    // Two items per trip with one exit at the bottom: every path through
    // the body parks and reissues both buffers in the same order (an odd
    // last item parks and reloads B once more, from L2, without using it).
    for (int it = 0; it < nitems; it += 2) {
        park(stA, wl);
        issue(stA, it + 2);
        compute(it);
        park(stB, wl);
        issue(stB, it + 3);
        if (it + 1 < nitems) compute(it + 1);
    }
    amx_finish();
}

template <int FMT, int MT>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs p) {
    gemv_run<FMT, MT, 8, 2>(p);
}
// Four-row items.  NBUF = 1 (one slice in flight): four workgroups of four
// waves per CU, at most 128 VGPRs, for grids that fill the GPU; NBUF = 2
// (two slices in flight, up to 144 VGPRs) for grids of under two
// workgroups per CU, whose waves have nothing to overlap with but their own
// next slice (Q8_0 [4096 x 2048] 6.9 -> 6.3 us, [4096 x 4096] 9.8 -> 8.2 us;
// [16384 x 2048] 11.3 against 13.0 us the other way round).
// AMX: greedy selection fused (GemvArgs::amx_key).
template <int FMT, int NBUF, bool AMX = false>
__global__ __launch_bounds__(256, NBUF == 1 ? 4 : 3) void k_gemv4(GemvArgs p) {
    gemv_run<FMT, 1, 4, NBUF, AMX>(p);
}

struct DevLimits {
    int cus = 0, lds_block = 0, lds_cu = 0;
};
DevLimits g_limits[64];

const DevLimits& limits() {
    static const DevLimits fallback{256, 64 * 1024, 64 * 1024};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fallback;
    DevLimits& L = g_limits[dev];
    if (L.cus == 0) {
        int v = 0;
        L.lds_block = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0
                          ? v : 64 * 1024;
        L.lds_cu = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess &&
                           v > 0 ? v : L.lds_block;
        L.cus = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v : 256;
    }
    return L;
}

template <int FMT, int MT, int RPW, int NBUF, bool AMX = false>
const void* kfn() {
    if constexpr (RPW == 4) return (const void*)k_gemv4<FMT, NBUF, AMX>;
    else return (const void*)k_gemv<FMT, MT>;
}
// Workgroups per CU the kernel's registers allow at `lds` bytes of LDS,
// queried once per LDS size (0: unknown).
template <int FMT, int MT, int RPW, int NBUF, bool AMX = false>
int occupancy(size_t lds) {
    static std::atomic<long long> cache[8];  // (lds << 8) | blocks; 0 = empty
    for (auto& c : cache) {
        const long long v = c.load(std::memory_order_relaxed);
        if (v == 0) break;
        if ((size_t)(v >> 8) == lds) return (int)(v & 0xff);
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn<FMT, MT, RPW, NBUF, AMX>(), 256, lds) != hipSuccess) {
        (void)hipGetLastError();  // clear this query's own error
        return 0;
    }
    const long long v = ((long long)lds << 8) | (occ & 0xff);
    for (auto& c : cache) {
        long long z = 0;
        if (c.compare_exchange_strong(z, v) || z == v) break;
    }
    return occ;
}

template <int FMT, int MT, int RPW = 8, int NBUF = 2, bool AMX = false>
hipError_t launch_t(GemvArgs args, hipStream_t s, int* nparts = nullptr) {
    using G = GvGeom<FMT, RPW>;
    args.act_lds = act_lds_bytes<FMT, MT>(args.nu);
    args.groups = (int)((args.n + RPW - 1) / RPW);
    const size_t lds = (size_t)args.act_lds + 4 * G::WAVE_LDS;
    const DevLimits& L = limits();
    if (lds > (size_t)L.lds_block) return hipErrorNotSupported;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(kfn<FMT, MT, RPW, NBUF, AMX>(), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
    }
    int per_cu = (int)(L.lds_cu / lds);
    const int occ = occupancy<FMT, MT, RPW, NBUF, AMX>(lds);
    if (occ > 0 && occ < per_cu) per_cu = occ;
    const int64_t wgs = ((int64_t)args.groups + 3) / 4;
    const int64_t cap = (int64_t)L.cus * (per_cu < 1 ? 1 : per_cu);
    dim3 grid((unsigned)(wgs < cap ? wgs : cap), (unsigned)((args.m + MT - 1) / MT));
    if (nparts) *nparts = (int)grid.x * 4;
    if constexpr (RPW == 4) hipLaunchKernelGGL((k_gemv4<FMT, NBUF, AMX>), grid, dim3(256), lds, s, args);
    else hipLaunchKernelGGL((k_gemv<FMT, MT>), grid, dim3(256), lds, s, args);
    return hipGetLastError();
}

// One input row on four-row items: one slice in flight where the grid fills
// the GPU twice over, two otherwise.
template <int FMT, bool AMX>
hipError_t launch_one_row(const GemvArgs& args, hipStream_t s, int* nparts) {
    const int64_t wgs = ((args.n + 3) / 4 + 3) / 4 * args.m;  // four-row items, one-row tiles
    if (wgs < 2 * (int64_t)limits().cus) return launch_t<FMT, 1, 4, 2, AMX>(args, s, nparts);
    return launch_t<FMT, 1, 4, 1, AMX>(args, s, nparts);
}

// Input rows per tile: the fewest tiles that still give every SIMD a few
// waves.  A large matrix (LM head) takes all rows in one tile and streams
// its weights once; a small one splits the rows over tiles, so that more
// waves share the per-row work (the extra weight reads hit L2).
template <int FMT>
hipError_t launch_fmt(const GemvArgs& args, hipStream_t s) {
    const int m = args.m;
    int mt = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const int mt_min = args.nu <= 16 ? 1 : 2;  // one-row tiles quantise at most 16 groups
    while (mt > mt_min && (int64_t)args.groups * ((m + mt - 1) / mt) < 2048) mt /= 2;
    switch (mt) {
    case 1: return launch_one_row<FMT, false>(args, s, nullptr);
    case 2: return launch_t<FMT, 2>(args, s);
    case 4: return launch_t<FMT, 4>(args, s);
    default: return launch_t<FMT, 8>(args, s);
    }
}

// One input row, K-quant weights of 8 or 16 blocks per row: y = x . W^T
// with the row's K split over the 4 waves of a workgroup (8 weight rows per
// workgroup), as in the one-token MoE kernels.  Each wave issues its blocks'
// weight burst, quantises its x blocks into LDS under it and forms the
// exact per-block lane integers; wave 0 then advances the reference's
// in-order FMA chains over all blocks and reduces them with the hsum trees.
// A mid-size matrix at one row is latency-bound, and a quarter of the
// decode per wave shortens its critical path.
template <int FMT, int NG>
__global__ __launch_bounds__(256) void k_gemv1_sk(const uint8_t* __restrict__ w, int64_t n, int64_t row_bytes,
                                                  const float* __restrict__ x, float* __restrict__ y) {
    constexpr int NW = 4, NB = NG / NW, VPL = NB * 4;  // blocks and x values per lane per wave
    static_assert(NG % NW == 0 && (VPL == 8 || VPL == 16), "shape");
    __shared__ __align__(16) int8_t s_q[NG * 256];
    __shared__ __align__(16) float s_d[NG * 8];
    __shared__ __align__(16) int16_t s_s8[NG * 8];
    __shared__ int s_isum[8][8][NG];  // [row][lane k][block]
    __shared__ int s_msum[8][4][NG];
    __shared__ float s_dd[8][NG], s_dm[8][NG];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int LPB = 256 / VPL;
    const int g0 = wave * NB;
    const int gx = g0 + lane / LPB;  // x block this lane quantises
    float xv[VPL];
    q8k_vpl_load<VPL>(x + (int64_t)gx * 256, xv);
    const int64_t i = (int64_t)blockIdx.x * 8 + slot;
    const int64_t ic = i < n ? i : n - 1;
    const uint8_t* wrow[1] = {w + ic * row_bytes + (int64_t)g0 * WT<FMT>::kBlockBytes};
    typename WT<FMT>::T wb[1][NB];
    lanes_load_exact<FMT, 1, NB>(wrow, k, wb);
    ActView a;
    a.ng = NG;
    a.ldq = NG * 256;
    a.ldd = NG * 8;
    a.m = 1;
    a.q = s_q;
    a.d = s_d;
    a.s8 = s_s8;
    quant_q8k_vpl<VPL>(xv, true, 0, gx, a);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int g = g0 + b;
        uint32_t av[8];
        load_act(a, 0, g, k, av);
        const float yd = a.d[g];
        if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
            Q4Dec dec;
            if constexpr (FMT == kQ4_K) dec = q4_decode(wb[0][b], k);
            else dec = q5_decode(wb[0][b], k);
            const uint32_t q8s = *(const uint32_t*)(a.s8 + g * 8 + 2 * (k & 3));
            int32_t isum, msum;
            float d, dmin;
            q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
            s_isum[slot][k][g] = isum;
            if constexpr (FMT == kQ5_K) {
                // the Q5_K mins: one integer per (row, block), one f32 scalar per row
                const int32_t mtot = isum_quad(msum);
                if (k == 0) s_msum[slot][0][g] = mtot;
            } else if (k < 4) {
                s_msum[slot][k][g] = msum;
            }
            if (k == 0) {
                s_dd[slot][g] = d;
                s_dm[slot][g] = dmin;
            }
        } else {
            const Q6Dec dec = q6_decode(wb[0][b], k);
            int32_t isum;
            float d;
            q6_dot(dec, av, yd, isum, d);
            s_isum[slot][k][g] = isum;
            if (k == 0) s_dd[slot][g] = d;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    float acc = 0.f, accm = 0.f;
#pragma unroll
    for (int g = 0; g < NG; g++) {
        acc = __builtin_fmaf(s_dd[slot][g], (float)s_isum[slot][k][g], acc);
        if constexpr (FMT == kQ4_K) accm = __builtin_fmaf(s_dm[slot][g], (float)s_msum[slot][k & 3][g], accm);
        if constexpr (FMT == kQ5_K) accm = accm + s_dm[slot][g] * (float)s_msum[slot][0][g];
    }
    float v = hsum8(acc);
    if constexpr (FMT == kQ4_K) v = v + hsum4(accm);
    if constexpr (FMT == kQ5_K) v = v + accm;
    if (k == 0 && i < n) y[i] = v;
}

// The same split for a tile of MT input rows: each wave quantises its x
// blocks of every row into LDS and forms the exact per-block integers of its
// blocks for every row, sharing one decode of its weights; the in-order
// chains of row r then run on wave r % 4.  Each row's result is the one-row
// kernel's.  Launched at two rows, where it takes q/gate [8192 x 2048] from
// 10.7 to 8.4 us and k/v [512 x 2048] from 7.1 to 4.9 us; at 3-8 rows the
// row-tiled k_gemv is faster (the per-row LDS traffic and chains grow with
// the rows while the weight bytes do not).
template <int FMT, int NG, int MT>
__global__ __launch_bounds__(256) void k_gemv_sk(const uint8_t* __restrict__ w, int64_t n, int64_t row_bytes,
                                                 const float* __restrict__ x, int64_t ldx, int m, float* __restrict__ y,
                                                 int64_t ldy) {
    constexpr int NW = 4, NB = NG / NW, VPL = NB * 4;  // blocks and x values per lane per wave
    static_assert(NG % NW == 0 && (VPL == 8 || VPL == 16), "shape");
    __shared__ __align__(16) int8_t s_q[MT * NG * 256];
    __shared__ __align__(16) float s_d[MT * NG * 8];
    __shared__ __align__(16) int16_t s_s8[MT * NG * 8];
    __shared__ int s_isum[MT][8][8][NG];  // [input row][weight row][lane k][block]
    __shared__ int s_msum[MT][8][4][NG];
    __shared__ float s_dd[MT][8][NG], s_dm[MT][8][NG];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = (int)blockIdx.y * MT, mc = min(MT, m - m0);
    constexpr int LPB = 256 / VPL;
    const int g0 = wave * NB;
    const int gx = g0 + lane / LPB;  // x block this lane quantises
    float xv[MT][VPL];
#pragma unroll
    for (int r = 0; r < MT; r++)
        q8k_vpl_load<VPL>(r < mc ? x + (int64_t)(m0 + r) * ldx + (int64_t)gx * 256 : nullptr, xv[r]);
    const int64_t i = (int64_t)blockIdx.x * 8 + slot;
    const int64_t ic = i < n ? i : n - 1;
    const uint8_t* wrow[1] = {w + ic * row_bytes + (int64_t)g0 * WT<FMT>::kBlockBytes};
    typename WT<FMT>::T wb[1][NB];
    lanes_load_exact<FMT, 1, NB>(wrow, k, wb);
    ActView a;
    a.ng = NG;
    a.ldq = NG * 256;
    a.ldd = NG * 8;
    a.m = MT;
    a.q = s_q;
    a.d = s_d;
    a.s8 = s_s8;
#pragma unroll
    for (int r = 0; r < MT; r++) quant_q8k_vpl<VPL>(xv[r], r < mc, r, gx, a);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int g = g0 + b;
        if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
            Q4Dec dec;
            if constexpr (FMT == kQ4_K) dec = q4_decode(wb[0][b], k);
            else dec = q5_decode(wb[0][b], k);
#pragma unroll
            for (int r = 0; r < MT; r++) {
                if (r < mc) {  // uniform
                    uint32_t av[8];
                    load_act(a, r, g, k, av);
                    const float yd = a.d[r * a.ldd + g];
                    const uint32_t q8s = *(const uint32_t*)(a.s8 + (r * NG + g) * 8 + 2 * (k & 3));
                    int32_t isum, msum;
                    float d, dmin;
                    q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
                    s_isum[r][slot][k][g] = isum;
                    if constexpr (FMT == kQ5_K) {
                        const int32_t mtot = isum_quad(msum);  // one f32 mins scalar per row
                        if (k == 0) s_msum[r][slot][0][g] = mtot;
                    } else if (k < 4) {
                        s_msum[r][slot][k][g] = msum;
                    }
                    if (k == 0) {
                        s_dd[r][slot][g] = d;
                        s_dm[r][slot][g] = dmin;
                    }
                }
            }
        } else {
            const Q6Dec dec = q6_decode(wb[0][b], k);
#pragma unroll
            for (int r = 0; r < MT; r++) {
                if (r < mc) {  // uniform
                    uint32_t av[8];
                    load_act(a, r, g, k, av);
                    const float yd = a.d[r * a.ldd + g];
                    int32_t isum;
                    float d;
                    q6_dot(dec, av, yd, isum, d);
                    s_isum[r][slot][k][g] = isum;
                    if (k == 0) s_dd[r][slot][g] = d;
                }
            }
        }
    }
    __syncthreads();
    for (int r = wave; r < mc; r += NW) {
        float acc = 0.f, accm = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            acc = __builtin_fmaf(s_dd[r][slot][g], (float)s_isum[r][slot][k][g], acc);
            if constexpr (FMT == kQ4_K) accm = __builtin_fmaf(s_dm[r][slot][g], (float)s_msum[r][slot][k & 3][g], accm);
            if constexpr (FMT == kQ5_K) accm = accm + s_dm[r][slot][g] * (float)s_msum[r][slot][0][g];
        }
        float v = hsum8(acc);
        if constexpr (FMT == kQ4_K) v = v + hsum4(accm);
        if constexpr (FMT == kQ5_K) v = v + accm;
        if (k == 0 && i < n) y[(int64_t)(m0 + r) * ldy + i] = v;
    }
}

template <int FMT>
hipError_t launch_sk2(const WeightView& w, const float* x, int64_t ldx, float* y, int64_t ldy, hipStream_t s) {
    const dim3 grid((unsigned)((w.rows + 7) / 8), 1);
    if (w.cols == 2048)
        hipLaunchKernelGGL((k_gemv_sk<FMT, 8, 2>), grid, dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, ldx, 2, y, ldy);
    else
        hipLaunchKernelGGL((k_gemv_sk<FMT, 16, 2>), grid, dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, ldx, 2, y, ldy);
    return hipGetLastError();
}

// m single-row tiles of the split kernel, one per grid row.
template <int FMT>
hipError_t launch_sk_rows(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                          hipStream_t s) {
    const dim3 grid((unsigned)((w.rows + 7) / 8), (unsigned)m);
    if (w.cols == 2048)
        hipLaunchKernelGGL((k_gemv_sk<FMT, 8, 1>), grid, dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, ldx, (int)m, y,
                           ldy);
    else
        hipLaunchKernelGGL((k_gemv_sk<FMT, 16, 1>), grid, dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, ldx, (int)m,
                           y, ldy);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_sk(const WeightView& w, const float* x, float* y, hipStream_t s) {
    const unsigned groups = (unsigned)((w.rows + 7) / 8);
    if (w.cols == 2048) hipLaunchKernelGGL((k_gemv1_sk<FMT, 8>), dim3(groups), dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, y);
    else hipLaunchKernelGGL((k_gemv1_sk<FMT, 16>), dim3(groups), dim3(256), 0, s, w.w, w.rows, w.row_bytes, x, y);
    return hipGetLastError();
}

// The split kernels take K-quant matrices of width 2048 or 4096 up to
// kSkMaxBytes (larger ones stream better through k_gemv); Q6_K rows of 8 or
// 16 blocks keep the burst's dword alignment.
constexpr int64_t kSkMaxBytes = (int64_t)64 << 20;
bool sk_supported(const WeightView& w) {
    if (w.cols != 2048 && w.cols != 4096) return false;
    // Q5_K has no LDS-staged kernel to stream better, so any size
    if (w.dtype == kQ5_K) return ((uintptr_t)w.w & 15) == 0;
    if (w.rows * w.row_bytes > kSkMaxBytes) return false;
    if (w.dtype == kQ4_K) return ((uintptr_t)w.w & 15) == 0;
    if (w.dtype == kQ6_K) return ((uintptr_t)w.w & 3) == 0;
    return false;
}

}  // namespace

// Up to 8 rows every matrix the MFMA kernel (iq_dense_mfma.hip) leaves
// takes this kernel.  Past 8 rows it runs one tile of 8 rows per grid row,
// and each tile redoes the per-row lane work while its weight reads hit L2:
// that wins (by 2x to 8x) on matrices up to a few MiB; wider calls on other
// matrices go to the lane kernel (iq_lanes.hip).
bool gemv_supported(const WeightView& w, int64_t m) {
    if (m < 1 || m >= kPrefillMinRows || w.rows < 1) return false;
    // Q5_K: the split kernels only, one to eight rows (the reference keeps
    // Q5_K on its per-row path, src/gguf.rs:588-593; the lane order is the
    // same)
    if (w.dtype == kQ5_K) return m <= 8 && w.rows <= (int64_t)1 << 31 && sk_supported(w);
    const int64_t bytes = w.rows * w.row_bytes;
    if (m > 8 && bytes > (m <= 16 ? (int64_t)64 << 20 : (int64_t)8 << 20)) return false;
    const int64_t nu = w.cols / 256;
    if (w.cols % 256 != 0 || w.rows > (int64_t)1 << 31) return false;
    if (m == 1 && nu > 16) return false;  // one quantisation batch per wave at one row
    switch (w.dtype) {
    case kQ4_K: return nu % GvFmt<kQ4_K>::SU == 0;
    case kQ6_K: return nu % GvFmt<kQ6_K>::SU == 0;
    case kQ8_0: return nu % GvFmt<kQ8_0>::SU == 0;
    default: return false;
    }
}

hipError_t launch_gemv(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                       hipStream_t s) {
    if (!gemv_supported(w, m)) return hipErrorNotSupported;
    if (m == 1 && sk_supported(w))
        return w.dtype == kQ4_K ? launch_sk<kQ4_K>(w, x, y, s)
                                : w.dtype == kQ5_K ? launch_sk<kQ5_K>(w, x, y, s) : launch_sk<kQ6_K>(w, x, y, s);
    if (m == 2 && sk_supported(w))
        return w.dtype == kQ4_K ? launch_sk2<kQ4_K>(w, x, ldx, y, ldy, s)
                                : w.dtype == kQ5_K ? launch_sk2<kQ5_K>(w, x, ldx, y, ldy, s)
                                                   : launch_sk2<kQ6_K>(w, x, ldx, y, ldy, s);
    if (w.dtype == kQ5_K) return launch_sk_rows<kQ5_K>(w, x, ldx, m, y, ldy, s);  // 3..8 rows
    // Three to eight rows as single-row tiles of the split kernel while the
    // tiles total at most 4096 workgroups at width 2048 (768 at width 4096,
    // whose tiles quantise and chain twice the blocks); past that the
    // row-tiled kernel, which decodes each weight once per tile of rows,
    // is faster.  k/v [512 x 2048] at 4 rows 6.1 -> 3.8 us, at 8 rows 6.1 ->
    // 4.1 us; q/gate [8192 x 2048] at 4 rows 13.4 -> 11.7 us (at 5 rows 13.1
    // against 15.6); [4096 x 2048] at 6 rows 11.3 -> 9.6 us; o [2048 x 4096]
    // at 3 rows 7.7 -> 7.1 us.
    const int64_t sk_tiles = (w.rows + 7) / 8 * m;
    if (m <= 8 && sk_supported(w) && sk_tiles <= (w.cols == 2048 ? 4096 : 768))
        return w.dtype == kQ4_K ? launch_sk_rows<kQ4_K>(w, x, ldx, m, y, ldy, s)
                                : launch_sk_rows<kQ6_K>(w, x, ldx, m, y, ldy, s);
    GemvArgs args;
    args.w = w.w;
    args.n = w.rows;
    args.row_bytes = w.row_bytes;
    args.nu = (int)(w.cols / 256);
    args.groups = (int)((w.rows + 7) / 8);
    args.x = x;
    args.ldx = ldx;
    args.m = (int)m;
    args.y = y;
    args.ldy = ldy;
    args.act_lds = 0;
    switch (w.dtype) {
    case kQ4_K: return launch_fmt<kQ4_K>(args, s);
    case kQ6_K: return launch_fmt<kQ6_K>(args, s);
    case kQ8_0: return launch_fmt<kQ8_0>(args, s);
    default: return hipErrorInvalidValue;
    }
}

// The dispatch runs one-row products on the four-row-item kernel wherever
// the split kernel does not take them (launch_gemv above): the LM head
// (417 MB, past kSkMaxBytes), Q8_0 matrices, other widths.
bool gemv_argmax_supported(const WeightView& w) { return gemv_supported(w, 1) && !sk_supported(w); }

// Waves of the four-row-item grid at most: four per workgroup, one
// workgroup per four items of four rows.
int64_t gemv_argmax_parts(const WeightView& w) { return ((w.rows + 3) / 4 + 3) / 4 * 4; }

hipError_t launch_gemv_argmax(const WeightView& w, const float* x, float* y, uint64_t* keys, float* vals, int* nparts,
                              hipStream_t s) {
    if (!gemv_argmax_supported(w) || !keys || !vals || !nparts) return hipErrorNotSupported;
    GemvArgs args;
    args.w = w.w;
    args.n = w.rows;
    args.row_bytes = w.row_bytes;
    args.nu = (int)(w.cols / 256);
    args.x = x;
    args.ldx = w.cols;
    args.m = 1;
    args.y = y;
    args.ldy = w.rows;
    args.act_lds = 0;
    args.amx_key = keys;
    args.amx_val = vals;
    switch (w.dtype) {
    case kQ4_K: return launch_one_row<kQ4_K, true>(args, s, nparts);
    case kQ6_K: return launch_one_row<kQ6_K, true>(args, s, nparts);
    case kQ8_0: return launch_one_row<kQ8_0, true>(args, s, nparts);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace iq
