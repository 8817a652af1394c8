// iq_moe_verify.hip -- the MoE sublayer for 2..16 tokens (the speculative
// verify pass), grouped by expert (routed_grouped_by_expert,
// src/qwen/quantized_moe.rs:336-460) with the single-token kernels'
// techniques: hidden split over the waves of a workgroup with an in-order
// FMA chain, weight bursts issued before the activation work, activations
// quantised where they are consumed, no device-scope fences.
//
// Four launches per call:
//   k_moev_prep     workgroup 0 (one wave per token) routes every token and
//                   computes its shared-expert gate, then groups the (token,
//                   route) pairs by expert, ascending; the other workgroups
//                   quantise x.
//   k_moev_gate_up  workgroup (8 intermediate rows, expert group): gate and
//                   up rows of that expert against the group's tokens,
//                   SwiGLU into act.
//   k_moev_down     workgroup (8 hidden rows, 4 groups): one wave per group
//                   quantises the group's SwiGLU rows into LDS while its
//                   down rows load, then writes the expert outputs to vals.
//   k_moev_combine  per (token, hidden row): routes in order (multiply, then
//                   add), then shared * gate.
// Every product follows the same per-lane order as the single-token path,
// so a token's output is bitwise what a one-token call gives.
#include "iq_lanes.h"
#include "iq_moe.h"
#include "iq_quant.h"
#include "iq_route.h"

namespace iq {

namespace {

constexpr int kVerifyMaxTokens = 16;
constexpr int kPrepThreads = 1024;  // one routing wave per token

// ------------------------------------------------------------------ prep
template <int AFMT>
__global__ __launch_bounds__(kPrepThreads) void k_moev_prep(MoeParams p) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (blockIdx.x > 0) {  // x quantisation: one wave per (row, 256-value group)
        const int64_t wid = (int64_t)(blockIdx.x - 1) * (kPrepThreads / 64) + wave;
        const int ng = p.xq.ng;
        if (wid >= (int64_t)p.M * ng) return;
        const int64_t row = wid / ng;
        const int g = (int)(wid % ng);
        if constexpr (AFMT == kQ8_0) quant_q80_wave(p.x + row * p.H, p.H, row, g, p.xq, nullptr);
        else quant_q8k_wave(p.x + row * p.H + (int64_t)g * 256, row, g, p.xq, nullptr);
        return;
    }
    __shared__ __align__(16) float s_ev[kVerifyMaxTokens][kMoeMaxExperts];
    __shared__ int s_exp[kVerifyMaxTokens * kMoeMaxTopK];
    __shared__ int s_cnt[kMoeMaxExperts], s_start[kMoeMaxExperts];
    __shared__ int s_scan[kPrepThreads / 64];
    const int E = (int)p.E, K = (int)p.K, M = p.M;
    // wave t < M routes token t; the shared-expert gate of token t runs on
    // wave M + t when there are waves to spare, else after the routing
    const bool split_gate = 2 * M <= kPrepThreads / 64;
    if (wave < M) {
        const int t = wave;
        int sel[kMoeMaxTopK];
        float lv[kRoutePer], w[kMoeMaxTopK];
        route_topk<kMoeMaxTopK>(p.logits + (int64_t)t * E, E, K, sel, lv);
        route_weights<kMoeMaxTopK>(lv, E, K, sel, p.normalize, s_ev[t], w);
        if (lane == 0) {
            for (int s = 0; s < K; s++) {
                p.experts[t * K + s] = sel[s];
                p.weights[t * K + s] = w[s];
                s_exp[t * K + s] = sel[s];
            }
        }
    }
    if (p.selector) {
        const int t = split_gate ? wave - M : wave;
        if (t >= 0 && t < M) {
            const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
            if (lane == 0) p.sgate[t] = gate;
        }
    }
    for (int e = tid; e < E; e += kPrepThreads) s_cnt[e] = 0;
    __syncthreads();
    const int NA = M * K;
    for (int a = tid; a < NA; a += kPrepThreads) atomicAdd(&s_cnt[s_exp[a]], 1);
    __syncthreads();
    // exclusive scans of the group flags and counts over experts (E <= 1024:
    // one expert per thread), by waves then across waves
    const int c = tid < E ? s_cnt[tid] : 0;
    int fl = c > 0, cs = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int f2 = __shfl_up(fl, off), c2 = __shfl_up(cs, off);
        if (lane >= off) {
            fl += f2;
            cs += c2;
        }
    }
    __shared__ int s_wf[kPrepThreads / 64], s_wc[kPrepThreads / 64];
    if (lane == 63) {
        s_wf[wave] = fl;
        s_wc[wave] = cs;
    }
    __syncthreads();
    int bf = 0, bc = 0;
    for (int w2 = 0; w2 < wave; w2++) {
        bf += s_wf[w2];
        bc += s_wc[w2];
    }
    const int gid = bf + fl - (c > 0), start = bc + cs - c;  // exclusive
    if (tid < E) {
        s_start[tid] = start;
        if (c > 0) {
            p.group_expert[gid] = tid;
            p.group_start[gid] = start;
            p.group_count[gid] = c;
        }
    }
    if (tid == kPrepThreads - 1) s_scan[0] = bf + fl;  // groups of routed experts
    __syncthreads();
    // position of (t, route): after every earlier token routed to the same
    // expert (each token lists an expert at most once)
    for (int a = tid; a < NA; a += kPrepThreads) {
        const int t = a / K, e = s_exp[a];
        int rank = 0;
        for (int b = 0; b < t * K; b++) rank += s_exp[b] == e;
        const int pos = s_start[e] + rank;
        p.assign_row[pos] = t;
        p.slot_pos[a] = pos;
    }
    const int n_routed = s_scan[0];
    const bool has_shared = p.sgate_w != nullptr;
    if (has_shared) {
        for (int t = tid; t < M; t += kPrepThreads) p.assign_row[NA + t] = t;
        if (tid == 0) {
            p.group_expert[n_routed] = E;
            p.group_start[n_routed] = NA;
            p.group_count[n_routed] = M;
        }
    }
    if (tid == 0) p.meta[0] = n_routed + (has_shared ? 1 : 0);
}

// --------------------------------------------------------------- gate/up
// Grid (I/8, M*K+1).  Workgroup (x, g): 8 intermediate rows of expert group
// g, 4 waves each taking a quarter of the NG blocks along hidden; per chunk
// of MT tokens each wave forms its blocks' exact terms, then wave w runs the
// in-order chains of tokens w, w+4, ... and stores SwiGLU.
template <int GFMT, int NG, int MT>
__global__ __launch_bounds__(256) void k_moev_gate_up(MoeParams p) {
    constexpr int NW = 4, NB = NG / NW;
    static_assert(NG % NW == 0, "shape");
    const int g = blockIdx.y;
    if (g >= p.meta[0]) return;  // whole workgroup
    __shared__ int s_isum[2][8][8][MT][NG];  // [gate/up][row][lane k][token][block]
    __shared__ int s_msum[2][8][4][MT][NG];
    __shared__ float s_dd[2][8][MT][NG], s_dm[2][8][MT][NG];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = p.group_expert[g], start = p.group_start[g], count = p.group_count[g];
    const bool shared = e == (int)p.E;
    const uint8_t* gb = shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes;
    const uint8_t* ub = shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes;
    const int64_t i = (int64_t)blockIdx.x * 8 + slot;
    const bool ok = i < p.I;
    const int64_t ic = ok ? i : p.I - 1;
    const int g0 = wave * NB;
    const uint8_t* wrow[2] = {gb + ic * p.g_row_bytes + (int64_t)g0 * WT<GFMT>::kBlockBytes,
                              ub + ic * p.g_row_bytes + (int64_t)g0 * WT<GFMT>::kBlockBytes};
    // the first token's activation blocks go out ahead of the weight burst
    const int64_t row0 = p.assign_row[start];
    uint32_t av0[NB][8];
    float yd0[NB];
    uint32_t q8s0[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        load_act(p.xq, row0, g0 + b, k, av0[b]);
        yd0[b] = p.xq.d[row0 * p.xq.ldd + g0 + b];
        q8s0[b] = GFMT == kQ4_K ? *(const uint32_t*)(p.xq.s8 + (row0 * p.xq.ng + g0 + b) * 8 + 2 * (k & 3)) : 0u;
    }
    typename WT<GFMT>::T w[2][NB];
    lanes_load_exact<GFMT, 2, NB>(wrow, k, w);
    for (int t0 = 0; t0 < count; t0 += MT) {
        const int mc = min(MT, count - t0);
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            if (tt < mc) {  // uniform
                const bool first = t0 + tt == 0;
                const int64_t row = first ? row0 : p.assign_row[start + t0 + tt];
#pragma unroll
                for (int r = 0; r < 2; r++) {
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const int gg = g0 + b;
                        uint32_t av[8];
                        float yd;
                        if (first) {
#pragma unroll
                            for (int j = 0; j < 8; j++) av[j] = av0[b][j];
                            yd = yd0[b];
                        } else {
                            load_act(p.xq, row, gg, k, av);
                            yd = p.xq.d[row * p.xq.ldd + gg];
                        }
                        if constexpr (GFMT == kQ4_K) {
                            const Q4Dec dec = q4_decode(w[r][b], k);
                            const uint32_t q8s =
                                first ? q8s0[b] : *(const uint32_t*)(p.xq.s8 + (row * p.xq.ng + gg) * 8 + 2 * (k & 3));
                            int32_t isum, msum;
                            float d, dmin;
                            q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
                            s_isum[r][slot][k][tt][gg] = isum;
                            if (k < 4) s_msum[r][slot][k][tt][gg] = msum;
                            if (k == 0) {
                                s_dd[r][slot][tt][gg] = d;
                                s_dm[r][slot][tt][gg] = dmin;
                            }
                        } else {
                            const Q6Dec dec = q6_decode(w[r][b], k);
                            int32_t isum;
                            float d;
                            q6_dot(dec, av, yd, isum, d);
                            s_isum[r][slot][k][tt][gg] = isum;
                            if (k == 0) s_dd[r][slot][tt][gg] = d;
                        }
                    }
                }
            }
        }
        __syncthreads();
        for (int tt = wave; tt < mc; tt += NW) {
            float o[2];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                float acc = 0.f, accm = 0.f;
#pragma unroll
                for (int gg = 0; gg < NG; gg++) {
                    acc = __builtin_fmaf(s_dd[r][slot][tt][gg], (float)s_isum[r][slot][k][tt][gg], acc);
                    if constexpr (GFMT == kQ4_K)
                        accm = __builtin_fmaf(s_dm[r][slot][tt][gg], (float)s_msum[r][slot][k & 3][tt][gg], accm);
                }
                float v = hsum8(acc);
                if constexpr (GFMT == kQ4_K) v = v + hsum4(accm);
                o[r] = v;
            }
            // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
            if (k == 0 && ok)
                p.act[(int64_t)(start + t0 + tt) * p.I + i] = __fdiv_rn(o[0], 1.f + exp_f32(-o[0])) * o[1];
        }
        __syncthreads();  // the terms of the next chunk reuse the arrays
    }
}

// ----------------------------------------------------------------- down
// Grid (H/8, ceil((M*K+1)/4)).  Wave w of workgroup (x, c): expert group
// 4c + w on hidden rows 8x..8x+7.  Its SwiGLU rows (up to kPre before the
// down rows are issued) are quantised into the wave's own LDS region while
// the down rows load; the products go to vals.
template <int DFMT, int NG>
__global__ __launch_bounds__(256) void k_moev_down(MoeParams p) {
    constexpr int VPL = NG * 4;  // SwiGLU values per lane (I = NG * 256)
    constexpr int LPB = 256 / VPL;
    constexpr int kPre = 4;
    static_assert(VPL == 8 || VPL == 16 || VPL == 32, "shape");
    __shared__ __align__(16) int8_t s_q[4][kVerifyMaxTokens * NG * 256];
    __shared__ __align__(16) float s_d[4][kVerifyMaxTokens * NG * 8];
    __shared__ __align__(16) int16_t s_s8[4][kVerifyMaxTokens * NG * 8];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.y * 4 + wave;
    if (g >= p.meta[0]) return;  // this wave only; no barrier follows
    const int e = p.group_expert[g], start = p.group_start[g], count = p.group_count[g];
    const int gq = lane / LPB;
    float av[kPre][VPL];
#pragma unroll
    for (int tt = 0; tt < kPre; tt++)
        q8k_vpl_load<VPL>(tt < count ? p.act + (int64_t)(start + tt) * p.I + (int64_t)gq * 256 : nullptr, av[tt]);
    const int64_t n = (int64_t)blockIdx.x * 8 + slot;
    const bool ok = n < p.H;
    const int64_t nc = ok ? n : p.H - 1;
    const uint8_t* base = e == (int)p.E ? p.sdown_w : p.down + (int64_t)e * p.d_exp_bytes;
    const uint8_t* wrow[1] = {base + nc * p.d_row_bytes};
    typename WT<DFMT>::T w[1][NG];
    lanes_load_exact<DFMT, 1, NG>(wrow, k, w);
    ActView a;
    a.ng = NG;
    a.ldq = NG * 256;
    a.ldd = NG * 8;
    a.m = count;
    a.q = s_q[wave];
    a.d = s_d[wave];
    a.s8 = s_s8[wave];
#pragma unroll
    for (int tt = 0; tt < kPre; tt++) quant_q8k_vpl<VPL>(av[tt], tt < count, tt, gq, a);
    for (int tt = kPre; tt < count; tt++) {
        float v[VPL];
        q8k_vpl_load<VPL>(p.act + (int64_t)(start + tt) * p.I + (int64_t)gq * 256, v);
        quant_q8k_vpl<VPL>(v, true, tt, gq, a);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int tt = 0; tt < count; tt++) {
        float acc[1][1] = {{0.f}}, accm[1][1] = {{0.f}};
        const int64_t arow[1][1] = {{tt}};
        const int mc[1] = {1};
        lanes_accumulate<DFMT, 1, 1, NG>(w, wrow, 0, NG, p.d_nbw, a, arow, mc, k, acc, accm);
        float o[1][1];
        lanes_finish<DFMT, 1, 1>(acc, accm, o);
        if (k == 0 && ok) p.vals[(int64_t)(start + tt) * p.H + n] = o[0][0];
    }
}

// ---------------------------------------------------------------- combine
// routed = sum over routes in order of value * weight, then hidden = routed
// + shared * gate (src/qwen/quantized_moe.rs:266-273, :384-400).
__global__ __launch_bounds__(256) void k_moev_combine(MoeParams p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.M * p.H) return;
    const int t = (int)(idx / p.H);
    const int64_t nn = idx - (int64_t)t * p.H;
    const int K = (int)p.K;
    // all positions, then all values, then the ordered sum (two round trips)
    int pos[kMoeMaxTopK];
    float wt[kMoeMaxTopK], v[kMoeMaxTopK];
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++) {
        pos[j] = j < K ? p.slot_pos[t * K + j] : 0;
        wt[j] = j < K ? p.weights[t * K + j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++) v[j] = j < K ? p.vals[(int64_t)pos[j] * p.H + nn] : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++)
        if (j < K) acc = acc + v[j] * wt[j];
    if (p.sgate_w) acc = acc + p.vals[(int64_t)(p.M * K + t) * p.H + nn] * p.sgate[t];
    p.out[(int64_t)t * p.H + nn] = acc;
}

template <int GFMT, int DFMT>
hipError_t launch_v(const MoeParams& p, hipStream_t s, hipEvent_t const* ev) {
    constexpr int AF = GFMT == kQ8_0 ? kQ8_0 : kQ4_K;
    const int gmax = p.M * (int)p.K + 1;
    const int64_t qwaves = (int64_t)p.M * p.xq.ng;
    if (ev) (void)hipEventRecord(ev[0], s);
    hipLaunchKernelGGL((k_moev_prep<AF>), dim3(1 + (unsigned)((qwaves + 15) / 16)), dim3(kPrepThreads), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[1], s);
    hipLaunchKernelGGL((k_moev_gate_up<GFMT, 8, 4>), dim3((unsigned)(p.I / 8), (unsigned)gmax), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[2], s);
    hipLaunchKernelGGL((k_moev_down<DFMT, 2>), dim3((unsigned)(p.H / 8), (unsigned)((gmax + 3) / 4)), dim3(256), 0,
                       s, p);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(k_moev_combine, dim3((unsigned)(((int64_t)p.M * p.H + 255) / 256)), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[3], s);
    return hipSuccess;
}

}  // namespace

bool moev_supported(const MoeParams& p, int gfmt, int dfmt) {
    return p.M >= 2 && p.M <= kVerifyMaxTokens && gfmt != kQ8_0 && dfmt != kQ8_0 && p.H == 2048 && p.I == 512 &&
           p.E <= kMoeMaxExperts && p.E <= kPrepThreads && p.K <= kMoeMaxTopK;
}

hipError_t launch_moe_verify(const MoeParams& p, int gfmt, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    if (!moev_supported(p, gfmt, dfmt)) return hipErrorNotSupported;
    if (gfmt == kQ4_K && dfmt == kQ6_K) return launch_v<kQ4_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ4_K && dfmt == kQ4_K) return launch_v<kQ4_K, kQ4_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ6_K) return launch_v<kQ6_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ4_K) return launch_v<kQ6_K, kQ4_K>(p, s, ev);
    return hipErrorNotSupported;
}

}  // namespace iq
