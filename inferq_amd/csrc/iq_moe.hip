// iq_moe.hip -- one quantised MoE sublayer on the GPU
// (QuantizedMoeLayer::forward, src/qwen/quantized_moe.rs:227-460).
//
// Three launches per layer:
//   k_moe_prep     workgroup 0 routes every token (softmax, top-k,
//                  renormalise: src/qwen/moe.rs:21-54), computes the shared
//                  expert's sigmoid gate and groups the (token, route) pairs
//                  by expert in ascending order (the BTreeMap order of
//                  routed_grouped_by_expert); the other workgroups quantise x.
//   k_moe_gate_up  one workgroup per (32 intermediate rows, expert group):
//                  gate and up rows of that expert against the group's
//                  tokens, SwiGLU fused; the last workgroup to finish a
//                  256-value block of an activation row quantises it for the
//                  down projection (no waiting: the last arrival does it).
//   k_moe_down     one workgroup per 8 hidden rows: the down rows of every
//                  group, then the ordered combine in token-then-route order
//                  (multiply, then add; never fused) and the shared expert.
// The shared expert is the group after the routed ones (expert id E).
// Grouping changes which rows share a launch, never what is summed or in
// which order, so the result equals token-major execution bit for bit.
#include "iq_lanes.h"
#include "iq_moe.h"
#include "iq_quant.h"
#include "iq_route.h"

namespace iq {

namespace {

constexpr int kMaxAssign = kMoeMaxAssign;

// ---------------------------------------------------------------- routing
__device__ void route_and_group(const MoeParams& p) {
    __shared__ __align__(16) float s_ev[4][kMoeMaxExperts];
    __shared__ int s_exp[kMaxAssign];
    __shared__ int s_cnt[kMoeMaxExperts];
    __shared__ int s_sg[256], s_sc[256];
    __shared__ int s_gid[kMoeMaxExperts], s_start[kMoeMaxExperts];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = (int)p.E, K = (int)p.K, M = p.M;

    for (int t = wave; t < M; t += 4) {
        int sel[kMoeMaxTopK];
        float lv[kRoutePer], w[kMoeMaxTopK];
        route_topk<kMoeMaxTopK>(p.logits + (int64_t)t * E, E, K, sel, lv);
        route_weights<kMoeMaxTopK>(lv, E, K, sel, p.normalize, s_ev[wave], w);
        if (lane == 0) {
            for (int s = 0; s < K; s++) {
                p.experts[t * K + s] = sel[s];
                p.weights[t * K + s] = w[s];
                s_exp[t * K + s] = sel[s];
            }
        }
        if (p.selector) {
            const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
            if (lane == 0) p.sgate[t] = gate;
        }
    }
    __syncthreads();

    // ---- group (token, route) pairs by expert, ascending ----
    const int NA = M * K;
    for (int e = tid; e < E; e += 256) s_cnt[e] = 0;
    __syncthreads();
    for (int a = tid; a < NA; a += 256) atomicAdd(&s_cnt[s_exp[a]], 1);
    __syncthreads();
    constexpr int EPT = kMoeMaxExperts / 256;  // experts per thread
    int lg = 0, lc = 0;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid * EPT + j;
        const int c = e < E ? s_cnt[e] : 0;
        lg += c > 0;
        lc += c;
    }
    s_sg[tid] = lg;
    s_sc[tid] = lc;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int vg = tid >= off ? s_sg[tid - off] : 0;
        const int vc = tid >= off ? s_sc[tid - off] : 0;
        __syncthreads();
        s_sg[tid] += vg;
        s_sc[tid] += vc;
        __syncthreads();
    }
    int bg = s_sg[tid] - lg, bc = s_sc[tid] - lc;  // exclusive prefixes
    const int n_routed = s_sg[255];
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid * EPT + j;
        if (e < E && s_cnt[e] > 0) {
            s_gid[e] = bg;
            s_start[e] = bc;
            p.group_expert[bg] = e;
            p.group_start[bg] = bc;
            p.group_count[bg] = s_cnt[e];
            bg += 1;
            bc += s_cnt[e];
        }
    }
    __syncthreads();
    // position of (t, route): after every earlier token routed to the same
    // expert (each token lists an expert at most once)
    for (int a = tid; a < NA; a += 256) {
        const int t = a / K, e = s_exp[a];
        int rank = 0;
        for (int b = 0; b < t * K; b++) rank += s_exp[b] == e;
        const int pos = s_start[e] + rank;
        p.assign_row[pos] = t;
        p.slot_pos[a] = pos;
    }
    const bool has_shared = p.sgate_w != nullptr;
    if (has_shared) {
        for (int t = tid; t < M; t += 256) p.assign_row[NA + t] = t;
        if (tid == 0) {
            p.group_expert[n_routed] = E;
            p.group_start[n_routed] = NA;
            p.group_count[n_routed] = M;
        }
    }
    if (tid == 0) p.meta[0] = n_routed + (has_shared ? 1 : 0);
}

template <int AFMT>
__global__ __launch_bounds__(256) void k_moe_prep(MoeParams p) {
    if (blockIdx.x == 0) {
        route_and_group(p);
        return;
    }
    const int64_t wid = (int64_t)(blockIdx.x - 1) * 4 + (threadIdx.x >> 6);
    const int ng = p.xq.ng;
    if (wid >= (int64_t)p.M * ng) return;
    const int64_t row = wid / ng;
    const int g = (int)(wid % ng);
    if constexpr (AFMT == kQ8_0) quant_q80_wave(p.x + row * p.H, p.H, row, g, p.xq, nullptr);
    else quant_q8k_wave(p.x + row * p.H + (int64_t)g * 256, row, g, p.xq, nullptr);
}

// ---------------------------------------------------------------- gate_up
template <int GFMT, int DAFMT, int MT, int BC>
__global__ __launch_bounds__(256) void k_moe_gate_up(MoeParams p) {
    const int g = blockIdx.y;
    if (g >= p.meta[0]) return;  // whole workgroup
    const int e = p.group_expert[g], start = p.group_start[g], count = p.group_count[g];
    const bool shared = e == (int)p.E;
    const uint8_t* gb = shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes;
    const uint8_t* ub = shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = lane & 7, slot = lane >> 3;
    const int64_t i = (int64_t)blockIdx.x * 32 + wave * 8 + slot;  // intermediate row
    const bool ok = i < p.I;
    const uint8_t* wrow[2] = {ok ? gb + i * p.g_row_bytes : nullptr, ok ? ub + i * p.g_row_bytes : nullptr};
    for (int m0 = 0; m0 < count; m0 += MT) {
        const int mcnt = min(MT, count - m0);
        int64_t arow[2][MT];
#pragma unroll
        for (int mi = 0; mi < MT; mi++) arow[0][mi] = arow[1][mi] = mi < mcnt ? p.assign_row[start + m0 + mi] : 0;
        const int mc[2] = {mcnt, mcnt};
        float o[2][MT];
        lanes_dot<GFMT, MT, 2, BC>(wrow, p.g_nbw, p.xq, arow, mc, k, o);
        if (k == 0 && ok) {
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                if (mi < mcnt) {
                    // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
                    const float gv = o[0][mi], uv = o[1][mi];
                    p.act[(int64_t)(start + m0 + mi) * p.I + i] = __fdiv_rn(gv, 1.f + exp_f32(-gv)) * uv;
                }
            }
        }
    }

    // The workgroup that completes a 256-value block of the activations
    // quantises it for the down projection.
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    const int tiles = (int)((p.I + 31) / 32);
    const int blk = blockIdx.x / 8;
    const int expect = min(8, tiles - blk * 8);
    const int ngI = (int)((p.I + 255) / 256);
    if (threadIdx.x == 0) {
        int* ctr = p.counters + (int64_t)g * ngI + blk;
        const int old = atomicAdd(ctr, 1);
        s_last = old == expect - 1;
        if (s_last) atomicExch(ctr, 0);  // ready for the next call
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int r = wave; r < count; r += 4) {
        const int64_t pos = start + r;
        if constexpr (DAFMT == kQ8_0) quant_q80_wave(p.act + pos * p.I, p.I, pos, blk, p.aq, nullptr);
        else quant_q8k_wave(p.act + pos * p.I + (int64_t)blk * 256, pos, blk, p.aq, nullptr);
    }
}

// ------------------------------------------------------------------- down
template <int DFMT, int MT, int R, int BC>
__global__ __launch_bounds__(256) void k_moe_down(MoeParams p) {
    const int ngroups = p.meta[0];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = lane & 7, slot = lane >> 3;
    const int64_t n = (int64_t)blockIdx.x * 8 + slot;  // hidden row
    const bool ok = n < p.H;
    for (int gc = wave; gc < ngroups; gc += 4 * R) {
        int cnt[R], st[R];
        const uint8_t* base[R];
        int maxc = 0;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int g = gc + 4 * r;
            if (g < ngroups) {
                const int e = p.group_expert[g];
                st[r] = p.group_start[g];
                cnt[r] = p.group_count[g];
                base[r] = e == (int)p.E ? p.sdown_w : p.down + (int64_t)e * p.d_exp_bytes;
            } else {
                st[r] = 0;
                cnt[r] = 0;
                base[r] = nullptr;
            }
            maxc = max(maxc, cnt[r]);
        }
        for (int m0 = 0; m0 < maxc; m0 += MT) {
            const uint8_t* wrow[R];
            int64_t arow[R][MT];
            int mc[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                mc[r] = max(0, min(MT, cnt[r] - m0));
                wrow[r] = (ok && mc[r] > 0) ? base[r] + n * p.d_row_bytes : nullptr;
#pragma unroll
                for (int mi = 0; mi < MT; mi++) arow[r][mi] = st[r] + m0 + mi;
            }
            float o[R][MT];
            lanes_dot<DFMT, MT, R, BC>(wrow, p.d_nbw, p.aq, arow, mc, k, o);
            if (k == 0 && ok) {
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int mi = 0; mi < MT; mi++)
                        if (mi < mc[r]) p.vals[(int64_t)(st[r] + m0 + mi) * p.H + n] = o[r][mi];
            }
        }
    }
    __syncthreads();
    // ordered combine: routed = sum over routes in order of value * weight,
    // then hidden = routed + shared * gate (src/qwen/quantized_moe.rs:266-273,
    // :384-400)
    const int K = (int)p.K;
    for (int idx = threadIdx.x; idx < p.M * 8; idx += 256) {
        const int t = idx >> 3;
        const int64_t nn = (int64_t)blockIdx.x * 8 + (idx & 7);
        if (nn >= p.H) continue;
        float acc = 0.f;
        for (int j = 0; j < K; j++) {
            const int pos = p.slot_pos[t * K + j];
            acc = acc + p.vals[(int64_t)pos * p.H + nn] * p.weights[t * K + j];
        }
        if (p.sgate_w) acc = acc + p.vals[(int64_t)(p.M * K + t) * p.H + nn] * p.sgate[t];
        if (p.residual) acc = p.residual[(int64_t)t * p.H + nn] + acc;  // src/qwen/quantized_layer.rs:212
        p.out[(int64_t)t * p.H + nn] = acc;
    }
}

// ------------------------------------- token-major kernels (decode, verify)
// Each token runs on its own slice of the grid (routed_token_major,
// src/qwen/quantized_moe.rs:283-318): no grouping is needed, so the routing
// is recomputed where it is used and each launch has a single dependent
// memory round trip before its weight loads (logits -> weights).  A token's
// output is bitwise the one-token call's, which is the grouped execution's
// too (the reference asserts grouped == token-major).  An expert picked by
// several tokens is read once per token, mostly from L2: up to a few dozen
// tokens this beats grouping, whose per-expert launches wait on the grouping
// pass and have far less weight traffic in flight per CU.

constexpr int kMoe1MaxSlots = 12;  // top-k routes plus the shared expert
// widest call served token-major (graph replays, grouped against
// token-major: 32 tokens 121.4 against 118.9 us, 36: 127.9 against 130.7,
// 48: 142.8 against 165.6)
constexpr int kMoeTokenMajorMax = 32;
constexpr int kMoeRouteLaunchMin = 12;  // calls this wide route in a launch of their own
// 8-row groups of gate (and of up) per workgroup of the multi-token form:
// 1, 2 and 4 measure 45.3 / 44.1 / 44.9 us at 8 tokens, 17.2 / 17.0 / 17.9
// at 2 and 118 / 111 / 109 at 28
constexpr int kMoe1RowGroups = 2;
// calls this wide quantise their SwiGLU rows in a launch of their own: 16
// tokens 71.8 -> 71.0 us, 28 tokens 113 -> 106.7 us; at 8 tokens the extra
// launch costs 2 us more than the repeated quantisation
constexpr int kMoe1ActqMin = 16;

// Routing workgroup of token t's gate/up slice: wave 0 routes the token
// (top-k), wave 2 forms the softmax denominator meanwhile (it does not
// depend on the selection) and wave 0 then the exact weights; wave 1
// computes the shared-expert gate.  In a workgroup of fewer than three
// waves wave 0 does both parts.  Both chains are serial, and the gate/up
// launch ends with the last of its workgroups: with both parts on wave 0
// that was this one (M=1 layer 13.1 -> 12.8 us with the split).
__device__ void moe1_route(const MoeParams& p, int wave, int t) {
    const int K = (int)p.K, E = (int)p.E, lane = threadIdx.x & 63;
    __shared__ __align__(16) float s_scratch[kMoeMaxExperts];
    __shared__ int s_sel[kMoeMaxTopK];
    __shared__ float s_wt[kMoeMaxTopK];
    __shared__ float s_den;
    const bool split = blockDim.x >= 192;
    if (wave == 1) {
        if (p.sdown_w) {
            const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
            if (lane == 0) p.sgate[t] = gate;
        }
        return;
    }
    if (wave > 2 || (wave == 2 && !split)) return;
    float lv[kRoutePer];
    route_load(p.logits + (int64_t)t * E, E, lv);
    if (wave == 2) {
        const float den = route_softmax_den(lv, E, s_scratch);
        if (lane == 0) s_den = den;
    } else {
        route_topk_each_any(lv, E, K, [&](int s, int e) {
            if (lane == 0) {
                p.experts[t * K + s] = e;  // the down launch needs the ids first
                s_sel[s] = e;
            }
        });
        if (!split) {
            const float den = route_softmax_den(lv, E, s_scratch);
            if (lane == 0) s_den = den;
        }
    }
    if (split) lds_barrier();  // waves 0 and 2 (the others have ended)
    if (wave != 0) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    route_pick_weights(s_den, K, s_sel, p.normalize, s_scratch, s_wt);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < K) p.weights[t * K + lane] = s_wt[lane];
}

// The one-token form.  Grid (I/8, slots + 1, M): row 0 of each token
// holds its routing workgroup (x == 0); workgroup (x, K - s, t) forms the 8
// intermediate rows from 8 x of gate and up of token t's expert at route
// rank s (row K + 1: the shared expert), split by K over eight waves: gate on
// waves 0-3 and up on waves 4-7, each wave a quarter of the blocks of one
// matrix.  Each wave forms its blocks' exact lane integers and f32 scales;
// wave 0 then advances the accumulators through all NG blocks in order (the
// reference's chain), reduces them with the hsum trees and applies SwiGLU.
// Splitting by K shortens the one token's dependent chain: each wave decodes
// a quarter of a row.  Wave 0 alone runs the top-k and hands the expert id
// over in LDS (eight waves each repeating it were slower than four); waves
// 0-3 quantise x for all eight.
template <int GFMT, int NG>
__global__ __launch_bounds__(512) void k_moe1_gate_up8(MoeParams p) {
    constexpr int NW = 4, NB = NG / NW, VPL = NB * 4;  // blocks and x values per lane per wave
    static_assert(NG % NW == 0 && (VPL == 8 || VPL == 16 || VPL == 32), "shape");
    __shared__ __align__(16) int8_t s_q[NG * 256];
    __shared__ __align__(16) float s_d[NG * 8];
    __shared__ __align__(16) int16_t s_s8[NG * 8];
    __shared__ int s_isum[2][8][8][NG];  // [gate/up][row][lane k][block]
    __shared__ int s_msum[2][8][4][NG];
    __shared__ float s_dd[2][8][NG], s_dm[2][8][NG];
    __shared__ int s_e;
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int quarter = wave & 3, r = wave >> 2;  // r: 0 gate, 1 up
    const int K = (int)p.K, t = blockIdx.z;
    const int nslots = K + (p.sdown_w ? 1 : 0);
    if (blockIdx.y == 0) {
        if (blockIdx.x == 0) moe1_route(p, wave, t);
        return;
    }
    // grid rows 1..K hold route ranks K-1..0, row K+1 the shared expert: the
    // ranks whose top-k takes the most rounds are dispatched first (M=1 layer
    // 12.84 -> 12.70 us)
    const int sidx = (int)blockIdx.y <= K ? K - (int)blockIdx.y : K;
    constexpr int LPB = 256 / VPL;
    const int g0 = quarter * NB;
    const int gx = g0 + lane / LPB;  // x block this lane quantises (waves 0-3)
    float xv[VPL];
    if (r == 0) q8k_vpl_load<VPL>(p.x + (int64_t)t * p.H + (int64_t)gx * 256, xv);
    int e = (int)p.E;
    if (wave == 0 && sidx < K) {
        float lv[kRoutePer];
        route_load(p.logits + (int64_t)t * p.E, (int)p.E, lv);
        route_topk_each_any(lv, (int)p.E, sidx + 1, [&](int s, int pick) {
            if (s == sidx && lane == 0) s_e = pick;
        });
    }
    lds_barrier();
    if (sidx < K) e = __builtin_amdgcn_readfirstlane(s_e);
    const bool shared = sidx >= K;
    const uint8_t* mb = r == 0 ? (shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes)
                               : (shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes);
    const int64_t i = (int64_t)blockIdx.x * 8 + slot;
    const bool ok = i < p.I;
    const int64_t ic = ok ? i : p.I - 1;
    const uint8_t* wrow[1] = {mb + ic * p.g_row_bytes + (int64_t)g0 * WT<GFMT>::kBlockBytes};
    typename WT<GFMT>::T w[1][NB];
    lanes_load_exact<GFMT, 1, NB>(wrow, k, w);
    ActView a;
    a.ng = NG;
    a.ldq = NG * 256;
    a.ldd = NG * 8;
    a.m = 1;
    a.q = s_q;
    a.d = s_d;
    a.s8 = s_s8;
    if (r == 0) quant_q8k_vpl<VPL>(xv, true, 0, gx, a);
    lds_barrier();  // the quantised x, from waves 0-3, for all eight
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int g = g0 + b;
        uint32_t av[8];
        load_act(a, 0, g, k, av);
        const float yd = a.d[g];
        if constexpr (GFMT == kQ4_K || GFMT == kQ5_K) {
            Q4Dec dec;
            if constexpr (GFMT == kQ4_K) dec = q4_decode(w[0][b], k);
            else dec = q5_decode(w[0][b], k);
            const uint32_t q8s = *(const uint32_t*)(a.s8 + g * 8 + 2 * (k & 3));
            int32_t isum, msum;
            float d, dmin;
            q4_dot(dec, av, yd, q8s, isum, msum, d, dmin);
            s_isum[r][slot][k][g] = isum;
            if constexpr (GFMT == kQ5_K) {  // the Q5_K mins: one f32 scalar per row
                const int32_t mtot = isum_quad(msum);
                if (k == 0) s_msum[r][slot][0][g] = mtot;
            } else if (k < 4) {
                s_msum[r][slot][k][g] = msum;
            }
            if (k == 0) {
                s_dd[r][slot][g] = d;
                s_dm[r][slot][g] = dmin;
            }
        } else {
            const Q6Dec dec = q6_decode(w[0][b], k);
            int32_t isum;
            float d;
            q6_dot(dec, av, yd, isum, d);
            s_isum[r][slot][k][g] = isum;
            if (k == 0) s_dd[r][slot][g] = d;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    float o[2];
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
        float acc = 0.f, accm = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            acc = __builtin_fmaf(s_dd[rr][slot][g], (float)s_isum[rr][slot][k][g], acc);
            if constexpr (GFMT == kQ4_K)
                accm = __builtin_fmaf(s_dm[rr][slot][g], (float)s_msum[rr][slot][k & 3][g], accm);
            if constexpr (GFMT == kQ5_K) accm = accm + s_dm[rr][slot][g] * (float)s_msum[rr][slot][0][g];
        }
        float v = hsum8(acc);
        if constexpr (GFMT == kQ4_K) v = v + hsum4(accm);
        if constexpr (GFMT == kQ5_K) v = v + accm;
        o[rr] = v;
    }
    // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
    if (k == 0 && ok) p.act[((int64_t)t * nslots + sidx) * p.I + i] = __fdiv_rn(o[0], 1.f + exp_f32(-o[0])) * o[1];
}

// The form for 2..kMoeTokenMajorMax tokens: grid (I / (8 RG), slots (+1
// routing row when !PRE), M), 2 RG waves.  Workgroup (x, s, t): the 8 RG
// intermediate rows from 8 RG x of gate (waves 0..RG-1) and up (waves
// RG..2RG-1) of token t's expert at route rank s.  Every wave runs the
// reference chain of its own 8 rows through all NG blocks (no hand-over
// between waves), so a workgroup forms 8 RG rows of SwiGLU for one top-k
// and one x quantisation; the gate waves hand their products to the up
// waves in LDS.  With many tokens the GPU is full of such workgroups, and
// the shorter chain of the split-K form no longer pays for its hand-over
// and its repeated top-k (8 tokens 45.6 -> 44.0 us, 16 tokens 77.6 -> 69.2,
// 28 tokens 120 -> 111).  The chain, the hsum trees and SwiGLU are the
// one-token form's, so the outputs are the same bits.  PRE = false: every
// workgroup finds its expert by a top-k of its own; PRE = true (grid y =
// slots): k_moe1_route ran first and the workgroups read the expert ids,
// which wide calls amortise better.
template <int GFMT, int NG, bool PRE, int RG>
__global__ __launch_bounds__(128 * RG) void k_moe1_gate_up_rows(MoeParams p) {
    constexpr int NWQ = 2 * RG < 4 ? 2 * RG : 4;  // waves that quantise x
    constexpr int VPL = NG * 4 / NWQ;
    static_assert(VPL == 8 || VPL == 16 || VPL == 32, "shape");
    __shared__ __align__(16) int8_t s_q[NG * 256];
    __shared__ __align__(16) float s_d[NG * 8];
    __shared__ __align__(16) int16_t s_s8[NG * 8];
    __shared__ float s_g[RG][8];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = wave / RG, rg = wave - r * RG;  // r: 0 gate, 1 up
    const int K = (int)p.K, t = blockIdx.z;
    const int nslots = K + (p.sdown_w ? 1 : 0);
    if (!PRE && blockIdx.y == 0) {
        if (blockIdx.x == 0) moe1_route(p, wave, t);
        return;
    }
    const int sidx = PRE ? (int)blockIdx.y : (int)blockIdx.y - 1;
    constexpr int LPB = 256 / VPL;
    const int gx = wave * (64 / LPB) + lane / LPB;  // x block this lane quantises
    float xv[VPL];
    if (wave < NWQ) q8k_vpl_load<VPL>(p.x + (int64_t)t * p.H + (int64_t)gx * 256, xv);
    int e = (int)p.E;
    if constexpr (PRE) {
        if (sidx < K) e = __builtin_amdgcn_readfirstlane(p.experts[t * K + sidx]);
    } else {
        __shared__ int s_e;
        if (wave == 0 && sidx < K) {
            float lv[kRoutePer];
            route_load(p.logits + (int64_t)t * p.E, (int)p.E, lv);
            const int er = route_rank(lv, (int)p.E, sidx);  // 4 tokens: 24.5 -> 23.9 us
            if (lane == 0) s_e = er;
        }
        lds_barrier();
        if (sidx < K) e = __builtin_amdgcn_readfirstlane(s_e);
    }
    const bool shared = sidx >= K;
    const uint8_t* mb = r == 0 ? (shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes)
                               : (shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes);
    const int64_t i = ((int64_t)blockIdx.x * RG + rg) * 8 + slot;
    const bool ok = i < p.I;
    const int64_t ic = ok ? i : p.I - 1;
    const uint8_t* wrow[1] = {mb + ic * p.g_row_bytes};
    typename WT<GFMT>::T w[1][NG];
    lanes_load_exact<GFMT, 1, NG>(wrow, k, w);
    ActView a;
    a.ng = NG;
    a.ldq = NG * 256;
    a.ldd = NG * 8;
    a.m = 1;
    a.q = s_q;
    a.d = s_d;
    a.s8 = s_s8;
    if (wave < NWQ) quant_q8k_vpl<VPL>(xv, true, 0, gx, a);
    lds_barrier();  // the quantised x for every wave
    float acc[1][1] = {{0.f}}, accm[1][1] = {{0.f}};
    const int64_t arow[1][1] = {{0}};
    const int mc[1] = {1};
    lanes_accumulate<GFMT, 1, 1, NG>(w, wrow, 0, NG, NG, a, arow, mc, k, acc, accm);
    float o[1][1];
    lanes_finish<GFMT, 1, 1>(acc, accm, o);
    if (r == 0 && k == 0) s_g[rg][slot] = o[0][0];
    lds_barrier();
    // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
    if (r == 1 && k == 0 && ok) {
        const float g = s_g[rg][slot];
        p.act[((int64_t)t * nslots + sidx) * p.I + i] = __fdiv_rn(g, 1.f + exp_f32(-g)) * o[0][0];
    }
}

// Routing of every token of a call (grid M, three waves each: top-k, shared
// gate, softmax denominator).
__global__ __launch_bounds__(192) void k_moe1_route(MoeParams p) { moe1_route(p, (int)(threadIdx.x >> 6), blockIdx.x); }

// Grid (H/8, M); one wave per route slot of token t = blockIdx.y (blockDim
// 64 * slots), all on the same 8 hidden rows.  Each wave loads its slot's
// expert id and SwiGLU row, issues its down-row burst, quantises the SwiGLU
// row into LDS while the weights fly, and forms the row products; the 8
// rows are then combined in route order (multiply, then add) plus
// shared * gate.
// One wave per (token-major act row, 256-value block): Q8K for the down
// waves of wide calls (quant_q8k_wave: the bytes, scale and 32-value sums of
// from_float, as the down waves would form them).
__global__ __launch_bounds__(256) void k_moe1_actq(MoeParams p, int P) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = p.aq.ng;
    if (wid >= (int64_t)P * nb) return;  // uniform per wave
    const int64_t row = wid / nb;
    const int b = (int)(wid - row * nb);
    quant_q8k_wave(p.act + row * p.I + (int64_t)b * 256, row, b, p.aq, nullptr);
}

// QA: the SwiGLU rows come quantised (k_moe1_actq); otherwise each wave
// quantises its slot's row into LDS, which every workgroup of the token
// repeats -- cheaper than a launch of its own below kMoe1ActqMin tokens.
template <int DFMT, int NG, bool QA = false>
__global__ __launch_bounds__(1024) void k_moe1_down(MoeParams p) {
    constexpr int VPL = NG * 4;  // SwiGLU values per lane (I = NG * 256)
    static_assert(VPL == 8 || VPL == 16 || VPL == 32, "shape");
    __shared__ __align__(16) int8_t s_q[kMoe1MaxSlots * NG * 256];
    __shared__ __align__(16) float s_d[kMoe1MaxSlots * NG * 8];
    __shared__ __align__(16) int16_t s_s8[kMoe1MaxSlots * NG * 8];
    __shared__ float s_vals[kMoe1MaxSlots][8];
    const int lane = threadIdx.x & 63, k = lane & 7, slot = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // = route slot
    const int K = (int)p.K, t = blockIdx.y;
    const bool has_shared = p.sdown_w != nullptr;
    const int nslots = K + (has_shared ? 1 : 0);
    constexpr int LPB = 256 / VPL;
    const int gq = lane / LPB;
    float av[VPL];
    if constexpr (!QA) q8k_vpl_load<VPL>(p.act + ((int64_t)t * nslots + wave) * p.I + (int64_t)gq * 256, av);
    const int e = wave < K ? __builtin_amdgcn_readfirstlane(p.experts[t * K + wave]) : 0;
    const int64_t n = (int64_t)blockIdx.x * 8 + slot;
    const bool ok = n < p.H;
    const int64_t nc = ok ? n : p.H - 1;
    const uint8_t* base = wave < K ? p.down + (int64_t)e * p.d_exp_bytes : p.sdown_w;
    const uint8_t* wrow[1] = {base + nc * p.d_row_bytes};
    typename WT<DFMT>::T w[1][NG];
    lanes_load_exact<DFMT, 1, NG>(wrow, k, w);
    ActView a;
    int64_t ar0 = wave;
    if constexpr (QA) {
        a = p.aq;
        ar0 = (int64_t)t * nslots + wave;
    } else {
        a.ng = NG;
        a.ldq = NG * 256;
        a.ldd = NG * 8;
        a.m = nslots;
        a.q = s_q;
        a.d = s_d;
        a.s8 = s_s8;
        quant_q8k_vpl<VPL>(av, true, wave, gq, a);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float acc[1][1] = {{0.f}}, accm[1][1] = {{0.f}};
    const int64_t arow[1][1] = {{ar0}};
    const int mc[1] = {1};
    lanes_accumulate<DFMT, 1, 1, NG>(w, wrow, 0, NG, p.d_nbw, a, arow, mc, k, acc, accm);
    float o[1][1];
    lanes_finish<DFMT, 1, 1>(acc, accm, o);
    if (k == 0) s_vals[wave][slot] = o[0][0];
    __syncthreads();
    if (threadIdx.x < 8) {
        const int64_t nn = (int64_t)blockIdx.x * 8 + threadIdx.x;
        if (nn < p.H) {
            float v = 0.f;
            for (int j = 0; j < K; j++) v = v + s_vals[j][threadIdx.x] * p.weights[t * K + j];
            if (has_shared) v = v + s_vals[K][threadIdx.x] * p.sgate[t];
            if (p.residual) v = p.residual[(int64_t)t * p.H + nn] + v;  // src/qwen/quantized_layer.rs:212
            p.out[(int64_t)t * p.H + nn] = v;
        }
    }
}

// The token-major kernels cover K-quant experts with hidden 2048 and
// intermediate 512 (Qwen3.6-35B-A3B and Qwen3-Next) up to
// kMoeTokenMajorMax tokens; other calls take the grouped paths.
bool moe1_supported(const MoeParams& p, int gfmt, int dfmt) {
    const int nslots = (int)p.K + (p.sdown_w ? 1 : 0);
    // Q5_K experts: the lane kernel's products, its mins scalar
    const bool fmts = (gfmt == kQ4_K || gfmt == kQ5_K || gfmt == kQ6_K) &&
                      (dfmt == kQ4_K || dfmt == kQ5_K || dfmt == kQ6_K);
    return p.M >= 1 && p.M <= kMoeTokenMajorMax && fmts && p.H == 2048 && p.I == 512 && nslots <= kMoe1MaxSlots &&
           p.E <= kMoeMaxExperts;
}

// Stage 1 (gate/up, with the routing launch of a wide call) or 2 (down) of
// a token-major call.
template <int GFMT, int DFMT>
hipError_t launch_moe1_stage(const MoeParams& p, int stage, hipStream_t s) {
    const int nslots = (int)p.K + (p.sdown_w ? 1 : 0);
    const unsigned m = (unsigned)p.M, rows_i = (unsigned)(p.I / 8);
    if (stage == 1) {
        constexpr int RG = kMoe1RowGroups;
        const unsigned rows_g = (unsigned)(p.I / (8 * RG));
        if (p.M >= kMoeRouteLaunchMin) {
            hipLaunchKernelGGL(k_moe1_route, dim3(m), dim3(192), 0, s, p);
            hipLaunchKernelGGL((k_moe1_gate_up_rows<GFMT, 8, true, RG>), dim3(rows_g, nslots, m), dim3(128 * RG), 0, s,
                               p);
        } else if (m == 1) {
            hipLaunchKernelGGL((k_moe1_gate_up8<GFMT, 8>), dim3(rows_i, nslots + 1, m), dim3(512), 0, s, p);
        } else {
            hipLaunchKernelGGL((k_moe1_gate_up_rows<GFMT, 8, false, RG>), dim3(rows_g, nslots + 1, m), dim3(128 * RG), 0,
                               s, p);
        }
    } else if (stage == 2) {
        if (p.M >= kMoe1ActqMin) {
            const int P = p.M * nslots;
            const int64_t aw = (int64_t)P * p.aq.ng;
            hipLaunchKernelGGL(k_moe1_actq, dim3((unsigned)((aw + 3) / 4)), dim3(256), 0, s, p, P);
            hipLaunchKernelGGL((k_moe1_down<DFMT, 2, true>), dim3((unsigned)(p.H / 8), m), dim3(64 * nslots), 0, s, p);
        } else {
            hipLaunchKernelGGL((k_moe1_down<DFMT, 2>), dim3((unsigned)(p.H / 8), m), dim3(64 * nslots), 0, s, p);
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int GFMT, int DFMT>
hipError_t launch_moe1(const MoeParams& p, hipStream_t s, hipEvent_t const* ev) {
    if (ev) (void)hipEventRecord(ev[1], s);
    if (hipError_t e = launch_moe1_stage<GFMT, DFMT>(p, 1, s)) return e;
    if (ev) (void)hipEventRecord(ev[2], s);
    if (hipError_t e = launch_moe1_stage<GFMT, DFMT>(p, 2, s)) return e;
    if (ev) (void)hipEventRecord(ev[3], s);
    return hipSuccess;
}

template <int GFMT>
hipError_t launch_moe1_g(const MoeParams& p, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    switch (dfmt) {
    case kQ4_K: return launch_moe1<GFMT, kQ4_K>(p, s, ev);
    case kQ5_K: return launch_moe1<GFMT, kQ5_K>(p, s, ev);
    case kQ6_K: return launch_moe1<GFMT, kQ6_K>(p, s, ev);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------- router
// Grid (E, ceil(M / TT)), one wave per workgroup: expert e = blockIdx.x
// against tokens blockIdx.y * TT ..; each lane keeps one partial sum per
// token over h = lane + 64 j (the router row is read once per TT tokens).
// U values per lane are loaded before any is summed (one token: U = 32, the
// whole 2048-wide row in one round trip instead of four), in the same order.
template <int TT, int U>
__global__ __launch_bounds__(64) void k_moe_router(MoeParams p) {
    const int lane = threadIdx.x;
    const int e = blockIdx.x, t0 = blockIdx.y * TT;
    const int nt = min(TT, p.M - t0);
    const int64_t H = p.H;
    const float* r = p.router + (int64_t)e * H;
    float part[TT];
#pragma unroll
    for (int i = 0; i < TT; i++) part[i] = 0.f;
    int64_t h = lane;
    for (; h + 64 * (U - 1) < H; h += 64 * U) {
        float rv[U];
#pragma unroll
        for (int j = 0; j < U; j++) rv[j] = r[h + 64 * j];
#pragma unroll
        for (int i = 0; i < TT; i++) {
            if (i < nt) {
                const float* xr = p.x + (int64_t)(t0 + i) * H + h;
                float xv[U];
#pragma unroll
                for (int j = 0; j < U; j++) xv[j] = xr[64 * j];
#pragma unroll
                for (int j = 0; j < U; j++) part[i] = part[i] + xv[j] * rv[j];
            }
        }
    }
    for (; h < H; h += 64) {
        const float rv = r[h];
#pragma unroll
        for (int i = 0; i < TT; i++)
            if (i < nt) part[i] = part[i] + p.x[(int64_t)(t0 + i) * H + h] * rv;
    }
#pragma unroll
    for (int i = 0; i < TT; i++) {
        float v = part[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
        if (lane == 0 && i < nt) p.logits_ws[(int64_t)(t0 + i) * p.E + e] = v;
    }
}

// ------------------------------------------------------------- launchers
template <int GFMT, int DFMT>
hipError_t launch_gd(const MoeParams& p, hipStream_t s, hipEvent_t const* ev) {
    constexpr int GAF = GFMT == kQ8_0 ? kQ8_0 : kQ4_K;  // activation format of x
    constexpr int DAF = DFMT == kQ8_0 ? kQ8_0 : kQ4_K;  // activation format of act
    const int gmax = p.M * (int)p.K + 1;
    const unsigned tilesI = (unsigned)((p.I + 31) / 32);
    const unsigned groupsH = (unsigned)((p.H + 7) / 8);
    if (p.M == 1) {
        hipLaunchKernelGGL((k_moe_gate_up<GFMT, DAF, 1, GFMT == kQ8_0 ? 4 : 8>), dim3(tilesI, gmax), dim3(256), 0, s, p);
        if (hipError_t e = hipGetLastError()) return e;
        if (ev) (void)hipEventRecord(ev[2], s);
        hipLaunchKernelGGL((k_moe_down<DFMT, 1, 3, 2>), dim3(groupsH), dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((k_moe_gate_up<GFMT, DAF, 8, GFMT == kQ8_0 ? 2 : 4>), dim3(tilesI, gmax), dim3(256), 0, s, p);
        if (hipError_t e = hipGetLastError()) return e;
        if (ev) (void)hipEventRecord(ev[2], s);
        hipLaunchKernelGGL((k_moe_down<DFMT, 8, 2, 2>), dim3(groupsH), dim3(256), 0, s, p);
    }
    (void)GAF;
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[3], s);
    return hipSuccess;
}

template <int GFMT>
hipError_t launch_g(const MoeParams& p, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    switch (dfmt) {
    case kQ4_K: return launch_gd<GFMT, kQ4_K>(p, s, ev);
    case kQ5_K: return launch_gd<GFMT, kQ5_K>(p, s, ev);
    case kQ6_K: return launch_gd<GFMT, kQ6_K>(p, s, ev);
    case kQ8_0: return launch_gd<GFMT, kQ8_0>(p, s, ev);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_moe(const MoeParams& p, int gfmt, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    if (moe1_supported(p, gfmt, dfmt)) {
        if (ev) (void)hipEventRecord(ev[0], s);
        switch (gfmt) {
        case kQ4_K: return launch_moe1_g<kQ4_K>(p, dfmt, s, ev);
        case kQ5_K: return launch_moe1_g<kQ5_K>(p, dfmt, s, ev);
        case kQ6_K: return launch_moe1_g<kQ6_K>(p, dfmt, s, ev);
        default: return hipErrorInvalidValue;
        }
    }
    if (moep_supported(p, gfmt, dfmt)) return launch_moe_prefill(p, gfmt, dfmt, s, ev);
    const int64_t qwaves = (int64_t)p.M * p.xq.ng;
    const unsigned prep_blocks = 1 + (unsigned)((qwaves + 3) / 4);
    if (ev) (void)hipEventRecord(ev[0], s);
    if (gfmt == kQ8_0) hipLaunchKernelGGL((k_moe_prep<kQ8_0>), dim3(prep_blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((k_moe_prep<kQ4_K>), dim3(prep_blocks), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[1], s);
    switch (gfmt) {
    case kQ4_K: return launch_g<kQ4_K>(p, dfmt, s, ev);
    case kQ5_K: return launch_g<kQ5_K>(p, dfmt, s, ev);
    case kQ6_K: return launch_g<kQ6_K>(p, dfmt, s, ev);
    case kQ8_0: return launch_g<kQ8_0>(p, dfmt, s, ev);
    default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------- a shared expert run apart
// When the shared expert's formats differ from the routed experts', the
// layer runs it as plain products (gate and up on x, down on the SwiGLU
// rows: QuantizedMoeLayer's shared path, src/qwen/quantized_moe.rs:266-273)
// and these two kernels finish it.

// act[t][i] = (g / (1 + exp(-g))) * u, the reference's SwiGLU.
__global__ __launch_bounds__(256) void k_moe_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                                                    int64_t n, float* __restrict__ act) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    act[i] = __fdiv_rn(gv, 1.f + exp_f32(-gv)) * u[i];
}

// out[t] = residual[t] + (out[t] + shared[t] * sigmoid(x[t] . selector)):
// `out` holds the routed sum (the routed launches ran without the shared
// expert and the residual), so the additions keep the fused kernels' order.
// Grid (ceil(H / 256), M); wave 0 forms the token's gate.
__global__ __launch_bounds__(256) void k_moe_shared_combine(const float* __restrict__ x,
                                                            const float* __restrict__ selector,
                                                            const float* __restrict__ shared,
                                                            const float* __restrict__ residual, int64_t H,
                                                            float* __restrict__ out) {
    __shared__ float s_gate;
    const int64_t t = blockIdx.y;
    if (threadIdx.x < 64) {
        const float gate = selector_gate(x + t * H, selector, H);
        if (threadIdx.x == 0) s_gate = gate;
    }
    __syncthreads();
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= H) return;
    float v = out[t * H + n] + shared[t * H + n] * s_gate;
    if (residual) v = residual[t * H + n] + v;  // src/qwen/quantized_layer.rs:212
    out[t * H + n] = v;
}



hipError_t launch_moe_swiglu(const float* g, const float* u, int64_t n, float* act, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_moe_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, n, act);
    return hipGetLastError();
}

hipError_t launch_moe_shared_combine(const float* x, const float* selector, const float* shared, const float* residual,
                                     int64_t m, int64_t H, float* out, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_moe_shared_combine, dim3((unsigned)((H + 255) / 256), (unsigned)m), dim3(256), 0, s, x,
                       selector, shared, residual, H, out);
    return hipGetLastError();
}

hipError_t launch_moe_router(const MoeParams& p, hipStream_t s) {
    if (!p.router || !p.logits_ws || p.M < 1) return hipErrorInvalidValue;
    if (p.M <= 2) hipLaunchKernelGGL((k_moe_router<1, 32>), dim3((unsigned)p.E, (unsigned)p.M), dim3(64), 0, s, p);
    else hipLaunchKernelGGL((k_moe_router<8, 8>), dim3((unsigned)p.E, (unsigned)((p.M + 7) / 8)), dim3(64), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_moe_stage(const MoeParams& p, int gfmt, int dfmt, int stage, hipStream_t s) {
    if (!moe1_supported(p, gfmt, dfmt)) return hipErrorNotSupported;
    if (gfmt == kQ4_K && dfmt == kQ6_K) return launch_moe1_stage<kQ4_K, kQ6_K>(p, stage, s);
    if (gfmt == kQ4_K && dfmt == kQ4_K) return launch_moe1_stage<kQ4_K, kQ4_K>(p, stage, s);
    if (gfmt == kQ6_K && dfmt == kQ6_K) return launch_moe1_stage<kQ6_K, kQ6_K>(p, stage, s);
    if (gfmt == kQ6_K && dfmt == kQ4_K) return launch_moe1_stage<kQ6_K, kQ4_K>(p, stage, s);
    if (gfmt == kQ4_K && dfmt == kQ5_K) return launch_moe1_stage<kQ4_K, kQ5_K>(p, stage, s);
    if (gfmt == kQ6_K && dfmt == kQ5_K) return launch_moe1_stage<kQ6_K, kQ5_K>(p, stage, s);
    if (gfmt == kQ5_K && dfmt == kQ4_K) return launch_moe1_stage<kQ5_K, kQ4_K>(p, stage, s);
    if (gfmt == kQ5_K && dfmt == kQ5_K) return launch_moe1_stage<kQ5_K, kQ5_K>(p, stage, s);
    if (gfmt == kQ5_K && dfmt == kQ6_K) return launch_moe1_stage<kQ5_K, kQ6_K>(p, stage, s);
    return hipErrorNotSupported;
}

}  // namespace iq
