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

namespace iq {

namespace {

constexpr int kMaxAssign = kMoeMaxAssign;

// ---------------------------------------------------------------- routing
__device__ void route_and_group(const MoeParams& p) {
    __shared__ float s_ev[4][kMoeMaxExperts];
    __shared__ int s_exp[kMaxAssign];
    __shared__ int s_cnt[kMoeMaxExperts];
    __shared__ int s_sg[256], s_sc[256];
    __shared__ int s_gid[kMoeMaxExperts], s_start[kMoeMaxExperts];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = (int)p.E, K = (int)p.K, M = p.M;
    constexpr int PER = kMoeMaxExperts / 64;

    for (int t = wave; t < M; t += 4) {
        const float* lg = p.logits + (int64_t)t * E;
        float ev[PER];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = lane + 64 * j;
            ev[j] = i < E ? lg[i] : -INFINITY;
            mx = fmaxf(mx, ev[j]);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = lane + 64 * j;
            ev[j] = i < E ? exp_f32(ev[j] - mx) : 0.f;
            if (i < E) s_ev[wave][i] = ev[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // The softmax denominator is a sequential f32 sum in index order.
        float den = 0.f;
        for (int i = 0; i < E; i++) den = den + s_ev[wave][i];
        float pr[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) pr[j] = __fdiv_rn(ev[j], den);

        // top-k by probability, descending; equal probabilities keep index order
        uint32_t taken = 0;
        int sel_e[kMoeMaxTopK];
        float sel_p[kMoeMaxTopK];
        for (int s = 0; s < K; s++) {
            float bp = -1.f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int i = lane + 64 * j;
                // a NaN probability ranks below every number (the reference's
                // partial_cmp treats it as equal to everything)
                const float pv = pr[j] == pr[j] ? pr[j] : -0.5f;
                if (i < E && !((taken >> j) & 1u) && pv > bp) {
                    bp = pv;
                    bi = i;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float op = __shfl_xor(bp, off);
                const int oi = __shfl_xor(bi, off);
                if (op > bp || (op == bp && oi < bi)) {
                    bp = op;
                    bi = oi;
                }
            }
            if (bi != 0x7fffffff && (bi & 63) == lane) taken |= 1u << (bi >> 6);
            sel_e[s] = bi;
            sel_p[s] = bp;
        }
        if (p.normalize) {
            float sum = 0.f;
            for (int s = 0; s < K; s++) sum = sum + sel_p[s];
            for (int s = 0; s < K; s++) sel_p[s] = __fdiv_rn(sel_p[s], sum);
        }
        if (lane == 0) {
            for (int s = 0; s < K; s++) {
                p.experts[t * K + s] = sel_e[s];
                p.weights[t * K + s] = sel_p[s];
                s_exp[t * K + s] = sel_e[s];
            }
        }
        if (p.selector) {
            // x . selector (candle's f32 gemm order is not visible; a tree
            // reduction is used), then sigmoid = 1 / (exp(-v) + 1)
            float part = 0.f;
            for (int64_t h = lane; h < p.H; h += 64) part = part + p.x[t * p.H + h] * p.selector[h];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
            if (lane == 0) p.sgate[t] = __fdiv_rn(1.f, exp_f32(-part) + 1.f);
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
        p.out[(int64_t)t * p.H + nn] = acc;
    }
}

// ------------------------------------------------------------- launchers
template <int GFMT, int DFMT>
hipError_t launch_gd(const MoeParams& p, hipStream_t s) {
    constexpr int GAF = GFMT == kQ8_0 ? kQ8_0 : kQ4_K;  // activation format of x
    constexpr int DAF = DFMT == kQ8_0 ? kQ8_0 : kQ4_K;  // activation format of act
    const int gmax = p.M * (int)p.K + 1;
    const unsigned tilesI = (unsigned)((p.I + 31) / 32);
    const unsigned groupsH = (unsigned)((p.H + 7) / 8);
    if (p.M == 1) {
        hipLaunchKernelGGL((k_moe_gate_up<GFMT, DAF, 1, GFMT == kQ8_0 ? 4 : 8>), dim3(tilesI, gmax), dim3(256), 0, s, p);
        if (hipError_t e = hipGetLastError()) return e;
        hipLaunchKernelGGL((k_moe_down<DFMT, 1, 3, 2>), dim3(groupsH), dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((k_moe_gate_up<GFMT, DAF, 8, GFMT == kQ8_0 ? 2 : 4>), dim3(tilesI, gmax), dim3(256), 0, s, p);
        if (hipError_t e = hipGetLastError()) return e;
        hipLaunchKernelGGL((k_moe_down<DFMT, 8, 2, 2>), dim3(groupsH), dim3(256), 0, s, p);
    }
    (void)GAF;
    return hipGetLastError();
}

template <int GFMT>
hipError_t launch_g(const MoeParams& p, int dfmt, hipStream_t s) {
    switch (dfmt) {
    case kQ4_K: return launch_gd<GFMT, kQ4_K>(p, s);
    case kQ6_K: return launch_gd<GFMT, kQ6_K>(p, s);
    case kQ8_0: return launch_gd<GFMT, kQ8_0>(p, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_moe(const MoeParams& p, int gfmt, int dfmt, hipStream_t s) {
    const int64_t qwaves = (int64_t)p.M * p.xq.ng;
    const unsigned prep_blocks = 1 + (unsigned)((qwaves + 3) / 4);
    if (gfmt == kQ8_0) hipLaunchKernelGGL((k_moe_prep<kQ8_0>), dim3(prep_blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((k_moe_prep<kQ4_K>), dim3(prep_blocks), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    switch (gfmt) {
    case kQ4_K: return launch_g<kQ4_K>(p, dfmt, s);
    case kQ6_K: return launch_g<kQ6_K>(p, dfmt, s);
    case kQ8_0: return launch_g<kQ8_0>(p, dfmt, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace iq
