// iq_moe_prefill.hip -- the MoE sublayer for many tokens (prefill widths),
// grouped by expert (routed_grouped_by_expert, src/qwen/quantized_moe.rs:
// 336-460), with the expert products on int8 MFMA in the reference's exact
// per-lane order: every token's output is bitwise what a one-token call
// gives.
//
// The expert products are the exact lane-order MFMA tiles of
// iq_mfma_lanes.h, so the bit pattern of every output matches the
// reference's per-lane FMA chains.
//
// Six launches per call:
//   k_mp_route    two waves per token: top-k and routing weights, shared gate;
//                 other workgroups quantise x (Q8K, activation layout).
//   k_mp_group    one workgroup: per-expert token bitmasks give counts,
//                 groups (experts ascending), each (token, route)'s position
//                 (its rank among the expert's tokens) and a list of 16-row
//                 chunks of every group, the shared expert's last.
//   k_mp_mm<0>    per (chunk, 32 intermediate rows): gate and up tiles of
//                 the chunk's tokens, SwiGLU into act.
//   k_mp_actq     act rows quantised (Q8K) for the down products.
//   k_mp_mm<1>    per (chunk, 64 hidden rows): down products into vals.
//   k_mp_combine  routes in order (multiply, then add), then shared * gate.
#include <type_traits>

#include "iq_lanes.h"
#include "iq_mfma_lanes.h"
#include "iq_moe.h"
#include "iq_quant.h"
#include "iq_route.h"

namespace iq {

namespace {

constexpr int kMpThreads = 1024;  // routing and grouping workgroups
// Tokens per routing workgroup: wave 2i routes token i, wave 2i + 1 forms
// its shared-expert gate.  Four tokens keep the serial chains (top-k rounds,
// the index-order softmax sum) on separate SIMDs: 11.9 us for 256 tokens at
// sixteen tokens per workgroup, one wave each, against 8.9 at four.
constexpr int kMpRouteTok = 4;
// Chunks of one 16-row MFMA tile: at prefill widths most groups are small
// (Dirichlet(0.3) routing at 256 tokens: two thirds of the hit experts get
// 16 tokens or fewer), and the exact tile's work is mostly per output (the
// eight lane chains), so 16-row chunks waste less on padding than 32-row
// ones cost in repeated weight decode (the call: 184 -> 167 us).
constexpr int kMpRT = 1;             // 16-row MFMA tiles per chunk
constexpr int kMpRows = 16 * kMpRT;  // grouped rows per chunk

// ------------------------------------------------------------ routing
__global__ __launch_bounds__(kMpThreads) void k_mp_route(MoeParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nr = (p.M + kMpRouteTok - 1) / kMpRouteTok;
    if ((int)blockIdx.x < nr) {
        __shared__ __align__(16) float s_ev[kMpRouteTok][kMoeMaxExperts];
        const int t = (int)blockIdx.x * kMpRouteTok + (wave >> 1);
        if (wave >= 2 * kMpRouteTok || t >= p.M) return;
        if (wave & 1) {
            if (p.selector) {
                const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
                if (lane == 0) p.sgate[t] = gate;
            }
            return;
        }
        const int E = (int)p.E, K = (int)p.K;
        int sel[kMoeMaxTopK];
        float lv[kRoutePer], w[kMoeMaxTopK];
        route_topk<kMoeMaxTopK>(p.logits + (int64_t)t * E, E, K, sel, lv);
        if (lane == 0)
            for (int s = 0; s < K; s++) p.experts[t * K + s] = sel[s];
        route_weights<kMoeMaxTopK>(lv, E, K, sel, p.normalize, s_ev[wave >> 1], w);
        if (lane == 0)
            for (int s = 0; s < K; s++) p.weights[t * K + s] = w[s];
        return;
    }
    // x quantisation: one wave per (row, 256-value block)
    const int64_t wid = (int64_t)(blockIdx.x - nr) * 16 + wave;
    const int nb = p.xq.ng;
    if (wid >= (int64_t)p.M * nb) return;
    const int64_t row = wid / nb;
    const int b = (int)(wid - row * nb);
    const Q8KLane r = quant_q8k_core(load4(p.x + row * p.H + (int64_t)b * 256 + 4 * lane));
    ((uint32_t*)(p.xq.q + row * p.xq.ldq + (int64_t)b * 256))[perm_dword(lane >> 3, lane & 7)] = r.packed;
    if (lane == 0) p.xq.d[row * p.xq.ldd + b] = r.d;
    if ((lane & 3) == 0) p.xhs[(row * nb + b) * 16 + (lane >> 2)] = (_Float16)(float)r.bsum16;
}

// ----------------------------------------------------------- grouping
// Exclusive prefix sums over the 1024 threads of three per-thread values.
__device__ __forceinline__ void block_scan3(int& a, int& b, int& c, int* s_tmp /* [3][16] */, int& ta, int& tb,
                                            int& tc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int ia = a, ib = b, ic = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int xa = __shfl_up(ia, off), xb = __shfl_up(ib, off), xc = __shfl_up(ic, off);
        if (lane >= off) {
            ia += xa;
            ib += xb;
            ic += xc;
        }
    }
    if (lane == 63) {
        s_tmp[wave] = ia;
        s_tmp[16 + wave] = ib;
        s_tmp[32 + wave] = ic;
    }
    __syncthreads();
    int ba = 0, bb = 0, bc = 0;
    ta = tb = tc = 0;
    for (int w = 0; w < kMpThreads / 64; w++) {
        if (w < wave) {
            ba += s_tmp[w];
            bb += s_tmp[16 + w];
            bc += s_tmp[32 + w];
        }
        ta += s_tmp[w];
        tb += s_tmp[16 + w];
        tc += s_tmp[32 + w];
    }
    a = ba + ia - a;
    b = bb + ib - b;
    c = bc + ic - c;
}

__global__ __launch_bounds__(kMpThreads) void k_mp_group(MoeParams p) {
    extern __shared__ uint32_t s_mask[];  // [E][mw] token bitmask of each expert
    __shared__ int s_start[kMoeMaxExperts];
    __shared__ int s_tmp[48];
    const int tid = threadIdx.x;
    const int E = (int)p.E, K = (int)p.K, M = p.M, NA = M * K, mw = (M + 31) / 32;
    for (int i = tid; i < E * mw; i += kMpThreads) s_mask[i] = 0;
    __syncthreads();
    for (int a = tid; a < NA; a += kMpThreads) {
        const int t = a / K, e = p.experts[a];
        atomicOr(&s_mask[e * mw + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    int cnt = 0;
    if (tid < E)
        for (int w = 0; w < mw; w++) cnt += __popc(s_mask[tid * mw + w]);
    const int nch = (cnt + kMpRows - 1) / kMpRows;
    int gid = cnt > 0, start = cnt, cst = nch, n_routed, total, routed_chunks;
    block_scan3(gid, start, cst, s_tmp, n_routed, total, routed_chunks);
    if (tid < E) {
        s_start[tid] = start;
        if (cnt > 0) {
            p.group_expert[gid] = tid;
            p.group_start[gid] = start;
            p.group_count[gid] = cnt;
            for (int j = 0; j < nch; j++) {
                p.chunk_group[cst + j] = gid;
                p.chunk_r0[cst + j] = kMpRows * j;
            }
        }
    }
    __syncthreads();
    // position of (t, route): the expert's group start plus the number of
    // earlier tokens routed to it
    for (int a = tid; a < NA; a += kMpThreads) {
        const int t = a / K, e = p.experts[a];
        const uint32_t* m = s_mask + e * mw;
        int rank = __popc(m[t >> 5] & ((1u << (t & 31)) - 1u));
        for (int w = 0; w < (t >> 5); w++) rank += __popc(m[w]);
        const int pos = s_start[e] + rank;
        p.assign_row[pos] = t;
        p.slot_pos[a] = pos;
    }
    const bool has_shared = p.sgate_w != nullptr;
    const int sch = has_shared ? (M + kMpRows - 1) / kMpRows : 0;
    if (has_shared) {
        for (int t = tid; t < M; t += kMpThreads) p.assign_row[NA + t] = t;
        if (tid == 0) {
            p.group_expert[n_routed] = E;
            p.group_start[n_routed] = NA;
            p.group_count[n_routed] = M;
        }
        for (int j = tid; j < sch; j += kMpThreads) {
            p.chunk_group[routed_chunks + j] = n_routed;
            p.chunk_r0[routed_chunks + j] = kMpRows * j;
        }
    }
    if (tid == 0) {
        p.meta[0] = n_routed + (has_shared ? 1 : 0);
        p.meta[1] = routed_chunks + sch;
    }
}

// ------------------------------------------------------ expert products
// Grid (column tiles, chunk bound).  A workgroup owns one chunk (kMpRows
// grouped rows) and 64 weight rows (ml_product: wave w owns 16 of them and
// every 16-row tile of the chunk).  MODE 0: gate/up, weight rows i0 + 0..31 of
// gate (waves 0, 1) and of up (waves 2, 3), A the chunk's tokens of x;
// SwiGLU into act.  MODE 1: down, 64 hidden rows, A the chunk's act rows;
// results into vals.
template <int FMT, int MODE>
__global__ __launch_bounds__(256) void k_mp_mm(MoeParams p) {
    using L = MlStage<FMT, kMpRT>;
    using LP = MlStagePk<FMT>;
    constexpr int kStage = 2 * L::END > 2 * LP::END ? 2 * L::END : 2 * LP::END;
    __shared__ __align__(16) uint8_t lds[kStage + 256];
    auto st = (uint8_t (*)[L::END])lds;
    uint8_t* zero = lds + kStage;
    const int c = blockIdx.y;
    if (c >= p.meta[1]) return;  // whole workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int g = p.chunk_group[c], r0 = p.chunk_r0[c];
    const int e = p.group_expert[g], start = p.group_start[g];
    const int rows = min(kMpRows, p.group_count[g] - r0);
    const bool shared = e == (int)p.E;
    const int pos0 = start + r0;

    MlOperands op;
    const ActView& av = MODE == 0 ? p.xq : p.aq;
    op.aq = av.q;
    op.ldq = av.ldq;
    op.ad = av.d;
    op.ldd = av.ldd;
    op.hs = MODE == 0 ? p.xhs : p.ahs;
    op.nb = MODE == 0 ? p.g_nbw : p.d_nbw;  // weight blocks per row = activation blocks
    op.brow_bytes = MODE == 0 ? p.g_row_bytes : p.d_row_bytes;
    if constexpr (MODE == 0) {
        op.b0 = shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes;
        op.b1 = shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes;
        op.bsplit = 32;
    } else {
        op.b0 = op.b1 = shared ? p.sdown_w : p.down + (int64_t)e * p.d_exp_bytes;
        op.bsplit = kMlCols;
    }
    // weight row (within its matrix) of tile column t, clamped
    auto brow = [&](int t) -> int64_t {
        if constexpr (MODE == 0) return min((int64_t)blockIdx.x * 32 + (t & 31), p.I - 1);
        else return min((int64_t)blockIdx.x * kMlCols + t, p.H - 1);
    };
    // activation row of tile row rr (0..31), clamped to the chunk
    auto arow = [&](int rr) -> int64_t {
        const int pos = pos0 + min(rr, rows - 1);
        return MODE == 0 ? (int64_t)p.assign_row[pos] : (int64_t)pos;
    };
    // chunks of at most 8 rows take two reference lanes per MFMA; output r
    // of a lane is then row 4 (q & 1) + r (every lane group), else row
    // 16 (r / 4) + 4 q + r % 4
    float v[4 * kMpRT];
    const bool pk = rows <= 8;  // uniform per workgroup
    if (pk) {
        ((uint32_t*)zero)[threadIdx.x & 63] = 0u;  // read only after the product's first barrier
        float vp[4];
        ml_product_pk<FMT>(op, arow, brow, (uint8_t (*)[LP::END])lds, zero, vp);
#pragma unroll
        for (int r = 0; r < 4 * kMpRT; r++) v[r] = r < 4 ? vp[r] : 0.f;
    } else {
        ml_product<FMT, kMpRT>(op, arow, brow, st, v);
    }
    auto out_row = [&](int r) { return pk ? (r < 4 ? 4 * (q & 1) + r : kMpRows) : 16 * (r >> 2) + 4 * q + (r & 3); };
    const bool writer = !pk || q < 2;  // pair-lane tiles: lane groups 2, 3 repeat 0, 1

    if constexpr (MODE == 0) {
        // waves 2, 3 hold up of the columns waves 0, 1 hold gate of
        float* s_up = (float*)lds;  // [kMpRows][32]
        if (wave >= 2 && writer)
#pragma unroll
            for (int r = 0; r < 4 * kMpRT; r++) {
                const int rr = out_row(r);
                if (rr < kMpRows) s_up[rr * 32 + 16 * (wave - 2) + jj] = v[r];
            }
        lds_barrier();
        if (wave < 2 && writer) {
            const int64_t i = (int64_t)blockIdx.x * 32 + 16 * wave + jj;
#pragma unroll
            for (int r = 0; r < 4 * kMpRT; r++) {
                const int rr = out_row(r);
                if (rr < rows && i < p.I) {
                    const float u = s_up[rr * 32 + 16 * wave + jj];
                    // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
                    p.act[(int64_t)(pos0 + rr) * p.I + i] = __fdiv_rn(v[r], 1.f + exp_f32(-v[r])) * u;
                }
            }
        }
    } else {
        const int64_t n = (int64_t)blockIdx.x * kMlCols + 16 * wave + jj;
        if (writer)
#pragma unroll
            for (int r = 0; r < 4 * kMpRT; r++) {
                const int rr = out_row(r);
                if (rr < rows && n < p.H) p.vals[(int64_t)(pos0 + rr) * p.H + n] = v[r];
            }
    }
}

// ------------------------------------------- act quantisation, combine
// One wave per (grouped row, 256-value block) of act.
template <int DFMT>
__global__ __launch_bounds__(256) void k_mp_actq(MoeParams p, int P) {
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = p.aq.ng;
    if (wid >= (int64_t)P * nb) return;
    const int64_t row = wid / nb;
    const int b = (int)(wid - row * nb);
    const Q8KLane r = quant_q8k_core(load4(p.act + row * p.I + (int64_t)b * 256 + 4 * lane));
    ((uint32_t*)(p.aq.q + row * p.aq.ldq + (int64_t)b * 256))[perm_dword(lane >> 3, lane & 7)] = r.packed;
    if (lane == 0) p.aq.d[row * p.aq.ldd + b] = r.d;
    if constexpr (DFMT == kQ4_K)
        if ((lane & 3) == 0) p.ahs[(row * nb + b) * 16 + (lane >> 2)] = (_Float16)(float)r.bsum16;
}

// routed = sum over routes in order of value * weight, then hidden = routed
// + shared * gate (src/qwen/quantized_moe.rs:266-273, :384-400).  Grid
// (H / 1024, M): token t = blockIdx.y for the whole workgroup (its routes'
// positions and weights are scalar loads), four consecutive hidden columns
// per thread.
__global__ __launch_bounds__(256) void k_mp_combine(MoeParams p) {
    const int t = (int)blockIdx.y;
    const int64_t nn = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (nn >= p.H) return;
    const int K = (int)p.K;
    int pos[kMoeMaxTopK];
    float wt[kMoeMaxTopK];
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++) {
        pos[j] = j < K ? p.slot_pos[t * K + j] : 0;
        wt[j] = j < K ? p.weights[t * K + j] : 0.f;
    }
    f32x4 v[kMoeMaxTopK];
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++)
        if (j < K) v[j] = *(const f32x4*)(p.vals + (int64_t)pos[j] * p.H + nn);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kMoeMaxTopK; j++)
        if (j < K) {
            acc.x = acc.x + v[j].x * wt[j];
            acc.y = acc.y + v[j].y * wt[j];
            acc.z = acc.z + v[j].z * wt[j];
            acc.w = acc.w + v[j].w * wt[j];
        }
    if (p.sgate_w) {
        const f32x4 sv = *(const f32x4*)(p.vals + (int64_t)(p.M * K + t) * p.H + nn);
        const float gt = p.sgate[t];
        acc.x = acc.x + sv.x * gt;
        acc.y = acc.y + sv.y * gt;
        acc.z = acc.z + sv.z * gt;
        acc.w = acc.w + sv.w * gt;
    }
    if (p.residual) {  // src/qwen/quantized_layer.rs:212
        const f32x4 rv = *(const f32x4*)(p.residual + (int64_t)t * p.H + nn);
        acc.x = rv.x + acc.x;
        acc.y = rv.y + acc.y;
        acc.z = rv.z + acc.z;
        acc.w = rv.w + acc.w;
    }
    *(f32x4*)(p.out + (int64_t)t * p.H + nn) = acc;
}

template <int GFMT, int DFMT>
hipError_t launch_p(const MoeParams& p, hipStream_t s, hipEvent_t const* ev) {
    const int M = p.M, K = (int)p.K, nbH = p.xq.ng;
    const int P = M * K + (p.sgate_w ? M : 0);
    if (ev) (void)hipEventRecord(ev[0], s);
    const int nr = (M + kMpRouteTok - 1) / kMpRouteTok;
    const int64_t qw = (int64_t)M * nbH;
    hipLaunchKernelGGL(k_mp_route, dim3((unsigned)(nr + (qw + 15) / 16)), dim3(kMpThreads), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    const size_t mask_bytes = (size_t)p.E * ((M + 31) / 32) * 4;
    hipLaunchKernelGGL(k_mp_group, dim3(1), dim3(kMpThreads), mask_bytes, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[1], s);
    hipLaunchKernelGGL((k_mp_mm<GFMT, 0>), dim3((unsigned)(p.I / 32), (unsigned)p.max_chunks), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    const int64_t aw = (int64_t)P * p.aq.ng;
    hipLaunchKernelGGL((k_mp_actq<DFMT>), dim3((unsigned)((aw + 3) / 4)), dim3(256), 0, s, p, P);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[2], s);
    hipLaunchKernelGGL((k_mp_mm<DFMT, 1>), dim3((unsigned)((p.H + kMlCols - 1) / kMlCols), (unsigned)p.max_chunks),
                       dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(k_mp_combine, dim3((unsigned)((p.H + 1023) / 1024), (unsigned)M), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[3], s);
    return hipSuccess;
}

}  // namespace

int moep_max_chunks(int64_t M, int64_t K, int64_t E) {
    // sum over groups of ceil(count / 32) <= rows / 32 + groups
    const int64_t P = M * K + M;
    return (int)(P / kMpRows + std::min(E, M * K) + 2);
}

bool moep_supported(const MoeParams& p, int gfmt, int dfmt) {
    const bool kq = (gfmt == kQ4_K || gfmt == kQ6_K) && (dfmt == kQ4_K || dfmt == kQ6_K);
    auto al = [](const void* q, uintptr_t a) { return q == nullptr || ((uintptr_t)q & (a - 1)) == 0; };
    const uintptr_t ga = gfmt == kQ4_K ? 16 : 4, da = dfmt == kQ4_K ? 16 : 4;
    const bool aligned = al(p.gate, ga) && al(p.up, ga) && al(p.sgate_w, ga) && al(p.sup_w, ga) && al(p.down, da) &&
                         al(p.sdown_w, da) && al(p.out, 16) &&
                         al(p.residual, 16);  // k_mp_combine moves four floats at a time
    return kq && aligned && p.M >= kMoePrefillMinTokens && p.H % 256 == 0 && p.I % 256 == 0 && p.E <= kMoeMaxExperts &&
           p.K <= kMoeMaxTopK && p.g_row_bytes % 4 == 0 && p.d_row_bytes % 4 == 0 &&
           (int64_t)p.E * ((p.M + 31) / 32) * 4 <= 32768 && p.xhs != nullptr && p.chunk_group != nullptr &&
           (dfmt != kQ4_K || p.ahs != nullptr);
}

hipError_t launch_moe_prefill(const MoeParams& p, int gfmt, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    if (!moep_supported(p, gfmt, dfmt)) return hipErrorNotSupported;
    if (gfmt == kQ4_K && dfmt == kQ6_K) return launch_p<kQ4_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ4_K && dfmt == kQ4_K) return launch_p<kQ4_K, kQ4_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ6_K) return launch_p<kQ6_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ4_K) return launch_p<kQ6_K, kQ4_K>(p, s, ev);
    return hipErrorNotSupported;
}

}  // namespace iq
