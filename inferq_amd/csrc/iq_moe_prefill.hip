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
//   k_mp_route    three waves per token: top-k and routing weights, shared
//                 gate, softmax denominator;
//                 other workgroups quantise x (Q8K, activation layout).
//   k_mp_group    one workgroup: per-expert token bitmasks give counts,
//                 groups (experts ascending), each (token, route)'s position
//                 (its rank among the expert's tokens) and a list of 16-row
//                 chunks of every group, the shared expert's last.
//   k_mp_mm<0>    per (chunk, 32 intermediate rows): gate and up tiles of
//                 the chunk's tokens, SwiGLU into act.
//   k_mp_actq     act rows quantised (Q8K) for the down products.
//   k_mp_mm<1>    per (chunk, 64 hidden rows): down products into vals;
//                 on request k_mp_down_res (intermediate 512) or
//                 k_mp_down_tiles instead, per (chunk of up to 32 rows, 128
//                 or 64 hidden rows), in tile order (within 1e-4).
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
// Tokens per routing workgroup: wave 3i routes token i, wave 3i + 1 forms
// its shared-expert gate, wave 3i + 2 its softmax denominator.  Few tokens
// per workgroup keep the serial chains (top-k rounds, the index-order
// softmax sum) on separate SIMDs: 11.9 us for 256 tokens at sixteen tokens
// per workgroup, one wave each, against 8.9 at four.
constexpr int kMpRouteTok = 4;
// Chunks of one 16-row MFMA tile: at prefill widths most groups are small
// (Dirichlet(0.3) routing at 256 tokens: two thirds of the hit experts get
// 16 tokens or fewer), and the exact tile's work is mostly per output (the
// eight lane chains), so 16-row chunks waste less on padding than 32-row
// ones cost in repeated weight decode (the call: 184 -> 167 us).
constexpr int kMpRT = 1;  // 16-row MFMA tiles per chunk
static_assert(kMpRows == 16 * kMpRT, "chunk rows");
constexpr int kMpTileRT = kMpTileRows / 16;  // 16-row tiles per chunk of the tile-order down
#ifndef IQ_MP_RES_CT
#define IQ_MP_RES_CT 2
#endif
// Tiles of 64 hidden rows per workgroup of k_mp_down_res.  With chunks of
// 32 rows and two tiles per workgroup (136 VGPRs, 48 KB of LDS: three
// workgroups per CU) a 256-token call took 128.5 us, against 131.3-134.4 us
// for 64-row chunks with 1-8 tiles (fewer decodes of each expert's weights,
// but two workgroups per CU) and 131.7 us for 32-row chunks with 4 tiles.
constexpr int kMpResCT = IQ_MP_RES_CT;

// ------------------------------------------------------------ routing
__global__ __launch_bounds__(kMpThreads) void k_mp_route(MoeParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nr = (p.M + kMpRouteTok - 1) / kMpRouteTok;
    if ((int)blockIdx.x < nr) {
        // token i of the workgroup: wave 3i its top-k and then its weights,
        // wave 3i + 1 its shared-expert gate, wave 3i + 2 the softmax
        // denominator meanwhile (it does not depend on the selection)
        __shared__ __align__(16) float s_ev[kMpRouteTok][kMoeMaxExperts];
        __shared__ int s_sel[kMpRouteTok][kMoeMaxTopK];
        __shared__ float s_w[kMpRouteTok][kMoeMaxTopK];
        __shared__ float s_den[kMpRouteTok];
        const int ti = wave / 3, role = wave - 3 * ti;
        const int t = (int)blockIdx.x * kMpRouteTok + ti;
        if (ti >= kMpRouteTok) return;  // (a wave that has ended is not waited for at a barrier)
        const int E = (int)p.E, K = (int)p.K;
        if (role == 1) {
            if (p.selector && t < p.M) {
                const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
                if (lane == 0) p.sgate[t] = gate;
            }
            return;
        }
        float lv[kRoutePer];
        if (t < p.M) route_load(p.logits + (int64_t)t * E, E, lv);
        if (t < p.M && role == 2) {
            const float den = route_softmax_den(lv, E, s_ev[ti]);
            if (lane == 0) s_den[ti] = den;
        } else if (t < p.M) {
            route_topk_each_any(lv, E, K, [&](int s, int e) {
                if (lane == 0) {
                    p.experts[t * K + s] = e;
                    s_sel[ti][s] = e;
                }
            });
        }
        lds_barrier();  // the top-k and denominator waves of every token
        if (role != 0 || t >= p.M) return;
        route_pick_weights(s_den[ti], K, s_sel[ti], p.normalize, s_ev[ti], s_w[ti]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < K) p.weights[t * K + lane] = s_w[ti][lane];
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
// Exclusive prefix sums over the 1024 threads of N per-thread values; tot
// receives the totals.
template <int N>
__device__ __forceinline__ void block_scan(int (&v)[N], int* s_tmp /* [N][16] */, int (&tot)[N]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc[N];
#pragma unroll
    for (int i = 0; i < N; i++) inc[i] = v[i];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < N; i++) {
            const int x = __shfl_up(inc[i], off);
            if (lane >= off) inc[i] += x;
        }
    }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < N; i++) s_tmp[16 * i + wave] = inc[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; i++) {
        int base = 0;
        tot[i] = 0;
        for (int w = 0; w < kMpThreads / 64; w++) {
            if (w < wave) base += s_tmp[16 * i + w];
            tot[i] += s_tmp[16 * i + w];
        }
        v[i] = base + inc[i] - v[i];
    }
}

// The 16-row chunk list is ordered by the work of a chunk: the shared
// expert's full chunks, the routed groups' full chunks, then the partial
// chunks by descending row count.  A chunk's workgroups run 13-17 us (one
// per column tile) and the launch runs about four rounds of them per CU, so
// the long ones go first and the short ones fill the last round (the order
// changes which rows share a launch round, never a result).
__global__ __launch_bounds__(kMpThreads) void k_mp_group(MoeParams p) {
    extern __shared__ uint32_t s_mask[];  // [E][mw] token bitmask of each expert
    __shared__ int s_start[kMoeMaxExperts];
    __shared__ int s_tmp[64];
    __shared__ int s_pcnt[kMpRows], s_pbase[kMpRows], s_pnext[kMpRows];  // partial chunks by rows
    __shared__ int s_t1;  // tile-order chunks of one 16-row tile placed so far
    const int tid = threadIdx.x;
    const int E = (int)p.E, K = (int)p.K, M = p.M, NA = M * K, mw = (M + 31) / 32;
    for (int i = tid; i < E * mw; i += kMpThreads) s_mask[i] = 0;
    if (tid < kMpRows) s_pcnt[tid] = s_pnext[tid] = 0;
    if (tid == 0) s_t1 = 0;
    __syncthreads();
    for (int a = tid; a < NA; a += kMpThreads) {
        const int t = a / K, e = p.experts[a];
        atomicOr(&s_mask[e * mw + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    int cnt = 0;
    if (tid < E)
        for (int w = 0; w < mw; w++) cnt += __popc(s_mask[tid * mw + w]);
    const int nfull = cnt / kMpRows, rpart = cnt % kMpRows;  // full chunks, rows of the partial one (0: none)
    // tile-order chunks: those of two 16-row tiles (full, or more than 16
    // rows) first, then those of one
    const int tpart = cnt % kMpTileRows;
    const int nt2 = cnt / kMpTileRows + (tpart > 16 ? 1 : 0), nt1 = tpart > 0 && tpart <= 16 ? 1 : 0;
    // group id, first grouped row, first full chunk, first two-tile tile-order chunk
    int sv[4] = {cnt > 0, cnt, nfull, nt2}, tot[4];
    block_scan<4>(sv, s_tmp, tot);
    const int gid = sv[0], start = sv[1], cfs = sv[2], tst = sv[3];
    const int n_routed = tot[0], routed_full = tot[2], routed_t2 = tot[3];
    const bool has_shared = p.sgate_w != nullptr;
    const int sfull = has_shared ? M / kMpRows : 0, spart = has_shared ? M % kMpRows : 0;
    const int stpart = has_shared ? M % kMpTileRows : 0;
    const int snt2 = has_shared ? M / kMpTileRows + (stpart > 16 ? 1 : 0) : 0;
    const int snt1 = stpart > 0 && stpart <= 16 ? 1 : 0;
    const int t1base = routed_t2 + snt2;  // the one-tile chunks follow every two-tile chunk
    if (tid < E && rpart > 0) atomicAdd(&s_pcnt[rpart], 1);
    if (tid == 0 && spart > 0) atomicAdd(&s_pcnt[spart], 1);
    __syncthreads();
    if (tid == 0) {
        int b = sfull + routed_full;
        for (int r = kMpRows - 1; r >= 1; r--) {
            s_pbase[r] = b;
            b += s_pcnt[r];
        }
        s_pbase[0] = b;  // the number of chunks
    }
    __syncthreads();
    if (tid < E) {
        s_start[tid] = start;
        if (cnt > 0) {
            p.group_expert[gid] = tid;
            p.group_start[gid] = start;
            p.group_count[gid] = cnt;
            for (int j = 0; j < nfull; j++) {
                p.chunk_group[sfull + cfs + j] = gid;
                p.chunk_r0[sfull + cfs + j] = kMpRows * j;
            }
            if (rpart > 0) {
                const int c = s_pbase[rpart] + atomicAdd(&s_pnext[rpart], 1);
                p.chunk_group[c] = gid;
                p.chunk_r0[c] = kMpRows * nfull;
            }
            for (int j = 0; j < nt2; j++) {
                p.tchunk_group[tst + j] = gid;
                p.tchunk_r0[tst + j] = kMpTileRows * j;
            }
            if (nt1) {
                const int c = t1base + atomicAdd(&s_t1, 1);
                p.tchunk_group[c] = gid;
                p.tchunk_r0[c] = kMpTileRows * nt2;
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
    if (has_shared) {
        for (int t = tid; t < M; t += kMpThreads) p.assign_row[NA + t] = t;
        if (tid == 0) {
            p.group_expert[n_routed] = E;
            p.group_start[n_routed] = NA;
            p.group_count[n_routed] = M;
            if (spart > 0) {
                const int c = s_pbase[spart] + atomicAdd(&s_pnext[spart], 1);
                p.chunk_group[c] = n_routed;
                p.chunk_r0[c] = kMpRows * sfull;
            }
        }
        for (int j = tid; j < sfull; j += kMpThreads) {
            p.chunk_group[j] = n_routed;
            p.chunk_r0[j] = kMpRows * j;
        }
        for (int j = tid; j < snt2; j += kMpThreads) {
            p.tchunk_group[routed_t2 + j] = n_routed;
            p.tchunk_r0[routed_t2 + j] = kMpTileRows * j;
        }
        if (tid == 0 && snt1) {
            const int c = t1base + atomicAdd(&s_t1, 1);
            p.tchunk_group[c] = n_routed;
            p.tchunk_r0[c] = kMpTileRows * snt2;
        }
    }
    if (tid == 0) {
        p.meta[0] = n_routed + (has_shared ? 1 : 0);
        p.meta[1] = s_pbase[0];
        p.meta[2] = t1base + s_t1;
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
    // uniform per workgroup; Q5_K has no pair-lane form and takes the
    // 16-row tile for every chunk
    const bool pk = FMT != kQ5_K && rows <= 8;
    if (pk) {
        if constexpr (FMT != kQ5_K) {
            ((uint32_t*)zero)[threadIdx.x & 63] = 0u;  // read only after the product's first barrier
            float vp[4];
            ml_product_pk<FMT>(op, arow, brow, (uint8_t (*)[LP::END])lds, zero, vp);
#pragma unroll
            for (int r = 0; r < 4 * kMpRT; r++) v[r] = r < 4 ? vp[r] : 0.f;
        }
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

// Down products in tile order (on request: the outputs are not quantised
// again, so the per-lane f32 order is not needed for the rounding of a
// later stage).  A workgroup owns one chunk of up to kMpTileRows grouped
// rows of one group; each block of the expert's down rows is decoded once
// for all of them.  The chunk's row count picks, once per workgroup, a body
// compiled for that many 16-row tiles (NT), so no tile is skipped by a
// branch inside the product.
struct MpChunk {
    int rows, pos0;
    const uint8_t* w;  // the group's down matrix
};

__device__ __forceinline__ MpChunk mp_tile_chunk(const MoeParams& p, int c) {
    const int g = __builtin_amdgcn_readfirstlane(p.tchunk_group[c]);
    const int r0 = __builtin_amdgcn_readfirstlane(p.tchunk_r0[c]);
    const int e = __builtin_amdgcn_readfirstlane(p.group_expert[g]);
    MpChunk k;
    k.rows = min(kMpTileRows, __builtin_amdgcn_readfirstlane(p.group_count[g]) - r0);
    k.pos0 = __builtin_amdgcn_readfirstlane(p.group_start[g]) + r0;
    k.w = e == (int)p.E ? p.sdown_w : p.down + (int64_t)e * p.d_exp_bytes;
    return k;
}

// Grid (tiles of 64 hidden rows, tile-chunk bound), the activations staged
// per block beside the weights (any intermediate width).
template <int FMT, int NT>
__device__ __forceinline__ void mp_down_tiles_body(const MoeParams& p, const MpChunk& k, uint8_t* lds) {
    using L = MlStage<FMT, kMpTileRT>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    MlOperands op;
    op.aq = p.aq.q;
    op.ldq = p.aq.ldq;
    op.ad = p.aq.d;
    op.ldd = p.aq.ldd;
    op.hs = p.ahs;
    op.nb = p.d_nbw;
    op.brow_bytes = p.d_row_bytes;
    op.b0 = op.b1 = k.w;
    op.bsplit = kMlCols;
    auto brow = [&](int t) -> int64_t { return min((int64_t)blockIdx.x * kMlCols + t, p.H - 1); };
    auto arow = [&](int rr) -> int64_t { return (int64_t)(k.pos0 + min(rr, k.rows - 1)); };
    float v[4 * kMpTileRT];
    ml_product_tiles<FMT, kMpTileRT, NT>(op, arow, brow, (uint8_t (*)[L::END])lds, v);
    const int64_t n = (int64_t)blockIdx.x * kMlCols + 16 * wave + jj;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 16 * t + 4 * q + r;
            if (rr < k.rows && n < p.H) p.vals[(int64_t)(k.pos0 + rr) * p.H + n] = v[4 * t + r];
        }
}

template <int FMT>
__global__ __launch_bounds__(256) void k_mp_down_tiles(MoeParams p) {
    using L = MlStage<FMT, kMpTileRT>;
    __shared__ __align__(16) uint8_t lds[2 * L::END];
    const int c = blockIdx.y;
    if (c >= p.meta[2]) return;  // whole workgroup
    const MpChunk k = mp_tile_chunk(p, c);
    switch ((k.rows + 15) >> 4) {
        case 1: mp_down_tiles_body<FMT, 1>(p, k, lds); break;
        case 2: mp_down_tiles_body<FMT, (kMpTileRT < 2 ? kMpTileRT : 2)>(p, k, lds); break;
        case 3: mp_down_tiles_body<FMT, (kMpTileRT < 3 ? kMpTileRT : 3)>(p, k, lds); break;
        default: mp_down_tiles_body<FMT, kMpTileRT>(p, k, lds); break;
    }
}

// The same products with the chunk's activations resident, for down
// products of NB blocks (intermediate 256 NB): a workgroup owns one chunk
// and NCT consecutive tiles of 64 hidden rows.  The chunk's activation rows,
// scales and 16-value sums of every block are staged in LDS once; the
// expert's weight blocks stream through two stages, column tile after
// column tile, one stage loading while the other is decoded.
template <int NB, int FMT>
struct MpResident {
    static constexpr int R = kMpTileRows;
    static constexpr int A = 0;                                     // [NB][R][kMlAS] int8
    static constexpr int D = A + NB * R * kMlAS;                    // [NB][R] f32
    static constexpr int H = D + NB * R * 4;                        // [NB][R][16] f16 (Q4_K)
    static constexpr int B = H + (FMT == kQ4_K ? NB * R * 32 : 0);  // [2][64][BS]
    static constexpr int BST = kMlCols * MlFmt<FMT>::BS;
    static constexpr int END = B + 2 * BST;
};

template <int FMT, int NB, int NCT, int NT>
__device__ __forceinline__ void mp_down_res_body(const MoeParams& p, const MpChunk& k, uint8_t* lds) {
    using F = MlFmt<FMT>;
    using Lr = MpResident<NB, FMT>;
    constexpr int R = kMpTileRows, rows_live = 16 * NT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * (kMlCols * NCT);

    // ---- weight stages: stage s = (column tile s / NB, block s % NB)
    constexpr int kB = kMlCols * F::NL, kBPer = (kB + 255) / 256;
    uint32_t b_src[kBPer];
    int b_off[kBPer];
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kB - 1);
        const int c2 = t / F::NL, part = t - c2 * F::NL;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        b_src[i] = (uint32_t)(c2 * p.d_row_bytes + po);
        b_off[i] = (int)threadIdx.x + 256 * i < kB ? c2 * F::BS + po : -1;
    }
    u32x4 sb[2][kBPer];  // two stages of weight loads in flight
    auto issue = [&](int s) {
        const int ct = s / NB, b = s - ct * NB;
        // the launch keeps every tile inside the matrix (H % (64 NCT) == 0)
        const int64_t boff = FMT == kQ6_K ? ((int64_t)b * F::BB) & ~(int64_t)3 : (int64_t)b * F::BB;
        const uint8_t* src = k.w + (n0 + (int64_t)kMlCols * ct) * p.d_row_bytes + boff;
#pragma unroll
        for (int i = 0; i < kBPer; i++) sb[s & 1][i] = *(const u32x4*)(src + b_src[i]);
    };
    auto park = [&](int s) {
        uint8_t* st = lds + Lr::B + (s & 1) * Lr::BST;
#pragma unroll
        for (int i = 0; i < kBPer; i++)
            if (b_off[i] >= 0) *(u32x4*)(st + b_off[i]) = sb[s & 1][i];
    };
    constexpr int NS = NCT * NB;
    // ---- the chunk's activations, once: NB blocks x 16 NT rows x 16
    // granules, the scales (threads 0 .. NB R - 1) and the 16-value sums
    // (Q4_K: threads 0 .. 2 NB R - 1 over two passes); the first two weight
    // stages are issued behind their loads, so that storing the activations
    // waits for them alone
    {
        constexpr int kAG = NB * rows_live * 16, kAPer = (kAG + 255) / 256;
        v4i_ml sa[kAPer];
#pragma unroll
        for (int i = 0; i < kAPer; i++) {
            const int t = min((int)threadIdx.x + 256 * i, kAG - 1);
            const int b = t / (rows_live * 16), rr = (t >> 4) % rows_live, part = t & 15;
            sa[i] = *(const v4i_ml*)(p.aq.q + (int64_t)(k.pos0 + min(rr, k.rows - 1)) * p.aq.ldq + b * 256 + 16 * part);
        }
        float sd = 0.f;
        const int tb = (int)threadIdx.x / R, tr = (int)threadIdx.x % R;
        if ((int)threadIdx.x < NB * R) sd = p.aq.d[(int64_t)(k.pos0 + min(tr, k.rows - 1)) * p.aq.ldd + tb];
        v4i_ml sh16[2] = {};
        if constexpr (FMT == kQ4_K)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = (int)threadIdx.x + 256 * i;  // NB R rows x 2 halves
                const int hb = t / (2 * R), hr = (t >> 1) % R;
                if (t < 2 * NB * R)
                    sh16[i] = *(const v4i_ml*)(p.ahs + ((int64_t)(k.pos0 + min(hr, k.rows - 1)) * NB + hb) * 16 +
                                               8 * (t & 1));
            }
        issue(0);
        if (NS > 1) issue(1);
#pragma unroll
        for (int i = 0; i < kAPer; i++) {
            const int t = (int)threadIdx.x + 256 * i;
            const int b = t / (rows_live * 16), rr = (t >> 4) % rows_live, part = t & 15;
            if (t < kAG) *(v4i_ml*)(lds + Lr::A + (b * R + rr) * kMlAS + 16 * part) = sa[i];
        }
        if ((int)threadIdx.x < NB * R) *(float*)(lds + Lr::D + 4 * threadIdx.x) = sd;
        if constexpr (FMT == kQ4_K)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = (int)threadIdx.x + 256 * i;
                if (t < 2 * NB * R) *(v4i_ml*)(lds + Lr::H + 16 * t) = sh16[i];
            }
    }

    park(0);
    lds_barrier();
    const int col = 16 * wave + jj;
    float o[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) o[t][r] = 0.f;
    // stage s: its weights were parked at the end of stage s - 1; the loads
    // of s + 1 and s + 2 are in flight while it is decoded
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if (s + 2 < NS) issue(s + 2);
        const int ct = s / NB, b = s - ct * NB;
        const uint8_t* sa = lds + Lr::A + b * R * kMlAS;
        const uint8_t* sb = lds + Lr::B + (s & 1) * Lr::BST + col * F::BS;
        const float* sd = (const float*)(lds + Lr::D) + b * R;
        const uint8_t* sh16 = lds + Lr::H + b * R * 32;
        if (FMT == kQ6_K && (b & 1))  // block b of a row sits at shift 2 (b & 1)
            ml_tile_block<FMT, NT>(sa, sb, sd, sh16, MlShift<2>{}, q, jj, o);
        else
            ml_tile_block<FMT, NT>(sa, sb, sd, sh16, MlShift<0>{}, q, jj, o);
        if (b == NB - 1) {
            const int64_t n = n0 + (int64_t)kMlCols * ct + col;
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int rr = 16 * t + 4 * q + r;
                    if (rr < k.rows) p.vals[(int64_t)(k.pos0 + rr) * p.H + n] = o[t][r];
                    o[t][r] = 0.f;
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (s + 1 < NS) park(s + 1);
        lds_barrier();
    }
}

template <int FMT, int NB, int NCT>
__global__ __launch_bounds__(256) void k_mp_down_res(MoeParams p) {
    using Lr = MpResident<NB, FMT>;
    static_assert(Lr::END <= 160 * 1024, "LDS");
    __shared__ __align__(16) uint8_t lds[Lr::END];
    const int c = blockIdx.y;
    if (c >= p.meta[2]) return;  // whole workgroup
    const MpChunk k = mp_tile_chunk(p, c);
    switch ((k.rows + 15) >> 4) {
        case 1: mp_down_res_body<FMT, NB, NCT, 1>(p, k, lds); break;
        case 2: mp_down_res_body<FMT, NB, NCT, (kMpTileRT < 2 ? kMpTileRT : 2)>(p, k, lds); break;
        case 3: mp_down_res_body<FMT, NB, NCT, (kMpTileRT < 3 ? kMpTileRT : 3)>(p, k, lds); break;
        default: mp_down_res_body<FMT, NB, NCT, kMpTileRT>(p, k, lds); break;
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
    if constexpr (DFMT == kQ4_K || DFMT == kQ5_K)  // the down products' mins
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
    if constexpr (DFMT == kQ5_K) {  // no tile-order form: the exact products on either path
        hipLaunchKernelGGL((k_mp_mm<DFMT, 1>), dim3((unsigned)((p.H + kMlCols - 1) / kMlCols), (unsigned)p.max_chunks),
                           dim3(256), 0, s, p);
    } else if (p.down_tiles && p.d_nbw == 2 && p.H % (kMlCols * kMpResCT) == 0)
        hipLaunchKernelGGL((k_mp_down_res<DFMT, 2, kMpResCT>), dim3((unsigned)(p.H / (kMlCols * kMpResCT)),
                           (unsigned)p.max_tchunks), dim3(256), 0, s, p);
    else if (p.down_tiles)
        hipLaunchKernelGGL((k_mp_down_tiles<DFMT>), dim3((unsigned)((p.H + kMlCols - 1) / kMlCols), (unsigned)p.max_tchunks),
                           dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((k_mp_mm<DFMT, 1>), dim3((unsigned)((p.H + kMlCols - 1) / kMlCols), (unsigned)p.max_chunks),
                           dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(k_mp_combine, dim3((unsigned)((p.H + 1023) / 1024), (unsigned)M), dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    if (ev) (void)hipEventRecord(ev[3], s);
    return hipSuccess;
}

}  // namespace

int moep_max_chunks(int64_t M, int64_t K, int64_t E, int rows) {
    // sum over groups of ceil(count / rows) <= grouped rows / rows + groups
    const int64_t P = M * K + M;
    return (int)(P / rows + std::min(E, M * K) + 2);
}

bool moep_supported(const MoeParams& p, int gfmt, int dfmt) {
    const bool kq = (gfmt == kQ4_K || gfmt == kQ5_K || gfmt == kQ6_K) && (dfmt == kQ4_K || dfmt == kQ5_K || dfmt == kQ6_K);
    auto al = [](const void* q, uintptr_t a) { return q == nullptr || ((uintptr_t)q & (a - 1)) == 0; };
    const uintptr_t ga = gfmt == kQ6_K ? 4 : 16, da = dfmt == kQ6_K ? 4 : 16;
    const bool aligned = al(p.gate, ga) && al(p.up, ga) && al(p.sgate_w, ga) && al(p.sup_w, ga) && al(p.down, da) &&
                         al(p.sdown_w, da) && al(p.out, 16) &&
                         al(p.residual, 16);  // k_mp_combine moves four floats at a time
    return kq && aligned && p.M >= kMoePrefillMinTokens && p.H % 256 == 0 && p.I % 256 == 0 && p.E <= kMoeMaxExperts &&
           p.K <= kMoeMaxTopK && p.g_row_bytes % 4 == 0 && p.d_row_bytes % 4 == 0 &&
           (int64_t)p.E * ((p.M + 31) / 32) * 4 <= 32768 && p.xhs != nullptr && p.chunk_group != nullptr &&
           ((dfmt != kQ4_K && dfmt != kQ5_K) || p.ahs != nullptr);
}

hipError_t launch_moe_prefill(const MoeParams& p, int gfmt, int dfmt, hipStream_t s, hipEvent_t const* ev) {
    if (!moep_supported(p, gfmt, dfmt)) return hipErrorNotSupported;
    if (gfmt == kQ4_K && dfmt == kQ6_K) return launch_p<kQ4_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ4_K && dfmt == kQ4_K) return launch_p<kQ4_K, kQ4_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ6_K) return launch_p<kQ6_K, kQ6_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ4_K) return launch_p<kQ6_K, kQ4_K>(p, s, ev);
    if (gfmt == kQ4_K && dfmt == kQ5_K) return launch_p<kQ4_K, kQ5_K>(p, s, ev);
    if (gfmt == kQ6_K && dfmt == kQ5_K) return launch_p<kQ6_K, kQ5_K>(p, s, ev);
    if (gfmt == kQ5_K && dfmt == kQ4_K) return launch_p<kQ5_K, kQ4_K>(p, s, ev);
    if (gfmt == kQ5_K && dfmt == kQ5_K) return launch_p<kQ5_K, kQ5_K>(p, s, ev);
    if (gfmt == kQ5_K && dfmt == kQ6_K) return launch_p<kQ5_K, kQ6_K>(p, s, ev);
    return hipErrorNotSupported;
}

}  // namespace iq
