// iq_moe_prefill.hip -- the MoE sublayer for many tokens (prefill widths),
// grouped by expert (routed_grouped_by_expert, src/qwen/quantized_moe.rs:
// 336-460), with the expert products on int8 MFMA in the reference's exact
// per-lane order: every token's output is bitwise what a one-token call
// gives.
//
// Exact lane order on MFMA.  The reference's lane k (src/qgemm.rs:175-346)
// owns bytes 4k..4k+3 of every 32-value chunk c of a block: isum_k =
// sum_c sc_c * dot4(w[c][k], a[c][k]) with one scale per dword, and it
// advances acc_k = fma(y.d * x.d, isum_k, acc_k) once per block; the eight
// lanes meet in hsum_f32_8 (Q4_K mins: four lanes, hsum_f32_4).  Int8
// MFMAs whose K index runs over (c, e) for one fixed k yield isum_k for a
// whole 16 x 16 tile: A holds the activation dwords (c, k),
// c = 0..7, which the activation layout keeps contiguous (dword 8k + c), and
// B the weight dwords (c, k) with each dword's scale folded in.  Scaled
// weights exceed int8, so each is split into two int8 streams whose integer
// sums recombine exactly: Q4_K sc*q = 8 (sc >> 3) q + (sc & 7) q; Q6_K
// sc*(q - 32) = 64 hi + lo with lo in 0..63 and hi in -64..64.  The Q4_K
// mins msum_k = m_2k s_2k + m_2k+1 s_2k+1 (s = 32-value activation sums)
// come from an f16 MFMA over the 16-value sums (integers below 2^24: exact).
// A lane keeps the f32 chains of all eight reference lanes for its eight
// outputs and joins them at the end in the hsum trees' order,
// ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) plus (m0+m2) + (m1+m3).
//
// Six launches per call:
//   k_mp_route    one wave per token: top-k, routing weights, shared gate;
//                 other workgroups quantise x (Q8K, activation layout).
//   k_mp_group    one workgroup: per-expert token bitmasks give counts,
//                 groups (experts ascending), each (token, route)'s position
//                 (its rank among the expert's tokens) and a list of 32-row
//                 chunks of every group, the shared expert's last.
//   k_mp_mm<0>    per (chunk, 32 intermediate rows): gate and up tiles of
//                 the chunk's tokens, SwiGLU into act.
//   k_mp_actq     act rows quantised (Q8K) for the down products.
//   k_mp_mm<1>    per (chunk, 64 hidden rows): down products into vals.
//   k_mp_combine  routes in order (multiply, then add), then shared * gate.
#include <type_traits>

#include "iq_lanes.h"
#include "iq_moe.h"
#include "iq_quant.h"
#include "iq_route.h"

namespace iq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kMpThreads = 1024;  // routing and grouping workgroups
constexpr int kMpRows = 32;       // grouped rows per chunk (one MFMA row tile)
constexpr int kMpCols = 64;       // weight rows per product workgroup (16 per wave)
constexpr int kMpAS = 272;        // LDS stride of an activation row (256 + pad)

// ------------------------------------------------------------ routing
__global__ __launch_bounds__(kMpThreads) void k_mp_route(MoeParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nr = (p.M + 15) / 16;
    if ((int)blockIdx.x < nr) {
        __shared__ __align__(16) float s_ev[16][kMoeMaxExperts];
        const int t = (int)blockIdx.x * 16 + wave;
        if (t >= p.M) return;
        const int E = (int)p.E, K = (int)p.K;
        int sel[kMoeMaxTopK];
        float lv[kRoutePer], w[kMoeMaxTopK];
        route_topk<kMoeMaxTopK>(p.logits + (int64_t)t * E, E, K, sel, lv);
        if (lane == 0)
            for (int s = 0; s < K; s++) p.experts[t * K + s] = sel[s];
        route_weights<kMoeMaxTopK>(lv, E, K, sel, p.normalize, s_ev[wave], w);
        if (lane == 0)
            for (int s = 0; s < K; s++) p.weights[t * K + s] = w[s];
        if (p.selector) {
            const float gate = selector_gate(p.x + (int64_t)t * p.H, p.selector, p.H);
            if (lane == 0) p.sgate[t] = gate;
        }
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
template <int FMT>
struct MpFmt;
template <>
struct MpFmt<kQ4_K> {
    static constexpr int BB = 144;  // block bytes
    static constexpr int BS = 144;  // LDS bytes per staged row-block
    static constexpr int NL = 9;    // staging loads per row-block (16 bytes each)
    static constexpr bool kMins = true;
};
template <>
struct MpFmt<kQ6_K> {
    static constexpr int BB = 210;
    static constexpr int BS = 224;  // the block's 212-byte dword window, padded
    static constexpr int NL = 14;   // staging loads per row-block (16 bytes each)
    static constexpr bool kMins = false;
};

// LDS stage: A int8 [32][kMpAS], B [64][BS], D f32 [32], H f16 [32][16]
template <int FMT>
struct MpStage {
    static constexpr int A = 0;
    static constexpr int B = A + kMpRows * kMpAS;
    static constexpr int D = B + kMpCols * MpFmt<FMT>::BS;
    static constexpr int H = D + kMpRows * 4;
    static constexpr int END = H + (MpFmt<FMT>::kMins ? kMpRows * 32 : 0);
};

// Bytes of q (each < 16) times s (< 8) byte by byte: every product is below
// 128, so two 16-bit lanes never carry into each other.
__device__ __forceinline__ uint32_t bytes_mul_small(uint32_t q, uint32_t s) {
    const u16x2 a = __builtin_bit_cast(u16x2, q);
    const u16x2 b = {(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, a * b);
}

// Four unsigned six-bit values u (bytes) times a signed scale sc, minus
// 32 sc: p = sc * (u - 32) in -4064..4096, split p = 64 hi + lo; returns the
// lo bytes (0..63) and the hi bytes (-64..64), byte order kept.
__device__ __forceinline__ void q6_scaled_split(uint32_t u, int sc, uint32_t& lo, uint32_t& hi) {
    const s16x2 s2 = {(short)sc, (short)sc}, m2 = {(short)(-32 * sc), (short)(-32 * sc)};
    const s16x2 u02 = __builtin_bit_cast(s16x2, u & 0x00ff00ffu);         // bytes 0, 2
    const s16x2 u13 = __builtin_bit_cast(s16x2, (u >> 8) & 0x00ff00ffu);  // bytes 1, 3
    const s16x2 p02 = u02 * s2 + m2, p13 = u13 * s2 + m2;
    const uint32_t l02 = __builtin_bit_cast(uint32_t, p02) & 0x003f003fu;
    const uint32_t l13 = __builtin_bit_cast(uint32_t, p13) & 0x003f003fu;
    lo = l02 | (l13 << 8);
    const s16x2 six = {6, 6};
    const uint32_t h02 = __builtin_bit_cast(uint32_t, (s16x2)(p02 >> six));
    const uint32_t h13 = __builtin_bit_cast(uint32_t, (s16x2)(p13 >> six));
    // bytes 0 and 2 of h02 and of h13, interleaved
    hi = __builtin_amdgcn_perm(h13, h02, 0x06020400u);
}

// The 4 bytes at byte offset o of a block staged with a dword shift of sh
// (0 or 2) bytes.
__device__ __forceinline__ uint32_t lds_win(const uint8_t* row, int sh, int o) {
    const uint32_t w0 = *(const uint32_t*)(row + o), w1 = *(const uint32_t*)(row + o + 4);
    return __builtin_amdgcn_alignbyte(w1, w0, (uint32_t)sh);
}

// Grid (column tiles, chunk bound).  A workgroup owns one chunk (32 grouped
// rows) and 64 weight rows; wave w owns 16 of them and both 16-row halves of
// the chunk (two 16 x 16 MFMA tiles).  MODE 0: gate/up, weight rows
// i0 + 0..31 of gate (waves 0, 1) and of up (waves 2, 3), A the chunk's
// tokens of x; SwiGLU into act.  MODE 1: down, 64 hidden rows, A the chunk's
// act rows; results into vals.
//
// Fragments of v_mfma_i32_16x16x32_i8 for lane l (q = l / 16, j = l % 16):
// A row j, K 8q..8q+7; B column j, the same K; the result holds rows
// 4q..4q+3 of column j.  For lane k of the reference, K 8q..8q+7 are the
// dwords (c, k) with c = 2q, 2q+1.
template <int FMT, int MODE>
__global__ __launch_bounds__(256) void k_mp_mm(MoeParams p) {
    using F = MpFmt<FMT>;
    using L = MpStage<FMT>;
    __shared__ __align__(16) uint8_t st[2][L::END];
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

    // operands of this call
    const ActView& av = MODE == 0 ? p.xq : p.aq;
    const _Float16* hsrc = MODE == 0 ? p.xhs : p.ahs;
    const int nb = MODE == 0 ? p.g_nbw : p.d_nbw;  // weight blocks per row = activation blocks
    const int64_t wrow_bytes = MODE == 0 ? p.g_row_bytes : p.d_row_bytes;

    // ---- staging: every thread owns fixed slots, the same for every block.
    // Sources are a wave-uniform base plus a 32-bit offset.
    const uint8_t* gbase = nullptr;  // matrix of staged columns 0..31 (MODE 0) or all
    const uint8_t* ubase = nullptr;  // matrix of staged columns 32..63 (MODE 0)
    if constexpr (MODE == 0) {
        gbase = shared ? p.sgate_w : p.gate + (int64_t)e * p.g_exp_bytes;
        ubase = shared ? p.sup_w : p.up + (int64_t)e * p.g_exp_bytes;
    } else {
        gbase = shared ? p.sdown_w : p.down + (int64_t)e * p.d_exp_bytes;
        ubase = gbase;
    }
    // weight row (within its matrix) of staged column t, clamped
    auto wrow = [&](int t) -> int64_t {
        if constexpr (MODE == 0) return min((int64_t)blockIdx.x * 32 + (t & 31), p.I - 1);
        else return min((int64_t)blockIdx.x * kMpCols + t, p.H - 1);
    };
    // activation row of staged row rr (0..31), clamped to the chunk
    auto arow = [&](int rr) -> int64_t {
        const int pos = pos0 + min(rr, rows - 1);
        return MODE == 0 ? (int64_t)p.assign_row[pos] : (int64_t)pos;
    };

    constexpr int kA = kMpRows * 16;         // 16-byte A chunks
    constexpr int kB = kMpCols * F::NL;      // 16-byte B chunks
    constexpr int kAPer = kA / 256;          // 2
    constexpr int kBPer = (kB + 255) / 256;  // Q4_K 3, Q6_K 4
    uint32_t a_src[kAPer];
    int a_off[kAPer];
#pragma unroll
    for (int i = 0; i < kAPer; i++) {
        const int t = threadIdx.x + 256 * i;
        const int rr = t >> 4, part = t & 15;
        a_src[i] = (uint32_t)(arow(rr) * av.ldq + 16 * part);
        a_off[i] = L::A + rr * kMpAS + 16 * part;
    }
    // B chunk t: column t / NL, part t % NL.  Columns 0..31 and 32..63 of
    // MODE 0 split at t = 32 NL, a multiple of 32 but not of 64: the matrix
    // is chosen per lane.  Q6_K: the block's dword window (it starts 0 or 2
    // bytes before the block) as 13 chunks plus one ending at its last byte.
    uint32_t b_src[kBPer];
    int b_off[kBPer];
    bool b_up[kBPer];
#pragma unroll
    for (int i = 0; i < kBPer; i++) {
        const int t = min((int)threadIdx.x + 256 * i, kB - 1);
        const int c2 = t / F::NL, part = t - c2 * F::NL;
        const int po = FMT == kQ6_K && part == F::NL - 1 ? 196 : 16 * part;
        b_up[i] = MODE == 0 && c2 >= 32;
        b_src[i] = (uint32_t)(wrow(c2) * wrow_bytes + po);
        b_off[i] = (int)threadIdx.x + 256 * i < kB ? L::B + c2 * F::BS + po : -1;
    }
    // D (row scales) on threads 0..31, H (16-value sums, Q4_K) on 64..127
    const int tD = threadIdx.x, tH = threadIdx.x - 64;
    const int64_t d_row = arow(tD & 31);
    const int64_t h_row = arow((tH >> 1) & 31);

    v4i sa[kAPer];
    u32x4 sb[kBPer];
    float sd = 0.f;
    v4i sh16 = {};
    auto issue = [&](int b) {
        const int8_t* abase = av.q + (int64_t)b * 256;
#pragma unroll
        for (int i = 0; i < kAPer; i++) sa[i] = *(const v4i*)(abase + a_src[i]);
        const int64_t boff = FMT == kQ6_K ? ((int64_t)b * F::BB) & ~(int64_t)3 : (int64_t)b * F::BB;
#pragma unroll
        for (int i = 0; i < kBPer; i++) sb[i] = *(const u32x4*)((b_up[i] ? ubase : gbase) + boff + b_src[i]);
        if (tD < 32) sd = av.d[d_row * av.ldd + b];
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 64) sh16 = *(const v4i*)(hsrc + (h_row * nb + b) * 16 + 8 * (tH & 1));
    };
    auto park = [&](uint8_t* s) {
#pragma unroll
        for (int i = 0; i < kAPer; i++) *(v4i*)(s + a_off[i]) = sa[i];
#pragma unroll
        for (int i = 0; i < kBPer; i++)
            if (b_off[i] >= 0) *(u32x4*)(s + b_off[i]) = sb[i];
        if (tD < 32) *(float*)(s + L::D + 4 * tD) = sd;
        if constexpr (F::kMins)
            if (tH >= 0 && tH < 64) *(v4i*)(s + L::H + 32 * (tH >> 1) + 16 * (tH & 1)) = sh16;
    };

    const int col = 16 * wave + jj;  // this lane's staged weight row
    // output r of the lane: tile r / 4, row 16 (r / 4) + 4 q + r % 4;
    // acc[k]: the f32 chain of reference lane k, accm[k] of mins lane k
    float acc[8][8], accm[4][8];
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
        for (int r = 0; r < 8; r++) acc[k][r] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int r = 0; r < 8; r++) accm[k][r] = 0.f;
    issue(0);
    park(st[0]);
    lds_barrier();
    for (int b = 0; b < nb; b++) {
        const uint8_t* S = st[b & 1];
        if (b + 1 < nb) issue(b + 1);
        const int sh = FMT == kQ6_K ? (int)(((int64_t)b * F::BB) & 3) : 0;
        const uint8_t* bcol = S + L::B + col * F::BS;
        float dd[8], dm[8];
        float xd, xdm = 0.f;
        uint32_t s6a = 0, s6b = 0;  // Q4_K: six-bit scales of sub-blocks 2q, 2q+1
        uint32_t q6s = 0;           // Q6_K: scale bytes 4q..4q+3
        Q4Scales sc{};
        if constexpr (FMT == kQ4_K) {
            const u32x4a16 hdr = *(const u32x4a16*)bcol;
            xd = f16_to_f32(hdr.x);
            xdm = f16_to_f32(hdr.x >> 16);
            sc = q4_scales(hdr.y, hdr.z, hdr.w);
            const uint32_t sw = q < 2 ? sc.sc_lo : sc.sc_hi;
            s6a = byte_of(sw, 2 * (q & 1));
            s6b = byte_of(sw, 2 * (q & 1) + 1);
        } else {
            xd = f16_to_f32(lds_win(bcol, sh, 208) & 0xffffu);
            q6s = lds_win(bcol, sh, 192 + 4 * q);
        }
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const float yd = *(const float*)(S + L::D + 4 * (16 * (r >> 2) + 4 * q + (r & 3)));
            dd[r] = yd * xd;
            if constexpr (F::kMins) dm[r] = -yd * xdm;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t w1[2], w2[2];
            int mul;  // isum = mul * (stream 1) + (stream 2)
            if constexpr (FMT == kQ4_K) {
                const uint32_t qd = *(const uint32_t*)(bcol + 16 + 32 * q + 4 * k);
                const uint32_t lo = qd & 0x0f0f0f0fu, hi = (qd >> 4) & 0x0f0f0f0fu;
                w1[0] = bytes_mul_small(lo, s6a >> 3);
                w1[1] = bytes_mul_small(hi, s6b >> 3);
                w2[0] = bytes_mul_small(lo, s6a & 7u);
                w2[1] = bytes_mul_small(hi, s6b & 7u);
                mul = 8;
            } else {
                const int hk = k >= 4;
                const int qo = 64 * (q >> 1) + 4 * k;
                const uint32_t l0 = lds_win(bcol, sh, qo), l1 = lds_win(bcol, sh, qo + 32);
                const uint32_t qh = lds_win(bcol, sh, 128 + 32 * (q >> 1) + 4 * k);
#pragma unroll
                for (int cc = 0; cc < 2; cc++) {
                    const uint32_t l = cc ? l1 : l0;
                    const uint32_t lo4 = (q & 1) ? ((l >> 4) & 0x0f0f0f0fu) : (l & 0x0f0f0f0fu);
                    const uint32_t u = lo4 | (((qh >> (2 * (2 * (q & 1) + cc))) & 0x03030303u) << 4);
                    const int scv = (int)(int8_t)(uint8_t)(q6s >> (8 * (2 * cc + hk)));
                    q6_scaled_split(u, scv, w2[cc], w1[cc]);
                }
                mul = 64;
            }
            const long b1 = (long)(((uint64_t)w1[1] << 32) | w1[0]);
            const long b2 = (long)(((uint64_t)w2[1] << 32) | w2[0]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const long a = *(const long*)(S + L::A + (16 * t + jj) * kMpAS + 32 * k + 8 * q);
                const v4i z = {};
                const v4i i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, z, 0, 0, 0);
                const v4i i2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b2, z, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[k][4 * t + r] = __builtin_fmaf(dd[4 * t + r], (float)(i1[r] * mul + i2[r]), acc[k][4 * t + r]);
            }
            // one lane's products at a time: the chains are advanced here
            // (not sunk to the end of the block), which bounds the live
            // MFMA results
#pragma unroll
            for (int r = 0; r < 8; r++) asm volatile("" : "+v"(acc[k][r]));
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (F::kMins) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t mwd = k < 2 ? sc.mn_lo : sc.mn_hi;
                const _Float16 mA = (_Float16)(float)byte_of(mwd, 2 * (k & 1));
                const _Float16 mB = (_Float16)(float)byte_of(mwd, 2 * (k & 1) + 1);
                // B[kappa][col], kappa = 4 q + e: nonzero for q == k
                const _Float16 zh = (_Float16)0.f;
                const v4h bm = q == k ? v4h{mA, mA, mB, mB} : v4h{zh, zh, zh, zh};
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const v4h am = *(const v4h*)(S + L::H + (16 * t + jj) * 32 + 8 * q);
                    const v4f z = {};
                    const v4f ms = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) accm[k][4 * t + r] = __builtin_fmaf(dm[4 * t + r], ms[r], accm[k][4 * t + r]);
                }
#pragma unroll
                for (int r = 0; r < 8; r++) asm volatile("" : "+v"(accm[k][r]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (b + 1 < nb) park(st[(b + 1) & 1]);
        lds_barrier();
    }
    // hsum_f32_8 and hsum_f32_4 over the lane chains
    float v[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        v[r] = ((acc[0][r] + acc[4][r]) + (acc[2][r] + acc[6][r])) + ((acc[1][r] + acc[5][r]) + (acc[3][r] + acc[7][r]));
        if constexpr (F::kMins) v[r] = v[r] + ((accm[0][r] + accm[2][r]) + (accm[1][r] + accm[3][r]));
    }

    if constexpr (MODE == 0) {
        // waves 2, 3 hold up of the columns waves 0, 1 hold gate of
        float* s_up = (float*)st[0];  // [32][32]
        if (wave >= 2)
#pragma unroll
            for (int r = 0; r < 8; r++) s_up[(16 * (r >> 2) + 4 * q + (r & 3)) * 32 + 16 * (wave - 2) + jj] = v[r];
        lds_barrier();
        if (wave < 2) {
            const int64_t i = (int64_t)blockIdx.x * 32 + 16 * wave + jj;
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int rr = 16 * (r >> 2) + 4 * q + (r & 3);
                const float u = s_up[rr * 32 + 16 * wave + jj];
                // SwiGLU as the reference writes it: (g / (1 + exp(-g))) * u
                if (rr < rows && i < p.I)
                    p.act[(int64_t)(pos0 + rr) * p.I + i] = __fdiv_rn(v[r], 1.f + exp_f32(-v[r])) * u;
            }
        }
    } else {
        const int64_t n = (int64_t)blockIdx.x * kMpCols + col;
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int rr = 16 * (r >> 2) + 4 * q + (r & 3);
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
// + shared * gate (src/qwen/quantized_moe.rs:266-273, :384-400).
__global__ __launch_bounds__(256) void k_mp_combine(MoeParams p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.M * p.H) return;
    const int t = (int)(idx / p.H);
    const int64_t nn = idx - (int64_t)t * p.H;
    const int K = (int)p.K;
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
hipError_t launch_p(const MoeParams& p, hipStream_t s, hipEvent_t const* ev) {
    const int M = p.M, K = (int)p.K, nbH = p.xq.ng;
    const int P = M * K + (p.sgate_w ? M : 0);
    if (ev) (void)hipEventRecord(ev[0], s);
    const int nr = (M + 15) / 16;
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
    hipLaunchKernelGGL((k_mp_mm<DFMT, 1>), dim3((unsigned)((p.H + kMpCols - 1) / kMpCols), (unsigned)p.max_chunks),
                       dim3(256), 0, s, p);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(k_mp_combine, dim3((unsigned)(((int64_t)M * p.H + 255) / 256)), dim3(256), 0, s, p);
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
                         al(p.sdown_w, da);
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
