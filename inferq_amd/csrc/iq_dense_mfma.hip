// iq_dense_mfma.hip -- y = x . W^T for Q4_K / Q6_K weights at 2..63 input
// rows on large matrices (the LM head at verify widths), on int8 MFMA in the
// reference's exact per-lane order (iq_mfma_lanes.h): every output is
// bitwise what the one-row kernel gives, as src/gguf.rs:493-520 requires of
// its row tiles.  The per-lane GEMV (iq_gemv.hip) spends eight exact dot
// chains of VALU work per weight at 8 rows; here the integer dots run on
// MFMA and the VALU keeps only the f32 chains.
//
// Two launches per call: k_dm_quant quantises x (Q8K, the lane-transposed
// activation layout, block scales, 16-value sums as f16); k_dm_mm<FMT, RT>
// takes 64 weight rows x 16 RT input rows per workgroup, and k_dm_mm_pk
// 64 weight rows x up to 8 input rows with two reference lanes per MFMA.
#include "iq_internal.h"
#include "iq_mfma_lanes.h"
#include "iq_quant.h"

namespace iq {

namespace {

struct DmArgs {
    const uint8_t* w;  // [n][row_bytes]
    int64_t n, row_bytes;
    int nb;            // blocks per row
    const int8_t* q;   // [m][nb * 256] quantised x, lane-transposed
    const float* d;    // [m][nb] block scales
    const _Float16* hs;  // [m][nb][16] 16-value sums
    int m;
    float* y;  // [m][ldy]
    int64_t ldy;
    // fused greedy selection (k_dm_mm_pk): per input row r, workgroup b
    // leaves its 64 columns' largest (argmax key, logit) at r * gridDim.x + b
    uint64_t* amx_key = nullptr;
    float* amx_val = nullptr;
};

// One wave per (row, 256-value block): Q8K (bit-exact from_float).
__global__ __launch_bounds__(256) void k_dm_quant(const float* __restrict__ x, int64_t ldx, int m, int nb,
                                                  int8_t* __restrict__ q, float* __restrict__ d,
                                                  _Float16* __restrict__ hs) {
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (int64_t)m * nb) return;  // uniform per wave
    const int64_t row = wid / nb;
    const int b = (int)(wid - row * nb);
    const Q8KLane r = quant_q8k_core(load4(x + row * ldx + (int64_t)b * 256 + 4 * lane));
    ((uint32_t*)(q + (row * nb + b) * 256))[perm_dword(lane >> 3, lane & 7)] = r.packed;
    if (lane == 0) d[row * nb + b] = r.d;
    if ((lane & 3) == 0) hs[(row * nb + b) * 16 + (lane >> 2)] = (_Float16)(float)r.bsum16;
}

// Grid (n / 64, m / (16 RT)): 64 weight rows x 16 RT input rows.
template <int FMT, int RT>
__global__ __launch_bounds__(256) void k_dm_mm(DmArgs a) {
    using L = MlStage<FMT, RT>;
    __shared__ __align__(16) uint8_t st[2][L::END];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * kMlCols;
    const int row0 = (int)blockIdx.y * 16 * RT;
    const int rows = min(16 * RT, a.m - row0);
    MlOperands op;
    op.aq = a.q;
    op.ldq = (int64_t)a.nb * 256;
    op.ad = a.d;
    op.ldd = a.nb;
    op.hs = a.hs;
    op.b0 = op.b1 = a.w + n0 * a.row_bytes;  // byte offsets stay within the tile's 64 rows
    op.bsplit = kMlCols;
    op.brow_bytes = a.row_bytes;
    op.nb = a.nb;
    const int64_t last = a.n - 1 - n0;
    auto brow = [&](int t) -> int64_t { return t < last ? (int64_t)t : last; };
    auto arow = [&](int rr) -> int64_t { return row0 + min(rr, rows - 1); };
    float v[4 * RT];
    ml_product<FMT, RT>(op, arow, brow, st, v);
    const int64_t n = n0 + 16 * wave + jj;
#pragma unroll
    for (int r = 0; r < 4 * RT; r++) {
        const int rr = 16 * (r >> 2) + 4 * q + (r & 3);
        if (rr < rows && n < a.n) a.y[(int64_t)(row0 + rr) * a.ldy + n] = v[r];
    }
}

// At most 8 input rows: 64 weight rows x the 8 rows per workgroup, two
// reference lanes per MFMA (ml_product_pk).  AMX: greedy selection fused
// (DmArgs::amx_key).
template <int FMT, bool AMX = false>
__global__ __launch_bounds__(256) void k_dm_mm_pk(DmArgs a) {
    using L = MlStagePk<FMT>;
    __shared__ __align__(16) uint8_t st[2][L::END];
    __shared__ __align__(16) uint8_t zero[256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    ((uint32_t*)zero)[threadIdx.x & 63] = 0u;  // read only after the first barrier
    const int64_t n0 = (int64_t)blockIdx.x * kMlCols;
    const int rows = a.m;
    MlOperands op;
    op.aq = a.q;
    op.ldq = (int64_t)a.nb * 256;
    op.ad = a.d;
    op.ldd = a.nb;
    op.hs = a.hs;
    op.b0 = op.b1 = a.w + n0 * a.row_bytes;
    op.bsplit = kMlCols;
    op.brow_bytes = a.row_bytes;
    op.nb = a.nb;
    const int64_t last = a.n - 1 - n0;
    auto brow = [&](int t) -> int64_t { return t < last ? (int64_t)t : last; };
    auto arow = [&](int rr) -> int64_t { return min(rr, rows - 1); };
    float v[4];
    ml_product_pk<FMT>(op, arow, brow, st, zero, v);
    const int64_t n = n0 + 16 * wave + jj;
    if (q < 2) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 4 * q + r;
            if (rr < rows && n < a.n) a.y[(int64_t)rr * a.ldy + n] = v[r];
        }
    }
    if constexpr (AMX) {
        // lanes q and q + 2 hold the same outputs; the keys of lanes q < 2
        // (input rows 4 q + r, column n) meet over the 16 columns of a lane
        // group, then over the workgroup's four waves
        __shared__ uint64_t s_k[4][8];
        __shared__ float s_v[4][8];
        uint64_t key[4];
        float kv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 4 * (q & 1) + r;
            key[r] = q < 2 && rr < rows && n < a.n ? argmax_key(v[r], n) : 0;
            kv[r] = v[r];
            row16_max_kv(key[r], kv[r]);
        }
        if (q < 2 && jj == 0)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                s_k[wave][4 * q + r] = key[r];
                s_v[wave][4 * q + r] = kv[r];
            }
        __syncthreads();
        if (threadIdx.x < 8 && (int)threadIdx.x < rows) {
            const int rr = threadIdx.x;
            uint64_t bk = s_k[0][rr];
            float bv = s_v[0][rr];
            for (int w = 1; w < 4; w++)
                if (s_k[w][rr] > bk) {
                    bk = s_k[w][rr];
                    bv = s_v[w][rr];
                }
            const int64_t o = (int64_t)rr * gridDim.x + blockIdx.x;
            a.amx_key[o] = bk;
            a.amx_val[o] = bv;
        }
    }
}

// Mid-size matrices of width 2048 or 4096 at up to 8 rows: 64 weight rows
// per workgroup leave too few workgroups (128 for [8192 x 2048]), each a
// chain of dependent block loads.  Here a workgroup takes 16 weight rows
// and each of its NW waves two of the 2 NW blocks, all loaded at once; the
// waves form their blocks' exact integers in parallel, then the f32 chains
// pass from wave to wave in block order through LDS, so every output is
// the one-row kernel's bit for bit.
template <int FMT, int NW>
__global__ __launch_bounds__(NW * 64) void k_dm_sk(DmArgs a) {
    __shared__ __align__(16) uint8_t reg[NW][kSkBPW][MlSkRegion<FMT>::END];
    __shared__ __align__(16) uint8_t zero[256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, jj = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int rows = a.m;
    MlOperands op;
    op.aq = a.q;
    op.ldq = (int64_t)a.nb * 256;
    op.ad = a.d;
    op.ldd = a.nb;
    op.hs = a.hs;
    op.b0 = op.b1 = a.w + n0 * a.row_bytes;
    op.bsplit = 16;
    op.brow_bytes = a.row_bytes;
    op.nb = a.nb;
    const int64_t last = a.n - 1 - n0;
    auto brow = [&](int t) -> int64_t { return t < last ? (int64_t)t : last; };
    auto arow = [&](int rr) -> int64_t { return min(rr, rows - 1); };
    float v[4];
    ml_product_sk<FMT, NW>(op, arow, brow, reg, zero, v);
    if (wave == NW - 1 && q < 2) {
        const int64_t n = n0 + jj;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int rr = 4 * q + r;
            if (rr < rows && n < a.n) a.y[(int64_t)rr * a.ldy + n] = v[r];
        }
    }
}

constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct DmPlan {
    size_t q_bytes, d_bytes, hs_bytes;
    size_t total() const { return q_bytes + d_bytes + hs_bytes; }
};

DmPlan dm_plan(const WeightView& w, int64_t m) {
    const int64_t nb = w.cols / 256;
    DmPlan P;
    P.q_bytes = align256((size_t)(m * nb * 256));
    P.d_bytes = align256((size_t)(m * nb * 4));
    P.hs_bytes = align256((size_t)(m * nb * 32));
    return P;
}

template <int FMT>
hipError_t launch_sk(const DmArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.n + 15) / 16));
    if (a.nb == 8) hipLaunchKernelGGL((k_dm_sk<FMT, 4>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_dm_sk<FMT, 8>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_pk(const DmArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.n + kMlCols - 1) / kMlCols));
    if (a.amx_key) hipLaunchKernelGGL((k_dm_mm_pk<FMT, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_dm_mm_pk<FMT, false>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int FMT, int RT>
hipError_t launch_t(const DmArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.n + kMlCols - 1) / kMlCols), (unsigned)((a.m + 16 * RT - 1) / (16 * RT)));
    hipLaunchKernelGGL((k_dm_mm<FMT, RT>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

// Largest matrix the split-K tile takes (larger ones keep 64 weight rows per
// workgroup and load the activations once per 64 rows)
constexpr int64_t kDmSkMaxBytes = (int64_t)64 << 20;

// Whether the tile can read W at all: staging reads 16-byte chunks of Q4_K
// rows and 4-byte-aligned windows of Q6_K blocks, so rows must keep that
// alignment (Q6_K: an even block count per row).
bool dm_layout_ok(const WeightView& w) {
    if (w.cols % 256 != 0 || w.rows < 1) return false;
    if (w.dtype == kQ4_K || w.dtype == kQ5_K) return ((uintptr_t)w.w & 15) == 0;
    if (w.dtype == kQ6_K) return ((uintptr_t)w.w & 3) == 0 && w.row_bytes % 4 == 0;
    return false;
}

// Where the dispatch uses these kernels (measured on MI355X, per call over
// distinct matrices):
//  - from 64 MiB of weights at 2..63 rows (an LM head: the GEMV is 1.3x-2.3x
//    slower at 2-8 rows, 2.2x-4.5x at 8-48);
//  - at 3..8 rows from 8 MiB (the split-K tile: q/gate [8192 x 2048] at 4
//    rows 12.6 -> 10.2 us, at 8 rows 18.4 -> 10.3 us; q/gate + k + v joined
//    [9216 x 2048] at 4 rows 20.9 -> 11.3 us; qkvz + ba [12352 x 2048] at 3
//    rows 22.9 -> 12.2 us), and at 6..8 rows from 4 MiB (Q6_K [2048 x 4096]
//    at 6 rows 14.0 -> 10.6 us; Q4_K o [2048 x 4096] 11.0 -> 10.9 us); at 2
//    rows the GEMV stays faster (q/gate 8.3 against 9.9 us);
//  - at 9..63 rows from 8 MiB with 16 rows or more or 8192 weight rows or
//    more (q/gate at 12 rows 23.4 -> 15.9 us, at 16 rows 1.8x-2.4x);
//  - from 64 rows (prefill widths) every K-quant matrix the tile can read:
//    the result stays bitwise the one-row result, which speculative decoding
//    needs (src/gguf.rs:493-520 tiles prefill rows under the same guarantee).
// Smaller or narrower matrices keep the GEMV, whose latency is lower there
// (a [512 x 2048] matrix: 4.1 against 7.9 us at 8 rows).
// The tiles address activation rows with 32-bit byte offsets (MlOperands).
static bool dm_rows_ok(const WeightView& w, int64_t m) {
    return m >= 1 && m <= (int64_t)1 << 20 && (uint64_t)m * (uint64_t)w.cols <= 0xffffffffull;
}

bool dense_mfma_supported(const WeightView& w, int64_t m) {
    if (m < 2 || !dm_layout_ok(w) || !dm_rows_ok(w, m)) return false;
    // Q5_K: the 16- and 32-row tiles from 9 rows (up to 8 rows the split-K
    // GEMV or the lane kernel take it)
    if (w.dtype == kQ5_K) return m >= 9;
    if (m >= kPrefillMinRows) return true;
    const int64_t bytes = w.rows * w.row_bytes, MiB = (int64_t)1 << 20;
    if (bytes >= 64 * MiB) return true;
    if (m <= 8) return m >= 3 && (bytes >= 8 * MiB || (m >= 6 && bytes >= 4 * MiB));
    return bytes >= 8 * MiB && (m >= 16 || w.rows >= 8192);
}

size_t dense_mfma_workspace_any(const WeightView& w, int64_t m) {
    return dm_layout_ok(w) && dm_rows_ok(w, m) ? dm_plan(w, m).total() : 0;
}

hipError_t launch_dense_mfma_any(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                                 void* ws, hipStream_t s);

hipError_t launch_dense_mfma(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                             void* ws, hipStream_t s) {
    if (!dense_mfma_supported(w, m)) return hipErrorNotSupported;
    return launch_dense_mfma_any(w, x, ldx, m, y, ldy, ws, s);
}

// The split-K tile's choice: up to 8 rows on mid-size matrices of width
// 2048 or 4096.
static bool dm_takes_sk(const WeightView& w, int64_t m) {
    const int nb = (int)(w.cols / 256);
    return m <= 8 && (nb == 8 || nb == 16) && w.rows * w.row_bytes <= kDmSkMaxBytes;
}

static hipError_t dense_run(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                            void* ws, uint64_t* amx_key, float* amx_val, hipStream_t s);

hipError_t launch_dense_mfma_any(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                                 void* ws, hipStream_t s) {
    return dense_run(w, x, ldx, m, y, ldy, ws, nullptr, nullptr, s);
}

bool dense_argmax_supported(const WeightView& w, int64_t m) {
    return m >= 2 && m <= 8 && dense_mfma_supported(w, m) && !dm_takes_sk(w, m);
}

int64_t dense_argmax_parts(const WeightView& w) { return (w.rows + kMlCols - 1) / kMlCols; }

hipError_t launch_dense_argmax(const WeightView& w, const float* x, int64_t m, float* y, void* ws, uint64_t* keys,
                               float* vals, hipStream_t s) {
    if (!dense_argmax_supported(w, m) || !keys || !vals) return hipErrorNotSupported;
    return dense_run(w, x, w.cols, m, y, w.rows, ws, keys, vals, s);
}

static hipError_t dense_run(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                            void* ws, uint64_t* amx_key, float* amx_val, hipStream_t s) {
    if (!dm_layout_ok(w) || !dm_rows_ok(w, m)) return hipErrorNotSupported;
    const DmPlan P = dm_plan(w, m);
    uint8_t* base = (uint8_t*)ws;
    DmArgs a;
    a.w = w.w;
    a.n = w.rows;
    a.row_bytes = w.row_bytes;
    a.nb = (int)(w.cols / 256);
    a.q = (const int8_t*)base;
    a.d = (const float*)(base + P.q_bytes);
    a.hs = (const _Float16*)(base + P.q_bytes + P.d_bytes);
    a.m = (int)m;
    a.y = y;
    a.ldy = ldy;
    a.amx_key = amx_key;
    a.amx_val = amx_val;
    const int64_t qwaves = m * a.nb;
    hipLaunchKernelGGL(k_dm_quant, dim3((unsigned)((qwaves + 3) / 4)), dim3(256), 0, s, x, ldx, (int)m, a.nb,
                       (int8_t*)a.q, (float*)a.d, (_Float16*)a.hs);
    if (hipError_t e = hipGetLastError()) return e;
    // up to 8 rows: the split-K tile on mid-size matrices of width 2048 or 4096
    const bool sk = dm_takes_sk(w, m);
    if (amx_key && (sk || m > 8)) return hipErrorNotSupported;  // fused selection: pair-lane tile only
    if (w.dtype == kQ5_K && m <= 8) return hipErrorNotSupported;  // Q5_K: row tiles only
    // 16-row tiles up to 16 rows, and wider where 32-row tiles would leave
    // the GPU short of workgroups (at most 256 of them for Q4_K, 128 for
    // Q6_K, whose 16-row tiles cost more): [2048 x 4096] Q4_K at 64 / 256
    // rows 35.4 -> 27.1 / 37.2 -> 30.9 us, [4096 x 2048] Q6_K at 64 rows
    // 21.7 -> 18.2 us; from 512 workgroups the 32-row tiles win (Q6_K
    // [8192 x 2048] at 256 rows 45.4 against 59.5 us)
    const int64_t g32 = (w.rows + kMlCols - 1) / kMlCols * ((m + 31) / 32);
    const bool rt1 = m <= 16 || g32 <= (w.dtype == kQ6_K ? 128 : 256);
    if (w.dtype == kQ5_K) return rt1 ? launch_t<kQ5_K, 1>(a, s) : launch_t<kQ5_K, 2>(a, s);
    if (w.dtype == kQ4_K)
        return sk ? launch_sk<kQ4_K>(a, s) : m <= 8 ? launch_pk<kQ4_K>(a, s)
                                       : rt1 ? launch_t<kQ4_K, 1>(a, s) : launch_t<kQ4_K, 2>(a, s);
    return sk ? launch_sk<kQ6_K>(a, s) : m <= 8 ? launch_pk<kQ6_K>(a, s)
                                   : rt1 ? launch_t<kQ6_K, 1>(a, s) : launch_t<kQ6_K, 2>(a, s);
}

}  // namespace iq
