// iq_prefill.hip -- y = x . W^T for Q4_K weights at many input rows
// (prefill), on int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// Arithmetic (iq_pf_q4k.h).  Every per-block integer is the reference's
// (src/qgemm.rs:175-245), bit for bit; the f32 combination
// y += dx_b (dw_b isum_b - dmin_b msum_b) runs in a different order than the
// reference's per-lane FMA chains: results agree within the path's 1e-4
// normwise tolerance, not bitwise (this kernel serves 64+ input rows; fewer
// rows keep the bit-exact kernels).
//
// Tiling.  A workgroup (8 waves, two per SIMD) owns 64 input rows and 128
// output columns; each wave all 64 rows of 16 columns as four 16 x 16 tiles
// of the double-rate v_mfma_i32_16x16x64_i8.  Per block the workgroup
// stages the int8 activation tile (16 KiB), the 128 raw Q4_K blocks
// (18 KiB), the bsums and the block scales in LDS, in three stages: the
// next two blocks' loads in flight while the current one is multiplied.  Each wave
// dequantises its B fragments in registers (nibbles, then one packed 16-bit
// multiply per dword and stream).  Calls too small to fill the GPU with
// such tiles take 32 x 64 tiles (4 waves, two row tiles each) and, only if
// those are still too few, a split over K, with partial tiles summed in a
// fixed order by a second pass.
#include "iq_lanes.h"
#include "iq_pf_q4k.h"
#include "iq_quant.h"

namespace iq {

namespace {


// Tile shape: ROWS input rows x COLS output columns per workgroup, one
// wave per 16 columns, each wave all ROWS rows (RT = ROWS / 16 row tiles
// share every decoded B fragment).  64 x 128 on 8 waves (two per SIMD)
// measured fastest where 256 such tiles fill the GPU ([256 x 2048] ->
// 8192: kernel 16.5-17.0 us): 128 x 64 on 4 waves, 128 x 128 on 8 waves
// with split K, 64 x 64 on 4 waves at two workgroups per CU (17.0-18.4 us)
// and 32 x 64 (20.9 us) were all slower.  Fewer tiles than that take 32 x 64
// on 4 waves, which fill the GPU without the split over K and its reduce
// launch: [256 x 4096] -> 2048 per call 24.1-32.6 us as 64 x 128 tiles in
// four K splits, 22.7 us as 256 unsplit 32 x 64 tiles.
constexpr int kPfRows = 64, kPfCols = 128;      // large calls
constexpr int kPfRowsS = 32, kPfColsS = 64;     // calls with fewer than 256 large tiles
constexpr int kPfMinTiles = 256;

// ---- activation quantisation --------------------------------------------------
// Q8K (bit-exact from_float) into the layouts the MFMA kernel reads:
// q [mp][k] int8 row-major, dT [nb][mp] block scales, hs [mp][nb][16] the
// block's sixteen 16-value sums as f16 (exact: |bsum16| <= 2048).  Rows
// m..mp-1 are zero.
__global__ __launch_bounds__(256) void k_quant_prefill(const float* __restrict__ x, int64_t ldx, int m, int mp,
                                                       int nb, int8_t* __restrict__ q, float* __restrict__ dT,
                                                       _Float16* __restrict__ hs) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (int64_t)mp * nb) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int row = (int)(wid / nb), b = (int)(wid % nb);
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (row < m) v = load4(x + (int64_t)row * ldx + (int64_t)b * 256 + 4 * lane);
    const Q8KLane r = quant_q8k_core(v);
    ((uint32_t*)(q + (int64_t)row * nb * 256 + (int64_t)b * 256))[lane] = r.packed;
    if (lane == 0) dT[(int64_t)b * mp + row] = r.d;
    if ((lane & 3) == 0) hs[((int64_t)row * nb + b) * 16 + (lane >> 2)] = (_Float16)r.bsum16;
}

struct PrefillArgs {
    const uint8_t* w;  // Q4_K [n][nb]
    int64_t n, row_bytes;
    int nb;
    const int8_t* q;
    const float* dT;
    const _Float16* hs;
    int m, mp;
    float* y;  // [m][ldy] when splits == 1
    int64_t ldy;
    float* part;  // [splits][m][n] otherwise
    int splits, bps;
    int32_t* dbg_isum;  // optional [m][n][nb] per-block integers
    int32_t* dbg_msum;
};


// LDS stage of one block: A int8 [ROWS][kAS], B raw Q4_K [COLS][kBS], H f16
// bsums [ROWS][16], D block scales [ROWS].  Row strides of 32 mod 64 bytes
// let the fragment reads (16 rows, four 16-byte columns per row) run without
// bank conflicts on gfx950; strides of 16 mod 64 bytes measure 1.5x slower.
constexpr int kAS = 288;  // activation row stride (256 bytes + pad)
constexpr int kBS = 160;  // Q4_K block stride (144 bytes + pad)
template <int ROWS, int COLS>
struct PfTile {
    static constexpr int kThreads = COLS / 16 * 64;
    static constexpr int kRT = ROWS / 16;
    static constexpr int kStA = 0, kStB = kStA + ROWS * kAS, kStH = kStB + COLS * kBS, kStD = kStH + ROWS * 32;
    static constexpr int kStage = kStD + ROWS * 4;
    // Three stages, two blocks' loads in flight behind the one being
    // multiplied ([256 x 4096] -> 2048: 20.4 -> 19.3 us per call, [256 x
    // 2048] -> 8192: 19.2 -> 19.1 us against two stages).  Each stage is
    // followed by 1 KiB that takes the loads of lanes and of whole
    // instructions past the stage, so that every wave issues the same number
    // of loads per stage and a wait can count them.
    static constexpr int kNst = 3;
    static constexpr int kStagePad = kStage + 1024;
};

// Workgroup barrier once this wave's LDS reads have returned, without the
// release fence of lds_barrier: at workgroup scope that fence also waits for
// every LDS DMA load in flight (vmcnt(0)), which would drain the stages
// loading ahead.  Stage arrival is counted by explicit vmcnt waits.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wave w owns all ROWS rows and columns 16w .. 16w+15 of the tile as RT
// 16 x 16 tiles of v_mfma_i32_16x16x64_i8 (one decoded B fragment serves
// RT row tiles).  For lane l (g = l / 16, j = l % 16) a fragment holds K
// 16g..16g+15 of row / column j, and the result rows 4g..4g+3 of column j.
// One K step is 64 values: sub-blocks 2s and 2s+1 of the block, whose
// weights are the low and the high nibbles of qs bytes 32s..32s+31.
template <int ROWS, int COLS, bool DBG>
__global__ __launch_bounds__((PfTile<ROWS, COLS>::kThreads)) void k_prefill_q4k(PrefillArgs p) {
    using T = PfTile<ROWS, COLS>;
    constexpr int kThreads = T::kThreads;
    constexpr int kStA = T::kStA, kStB = T::kStB, kStH = T::kStH, kStD = T::kStD, kStage = T::kStage;
    constexpr int RT = T::kRT;
    constexpr int NST = T::kNst, kSP = T::kStagePad;
    __shared__ __align__(16) uint8_t st[NST][kSP];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, jj = lane & 15;
    // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs, so
    // ids L, L + 8, L + 16, ... (same XCD) take the m-tiles of one column
    // tile and share its weights in that XCD's L2.
    const int mtiles = p.mp / ROWS;
    const int grp = blockIdx.x / (8 * mtiles), rem = blockIdx.x - grp * 8 * mtiles;
    const int ntile = 8 * grp + (rem & 7), mtile = rem >> 3;
    if ((int64_t)ntile * COLS >= p.n) return;  // padding workgroup (whole group uniform)
    const int n0 = ntile * COLS;
    const int row0 = mtile * ROWS;
    const int b0 = blockIdx.z * p.bps;
    const int b1 = min(p.nb, b0 + p.bps);
    const int64_t K = (int64_t)p.nb * 256;

    // staging straight into LDS (global_load_lds_dwordx4): instruction i of
    // wave w of W fills the 64 consecutive 16-byte granules (W i + w) * 64 .. +63
    // of a stage, each lane the granule at base + 16 lane.  The stage keeps
    // its padded layout (A rows of 18 granules, B columns of 10, then H and
    // D).  Every lane loads, so that each wave issues the same count per
    // stage: pad granules land in the row padding, granules past the stage
    // (from clamped addresses) in the 1 KiB behind it.
    constexpr int kGA = ROWS * 18, kGB = COLS * 10, kGH = ROWS * 2, kGD = ROWS / 4;
    constexpr int kG = kGA + kGB + kGH + kGD;
    constexpr int kWaves = kThreads / 64, kIPer = (kG + kThreads - 1) / kThreads;
    static_assert(kStB == kGA * 16 && kStH == kStB + kGB * 16 && kStD == kStH + kGH * 16, "stage layout");
    const uint8_t* gsrc[kIPer];
    uint32_t gstr[kIPer];
#pragma unroll
    for (int i = 0; i < kIPer; i++) {
        int t = (i * kWaves + wave) * 64 + lane;
        t = min(t, kG - 1);
        if (t < kGA) {
            const int r = t / 18, gr = t - 18 * r;
            gsrc[i] = (const uint8_t*)p.q + (int64_t)(row0 + r) * K + 16 * min(gr, 15);
            gstr[i] = 256;
        } else if ((t -= kGA) < kGB) {
            const int col = t / 10, gr = t - 10 * col;
            const int64_t gc = min((int64_t)n0 + col, p.n - 1);
            gsrc[i] = p.w + gc * p.row_bytes + 16 * min(gr, 8);
            gstr[i] = 144;
        } else if ((t -= kGB) < kGH) {
            gsrc[i] = (const uint8_t*)(p.hs + (int64_t)(row0 + (t >> 1)) * p.nb * 16 + 8 * (t & 1));
            gstr[i] = 32;
        } else {
            t -= kGH;
            gsrc[i] = (const uint8_t*)(p.dT + row0 + 4 * t);
            gstr[i] = (uint32_t)p.mp * 4;
        }
    }
    auto issue = [&](int b, uint8_t* s) {
        b = min(b, b1 - 1);
#pragma unroll
        for (int i = 0; i < kIPer; i++)
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)(gsrc[i] + (int64_t)b * gstr[i]),
                (void __attribute__((address_space(3)))*)(s + min((i * kWaves + wave) * 1024, kStage)), 16, 0, 0);
    };
    static_assert(kIPer <= 15, "vmcnt field");

    float out[RT][4];  // [row tile][r]
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) out[rt][r] = 0.f;

    issue(b0, st[0]);
    if (!DBG && b0 + 1 < b1) {
        issue(b0 + 1, st[1]);
        __builtin_amdgcn_s_waitcnt(0x0f70 | kIPer);  // vmcnt(kIPer): stage 0 is in LDS
    } else {
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    }
    stage_barrier();

    int cur = 0;
    for (int b = b0; b < b1; b++) {
        const uint8_t* S = st[cur];
        const int nx = cur + 1 == NST ? 0 : cur + 1, nx2 = nx + 1 == NST ? 0 : nx + 1;
        if constexpr (DBG) {  // the debug stores share vmcnt: one block ahead, drained each block
            if (b + 1 < b1) issue(b + 1, st[nx]);
        } else {
            if (b + 2 < b1) issue(b + 2, st[nx2]);
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* bcol = S + kStB + (16 * wave + jj) * kBS;
        pf_q4k_block<RT, kAS>(S + kStA, bcol, S + kStH, (const float*)(S + kStD), g, jj, out,
                             [&](int rt, int r, int32_t isum, float msum) {
                                 if constexpr (DBG) {
                                     const int64_t row = row0 + 16 * rt + 4 * g + r, gc = n0 + 16 * wave + jj;
                                     if (row < p.m && gc < p.n) {
                                         p.dbg_isum[(row * p.n + gc) * p.nb + b] = isum;
                                         p.dbg_msum[(row * p.n + gc) * p.nb + b] = (int32_t)msum;
                                     }
                                 }
                             });
        __builtin_amdgcn_sched_barrier(0);
        if (!DBG && b + 2 < b1)
            __builtin_amdgcn_s_waitcnt(0x0f70 | kIPer);  // vmcnt(kIPer): stage b + 1 is in LDS
        else
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        stage_barrier();
        cur = nx;
    }

    float* dst = p.splits == 1 ? p.y : p.part + (int64_t)blockIdx.z * p.m * p.n;
    const int64_t ld = p.splits == 1 ? p.ldy : p.n;
    const int64_t gc = (int64_t)n0 + 16 * wave + jj;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t row = row0 + 16 * rt + 4 * g + r;
            // streaming stores: the 8 MB of a [256 x 8192] result are read
            // by the next launch, not this one (19.3-19.8 us per call
            // against 20.1-20.9 with ordinary stores)
            if (row < p.m && gc < p.n) __builtin_nontemporal_store(out[rt][r], dst + row * ld + gc);
        }
}

// y = sum over splits of the partial tiles, in split order.
__global__ __launch_bounds__(256) void k_prefill_reduce(const float* __restrict__ part, int splits, int m, int64_t n,
                                                        float* __restrict__ y, int64_t ldy) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)m * n) return;
    const int64_t row = i / n, col = i - row * n;
    float s = part[i];
    for (int z = 1; z < splits; z++) s = s + part[(int64_t)z * m * n + i];
    y[row * ldy + col] = s;
}

constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct PfPlan {
    int mp, nb, splits, bps;
    int rows, cols;  // workgroup tile
    size_t q_bytes, d_bytes, hs_bytes, part_bytes;
    size_t total() const { return q_bytes + d_bytes + hs_bytes + part_bytes; }
};

PfPlan plan(const WeightView& w, int64_t m) {
    PfPlan P;
    P.nb = (int)(w.cols / 256);
    const int64_t large = (w.rows + kPfCols - 1) / kPfCols * ((m + kPfRows - 1) / kPfRows);
    P.rows = large >= kPfMinTiles ? kPfRows : kPfRowsS;
    P.cols = large >= kPfMinTiles ? kPfCols : kPfColsS;
    P.mp = (int)((m + P.rows - 1) / P.rows * P.rows);
    const int64_t tiles = ((w.rows + P.cols - 1) / P.cols) * (P.mp / P.rows);  // real tiles (padding aside)
    int splits = 1;
    while (tiles * splits < kPfMinTiles && splits * 2 <= P.nb && splits < 8) splits *= 2;
    P.bps = (P.nb + splits - 1) / splits;
    P.splits = (P.nb + P.bps - 1) / P.bps;
    P.q_bytes = align256((size_t)P.mp * P.nb * 256);
    P.d_bytes = align256((size_t)P.nb * P.mp * 4);
    P.hs_bytes = align256((size_t)P.mp * P.nb * 32);
    P.part_bytes = P.splits > 1 ? align256((size_t)P.splits * m * w.rows * 4) : 0;
    return P;
}

}  // namespace

bool prefill_supported(const WeightView& w, int64_t m) {
    return w.dtype == kQ4_K && m >= kPrefillMinRows && w.cols % 256 == 0 && w.rows >= 1 && m <= (1 << 20);
}

size_t prefill_workspace_size(const WeightView& w, int64_t m) { return prefill_supported(w, m) ? plan(w, m).total() : 0; }

hipError_t launch_prefill(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                          void* ws, int32_t* dbg_isum, int32_t* dbg_msum, hipStream_t s) {
    if (!prefill_supported(w, m)) return hipErrorNotSupported;
    const PfPlan P = plan(w, m);
    uint8_t* base = (uint8_t*)ws;
    PrefillArgs a;
    a.w = w.w;
    a.n = w.rows;
    a.row_bytes = w.row_bytes;
    a.nb = P.nb;
    a.q = (const int8_t*)base;
    a.dT = (const float*)(base + P.q_bytes);
    a.hs = (const _Float16*)(base + P.q_bytes + P.d_bytes);
    a.part = P.splits > 1 ? (float*)(base + P.q_bytes + P.d_bytes + P.hs_bytes) : nullptr;
    a.m = (int)m;
    a.mp = P.mp;
    a.y = y;
    a.ldy = ldy;
    a.splits = P.splits;
    a.bps = P.bps;
    a.dbg_isum = dbg_isum;
    a.dbg_msum = dbg_msum;
    const int64_t qwaves = (int64_t)P.mp * P.nb;
    hipLaunchKernelGGL(k_quant_prefill, dim3((unsigned)((qwaves + 3) / 4)), dim3(256), 0, s, x, ldx, (int)m, P.mp,
                       P.nb, (int8_t*)a.q, (float*)a.dT, (_Float16*)a.hs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t ntiles = (w.rows + P.cols - 1) / P.cols;
    dim3 grid((unsigned)((ntiles + 7) / 8 * 8 * (P.mp / P.rows)), 1, (unsigned)P.splits);
    if (P.rows == kPfRows) {
        constexpr int TH = PfTile<kPfRows, kPfCols>::kThreads;
        if (dbg_isum) hipLaunchKernelGGL((k_prefill_q4k<kPfRows, kPfCols, true>), grid, dim3(TH), 0, s, a);
        else hipLaunchKernelGGL((k_prefill_q4k<kPfRows, kPfCols, false>), grid, dim3(TH), 0, s, a);
    } else {
        constexpr int TH = PfTile<kPfRowsS, kPfColsS>::kThreads;
        if (dbg_isum) hipLaunchKernelGGL((k_prefill_q4k<kPfRowsS, kPfColsS, true>), grid, dim3(TH), 0, s, a);
        else hipLaunchKernelGGL((k_prefill_q4k<kPfRowsS, kPfColsS, false>), grid, dim3(TH), 0, s, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess || P.splits == 1) return e;
    const int64_t tot = m * w.rows;
    hipLaunchKernelGGL(k_prefill_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, (const float*)a.part,
                       P.splits, (int)m, w.rows, y, ldy);
    return hipGetLastError();
}

}  // namespace iq
