// iq_lanes.hip -- y = act . W^T for one quantised matrix, in the reference's
// exact f32 order (src/qgemm.rs:175-397 via src/gguf.rs:608-690).
//
// Grid: x = 4-wave workgroups over output rows (8 rows per wave), y = tiles
// of MT input rows.  Weights stream once per input tile in native GGUF
// layout; the activations (a few KiB per row) stay in L2/L1.
#include "iq_lanes.h"

namespace iq {

namespace {

struct MMArgs {
    const uint8_t* w;
    int64_t n, row_bytes;
    int nbw;  // weight blocks per row (Q8_0: K/32)
    ActView a;
    int m;
    float* y;
    int64_t ldy;
    int32_t* isum;  // optional per-block lane integers
    int32_t* msum;
};

template <int FMT, int MT, int BC, bool DBG>
__global__ __launch_bounds__(256) void k_mm_lanes(MMArgs p) {
    const int lane = threadIdx.x & 63;
    const int k = lane & 7, slot = lane >> 3;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + slot;
    const bool ok = row < p.n;
    const int m0 = blockIdx.y * MT;
    const uint8_t* wrow[1] = {ok ? p.w + row * p.row_bytes : nullptr};
    int64_t arow[1][MT];
#pragma unroll
    for (int i = 0; i < MT; i++) arow[0][i] = m0 + i;
    const int mc[1] = {min(MT, p.m - m0)};
    float out[1][MT];
    DbgOut dbg;
    if constexpr (DBG) {
        dbg.isum = p.isum;
        dbg.msum = p.msum;
        dbg.n = p.n;
        dbg.row = row;
        dbg.nbw = p.nbw;
    }
    lanes_dot<FMT, MT, 1, BC, DBG>(wrow, p.nbw, p.a, arow, mc, k, out, dbg);
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
        if (k == 0 && ok && mi < mc[0]) p.y[(int64_t)(m0 + mi) * p.ldy + row] = out[0][mi];
}

template <int FMT, int MT, int BC>
hipError_t launch_t(const MMArgs& args, bool dbg, hipStream_t s) {
    const int64_t waves = (args.n + 7) / 8;
    dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((args.m + MT - 1) / MT));
    if (dbg) hipLaunchKernelGGL((k_mm_lanes<FMT, MT, BC, true>), grid, dim3(256), 0, s, args);
    else hipLaunchKernelGGL((k_mm_lanes<FMT, MT, BC, false>), grid, dim3(256), 0, s, args);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_fmt(const MMArgs& args, bool dbg, hipStream_t s) {
    constexpr int BC1 = FMT == kQ8_0 ? 4 : 8;
    constexpr int BCn = FMT == kQ8_0 ? 2 : 4;
    if (args.m <= 1) return launch_t<FMT, 1, BC1>(args, dbg, s);
    if (args.m <= 2) return launch_t<FMT, 2, BCn>(args, dbg, s);
    if (args.m <= 4) return launch_t<FMT, 4, BCn>(args, dbg, s);
    if (args.m <= 8) return launch_t<FMT, 8, BCn>(args, dbg, s);
    return launch_t<FMT, 16, BCn>(args, dbg, s);
}

}  // namespace

hipError_t launch_matmul_lanes(const WeightView& w, const ActView& a, float* y, int64_t ldy, int32_t* isum,
                               int32_t* msum, hipStream_t s) {
    MMArgs args;
    args.w = w.w;
    args.n = w.rows;
    args.row_bytes = w.row_bytes;
    args.nbw = (int)(w.dtype == kQ8_0 ? w.cols / 32 : w.cols / 256);
    args.a = a;
    args.m = a.m;
    args.y = y;
    args.ldy = ldy;
    args.isum = isum;
    args.msum = msum;
    if (args.n == 0 || args.m == 0) return hipSuccess;
    const bool dbg = isum != nullptr;
    switch (w.dtype) {
    case kQ4_K: return launch_fmt<kQ4_K>(args, dbg, s);
    case kQ5_K: return launch_fmt<kQ5_K>(args, dbg, s);
    case kQ6_K: return launch_fmt<kQ6_K>(args, dbg, s);
    case kQ8_0: return launch_fmt<kQ8_0>(args, dbg, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace iq
