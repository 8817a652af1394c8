// iq_dense_f32.hip -- y = x . W^T for F32 and BF16 matrices.  The
// reference's QuantizedMatrix accepts both (src/gguf.rs:305-317) and
// multiplies them through candle's f32 matmul, having no multi-row kernel
// for them (src/gguf.rs:533-535, :599); such matrices are small (routers,
// gate vectors), and the product is a plain f32 dot per output.
//
// Order: for each (input row, weight row) lane l sums x[k] * w[k] (the
// product rounded, then the add) over k = l + 64 j for j = 0, 1, ... in
// turn, then the 64 lanes meet in a butterfly (xor 32, 16, ..., 1) -- the
// MoE router's order (k_moe_router, iq_moe.hip), so an F32 router matrix
// gives the router's logits bit for bit.  BF16 weights widen to f32
// exactly first.  Every pair is formed the same way at any row count.
#include "iq_device.h"
#include "iq_internal.h"

namespace iq {

namespace {

// Grid (ceil(n / 4), ceil(m / TT)): wave w of workgroup b takes weight row
// 4 b + w against the tile's TT input rows; its row streams once per tile
// with U loads in flight per lane (one input row: U = 32, a 2048-wide row
// in one round trip), the input rows come from L2.
template <bool BF16, int TT, int U>
__global__ __launch_bounds__(256) void k_float_mm(const uint8_t* __restrict__ w, int64_t n, int64_t k,
                                                  const float* __restrict__ x, int64_t ldx, int m,
                                                  float* __restrict__ y, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wave
    const int t0 = (int)blockIdx.y * TT, nt = min(TT, m - t0);
    auto wv = [&](int64_t h) -> float {
        if constexpr (BF16) return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)w)[row * k + h] << 16);
        else return ((const float*)w)[row * k + h];
    };
    float part[TT];
#pragma unroll
    for (int i = 0; i < TT; i++) part[i] = 0.f;
    int64_t h = lane;
    for (; h + 64 * (U - 1) < k; h += 64 * U) {
        float rv[U];
#pragma unroll
        for (int j = 0; j < U; j++) rv[j] = wv(h + 64 * j);
#pragma unroll
        for (int i = 0; i < TT; i++) {
            if (i < nt) {
                const float* xr = x + (int64_t)(t0 + i) * ldx + h;
                float xv[U];
#pragma unroll
                for (int j = 0; j < U; j++) xv[j] = xr[64 * j];
#pragma unroll
                for (int j = 0; j < U; j++) part[i] = part[i] + xv[j] * rv[j];
            }
        }
    }
    for (; h < k; h += 64) {
        const float rv = wv(h);
#pragma unroll
        for (int i = 0; i < TT; i++)
            if (i < nt) part[i] = part[i] + x[(int64_t)(t0 + i) * ldx + h] * rv;
    }
#pragma unroll
    for (int i = 0; i < TT; i++) {
        float v = part[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
        if (lane == 0 && i < nt) y[(int64_t)(t0 + i) * ldy + row] = v;
    }
}

}  // namespace

hipError_t launch_float_mm(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                           hipStream_t s) {
    if ((w.dtype != kF32 && w.dtype != kBF16) || m < 1 || w.rows < 1 || w.cols < 1) return hipErrorNotSupported;
    const int tt = m == 1 ? 1 : 8;
    const int64_t gx = (w.rows + 3) / 4, gy = (m + tt - 1) / tt;
    if (gx > 0x7fffffff || gy > 65535) return hipErrorNotSupported;
    const dim3 grid((unsigned)gx, (unsigned)gy);
    const bool bf = w.dtype == kBF16;
    if (m == 1) {
        if (bf) hipLaunchKernelGGL((k_float_mm<true, 1, 32>), grid, dim3(256), 0, s, w.w, w.rows, w.cols, x, ldx, 1, y, ldy);
        else hipLaunchKernelGGL((k_float_mm<false, 1, 32>), grid, dim3(256), 0, s, w.w, w.rows, w.cols, x, ldx, 1, y, ldy);
    } else {
        if (bf) hipLaunchKernelGGL((k_float_mm<true, 8, 8>), grid, dim3(256), 0, s, w.w, w.rows, w.cols, x, ldx, (int)m, y, ldy);
        else hipLaunchKernelGGL((k_float_mm<false, 8, 8>), grid, dim3(256), 0, s, w.w, w.rows, w.cols, x, ldx, (int)m, y, ldy);
    }
    return hipGetLastError();
}

}  // namespace iq
