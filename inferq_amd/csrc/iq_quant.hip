// iq_quant.hip -- launchers of the activation quantisers (iq_quant.h):
// one wave per 256-value group of one row.
#include "iq_quant.h"

namespace iq {

namespace {

__global__ __launch_bounds__(256) void k_quant_q8k(const float* __restrict__ x, int64_t ldx, int64_t m, int ng,
                                                   ActView a, uint8_t* __restrict__ ref) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= m * ng) return;  // uniform per wave
    const int64_t row = wid / ng;
    const int g = (int)(wid % ng);
    quant_q8k_wave(x + row * ldx + (int64_t)g * 256, row, g, a, ref ? ref + (row * ng + g) * 292 : nullptr);
}

__global__ __launch_bounds__(256) void k_quant_q80(const float* __restrict__ x, int64_t ldx, int64_t m, int64_t k,
                                                   int ng, ActView a, uint8_t* __restrict__ ref) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= m * ng) return;
    const int64_t row = wid / ng;
    const int g = (int)(wid % ng);
    quant_q80_wave(x + row * ldx, k, row, g, a, ref ? ref + row * (k / 32) * 34 : nullptr);
}

constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

size_t act_bytes(int64_t m, int64_t k) {
    const int64_t ng = (k + 255) / 256;
    const int64_t ldq = ng * 256, ldd = ng * 8;
    return align256((size_t)(m * ldq)) + align256((size_t)(m * ldd) * 4) + align256((size_t)(m * ng * 8) * 2);
}

ActView act_carve(void* base, int64_t m, int64_t k) {
    ActView a;
    a.ng = (int)((k + 255) / 256);
    a.ldq = (int64_t)a.ng * 256;
    a.ldd = (int64_t)a.ng * 8;
    a.m = (int)m;
    uint8_t* p = (uint8_t*)base;
    a.q = (int8_t*)p;
    p += align256((size_t)(m * a.ldq));
    a.d = (float*)p;
    p += align256((size_t)(m * a.ldd) * 4);
    a.s8 = (int16_t*)p;
    return a;
}

hipError_t launch_quant_q8k(const float* x, int64_t ldx, int64_t m, int64_t k, const ActView& a, uint8_t* ref,
                            hipStream_t s) {
    const int ng = (int)(k / 256);
    const int64_t waves = m * ng;
    if (waves == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quant_q8k, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, ldx, m, ng, a, ref);
    return hipGetLastError();
}

hipError_t launch_quant_q80(const float* x, int64_t ldx, int64_t m, int64_t k, const ActView& a, uint8_t* ref,
                            hipStream_t s) {
    const int ng = (int)((k + 255) / 256);
    const int64_t waves = m * ng;
    if (waves == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quant_q80, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, ldx, m, k, ng, a, ref);
    return hipGetLastError();
}

}  // namespace iq
