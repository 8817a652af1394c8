// iq_rowcompat.cpp -- the reference's per-row kernel entries with their
// argument order (q4k_q8k_row / q6k_q8k_row / q80_q80_row,
// src/qgemm.rs:447-468): one weight row of GGUF blocks against `rows` input
// rows that the caller has already quantised (Q8K or Q8_0 blocks, block-major:
// inputs[block * rows + r]), host slices in and out.  The blocks are copied to
// the device, converted to the lane-transposed activation layout, and run on
// the lane kernel; outputs are bitwise the reference kernel's.  For callers
// that keep the per-row structure (unit tests, a CPU code path being moved
// over piecewise): a matrix-level entry (iq_matmul) is the fast path.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/iq_qgemm.h"
#include "iq_api_internal.h"
#include "iq_device.h"

#define IQ_API extern "C" __attribute__((visibility("default")))

namespace iq {

namespace {

constexpr size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

// Q8K block (292 B: f32 d, int8 qs[256], int16 bsums[16]) of input row r,
// block b -> the lane-transposed group b of activation row r; one wave per
// (r, b).  The 32-value sums are the pairs of the 16-value bsums.
__global__ __launch_bounds__(256) void k_q8k_blocks_to_act(const uint8_t* __restrict__ in, int64_t rows, int nb,
                                                          ActView a) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= rows * nb) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t b = wid / rows, r = wid - b * rows;
    const uint8_t* blk = in + (b * rows + r) * 292;
    const int c = lane >> 3, k = lane & 7;
    const uint32_t q = *(const uint32_t*)(blk + 4 + 4 * lane);  // values 4 lane .. +3 = chunk c, lane k
    ((uint32_t*)(a.q + r * a.ldq + b * 256))[8 * k + c] = q;
    if (lane == 0) a.d[r * a.ldd + b] = *(const float*)blk;
    if (lane < 8) {
        const int16_t* bs = (const int16_t*)(blk + 260);
        a.s8[(r * a.ng + b) * 8 + lane] = (int16_t)(bs[2 * lane] + bs[2 * lane + 1]);
    }
}

// Q8_0 blocks (34 B: f16 d, int8 qs[32]) of input row r: 32-value block
// b32 = 8 g + c of group g; one wave per (r, g).
__global__ __launch_bounds__(256) void k_q80_blocks_to_act(const uint8_t* __restrict__ in, int64_t rows, int nb32,
                                                          int ng, ActView a) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= rows * ng) return;  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int64_t g = wid / rows, r = wid - g * rows;
    const int c = lane >> 3, k = lane & 7;
    const int64_t b32 = g * 8 + c;
    uint32_t q = 0;
    if (b32 < nb32) {
        const uint8_t* blk = in + (b32 * rows + r) * 34;
        q = ld32_a2(blk + 2 + 4 * k);
        if (k == 0) a.d[r * a.ldd + b32] = f16_to_f32(ld16(blk));
    }
    ((uint32_t*)(a.q + r * a.ldq + g * 256))[8 * k + c] = q;
}

int row_entry(int dtype, const void* weight, size_t weight_blocks, const void* inputs, size_t input_blocks,
              size_t rows, float* out, size_t out_len) {
    const char* name = dtype == kQ4_K ? "q4k_q8k_row" : dtype == kQ6_K ? "q6k_q8k_row" : "q80_q80_row";
    if (!weight || !inputs || !out) return fail(IQ_ERR_INVALID, "%s: null slice", name);
    // the reference's preconditions (src/qgemm.rs:450-451)
    if (out_len != rows) return fail(IQ_ERR_SHAPE, "%s: out.len() %zu != rows %zu", name, out_len, rows);
    if (input_blocks != rows * weight_blocks)
        return fail(IQ_ERR_SHAPE, "%s: inputs.len() %zu != rows %zu x weight.len() %zu", name, input_blocks, rows,
                    weight_blocks);
    if (rows == 0 || weight_blocks == 0) {
        for (size_t i = 0; i < out_len; i++) out[i] = 0.f;  // an empty dot
        return IQ_OK;
    }
    const int64_t be = dtype == kQ8_0 ? 32 : 256;
    const int64_t K = (int64_t)weight_blocks * be;
    const size_t wbytes = weight_blocks * (size_t)block_bytes(dtype);
    const size_t ibytes = input_blocks * (dtype == kQ8_0 ? 34 : 292);
    const size_t wo = 0, io = wo + a256(wbytes + 256), ao = io + a256(ibytes), yo = ao + a256(act_bytes(rows, K));
    const size_t total = yo + a256(rows * 4);
    WsLease lease;
    if (int rc = lease.acquire(total, nullptr)) return rc;
    uint8_t* base = (uint8_t*)lease.ptr();
    hipError_t e = hipMemcpy(base + wo, weight, wbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(base + wo + wbytes, 0, 256);
    if (e == hipSuccess) e = hipMemcpy(base + io, inputs, ibytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (per-row entry inputs)");
    ActView a = act_carve(base + ao, (int64_t)rows, K);
    if (dtype == kQ8_0) {
        const int64_t waves = (int64_t)rows * a.ng;
        hipLaunchKernelGGL(k_q80_blocks_to_act, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, nullptr, base + io,
                           (int64_t)rows, (int)weight_blocks, a.ng, a);
    } else {
        const int64_t waves = (int64_t)rows * (int64_t)weight_blocks;
        hipLaunchKernelGGL(k_q8k_blocks_to_act, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, nullptr, base + io,
                           (int64_t)rows, (int)weight_blocks, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "per-row entry conversion launch");
    WeightView w;
    w.w = base + wo;
    w.dtype = dtype;
    w.rows = 1;
    w.cols = K;
    w.row_bytes = (int64_t)wbytes;
    e = launch_matmul_lanes(w, a, (float*)(base + yo), 1, nullptr, nullptr, nullptr);
    if (e != hipSuccess) return hip_fail(e, "per-row entry launch");
    e = hipMemcpy(out, base + yo, rows * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (per-row entry output)");
    return IQ_OK;
}

}  // namespace

}  // namespace iq

using namespace iq;

IQ_API int iq_q4k_q8k_row(const void* weight, size_t weight_blocks, const void* inputs, size_t input_blocks,
                          size_t rows, float* out, size_t out_len) {
    return row_entry(kQ4_K, weight, weight_blocks, inputs, input_blocks, rows, out, out_len);
}

IQ_API int iq_q6k_q8k_row(const void* weight, size_t weight_blocks, const void* inputs, size_t input_blocks,
                          size_t rows, float* out, size_t out_len) {
    return row_entry(kQ6_K, weight, weight_blocks, inputs, input_blocks, rows, out, out_len);
}

IQ_API int iq_q80_q80_row(const void* weight, size_t weight_blocks, const void* inputs, size_t input_blocks,
                          size_t rows, float* out, size_t out_len) {
    return row_entry(kQ8_0, weight, weight_blocks, inputs, input_blocks, rows, out, out_len);
}
