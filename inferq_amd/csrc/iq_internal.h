// iq_internal.h -- host-side declarations shared by the library's sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace iq {

// GGML type ids (GGUF dtype codes).
constexpr int kF32 = 0;
constexpr int kQ8_0 = 8;
constexpr int kQ4_K = 12;
constexpr int kQ5_K = 13;
constexpr int kQ6_K = 14;
constexpr int kBF16 = 30;

// Quantised activations in the internal (lane-transposed) layout.
struct ActView {
    int8_t* q = nullptr;     // [m][ldq] int8, 256-value groups lane-transposed
    float* d = nullptr;      // [m][ldd] scale per block (Q8K: per 256; Q8_0: per 32)
    int16_t* s8 = nullptr;   // [m][ng][8] Q8K 32-value sub-block sums (K-quants only)
    int64_t ldq = 0, ldd = 0;
    int ng = 0;              // 256-value groups per row
    int m = 0;
};

// Bytes of workspace an ActView of m rows and width k needs (all parts,
// each 256-byte aligned).
size_t act_bytes(int64_t m, int64_t k);
// Carve an ActView out of `base` (which holds at least act_bytes(m, k)).
ActView act_carve(void* base, int64_t m, int64_t k);

// Activation quantisers.  x is f32 [m][ldx]; `ref`, when not null, also
// receives the reference block layout (292-byte Q8K or 34-byte Q8_0 blocks,
// [m][k/256] or [m][k/32]).
hipError_t launch_quant_q8k(const float* x, int64_t ldx, int64_t m, int64_t k, const ActView& a, uint8_t* ref,
                            hipStream_t s);
hipError_t launch_quant_q80(const float* x, int64_t ldx, int64_t m, int64_t k, const ActView& a, uint8_t* ref,
                            hipStream_t s);

// Weight matrix in native GGUF block layout.
struct WeightView {
    const uint8_t* w = nullptr;
    int dtype = 0;
    int64_t rows = 0, cols = 0, row_bytes = 0;
};

// y[m][ldy] = act . W^T with the reference's exact f32 order.  When isum is
// not null, the per-block lane integers are also written:
// isum [m][rows][blocks][8], msum [m][rows][blocks][4] (Q4_K only).
hipError_t launch_matmul_lanes(const WeightView& w, const ActView& a, float* y, int64_t ldy, int32_t* isum,
                               int32_t* msum, hipStream_t s);

// The LDS-staged kernel for many output rows at 1..8 input rows
// (iq_gemv.hip); it quantises the f32 input rows x [m][ldx] itself.
// gemv_supported tells whether it covers a shape; launch_gemv returns
// hipErrorNotSupported when it does not.
bool gemv_supported(const WeightView& w, int64_t m);
hipError_t launch_gemv(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                       hipStream_t s);

// The int8-MFMA prefill-tile kernel for Q4_K weights at kPrefillMinRows or
// more input rows (iq_prefill.hip): per-block integers exact, f32
// combination in its own order, so only an explicit request runs it.  launch_prefill quantises x itself into `ws` (at least
// prefill_workspace_size bytes); dbg_isum / dbg_msum, when not null, receive
// the per-block integer totals [m][rows][cols / 256].
constexpr int64_t kPrefillMinRows = 64;
bool prefill_supported(const WeightView& w, int64_t m);
size_t prefill_workspace_size(const WeightView& w, int64_t m);
hipError_t launch_prefill(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                          void* ws, int32_t* dbg_isum, int32_t* dbg_msum, hipStream_t s);

// The exact lane-order int8-MFMA kernel for Q4_K / Q6_K matrices
// (iq_dense_mfma.hip): bitwise the one-row results.  dense_mfma_supported
// says where the dispatch uses it (large matrices at 2..63 input rows, every
// readable matrix from kPrefillMinRows rows); launch_dense_mfma_any runs it
// at any row count on any matrix whose layout it can read.  Both quantise x
// themselves into `ws` (at least dense_mfma_workspace_any bytes).
bool dense_mfma_supported(const WeightView& w, int64_t m);
size_t dense_mfma_workspace_any(const WeightView& w, int64_t m);
hipError_t launch_dense_mfma(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                             void* ws, hipStream_t s);
hipError_t launch_dense_mfma_any(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                                 void* ws, hipStream_t s);

// y[m][ldy] = x . W^T for F32 and BF16 matrices (iq_dense_f32.hip), in the
// MoE router's f32 order; hipErrorNotSupported for other dtypes.
hipError_t launch_float_mm(const WeightView& w, const float* x, int64_t ldx, int64_t m, float* y, int64_t ldy,
                           hipStream_t s);

// Greedy selection over logit rows y [m][ldy] (iq_argmax.hip): idx[r] the
// last index of the largest finite value of row r (-1 when none is finite),
// val[r] (may be null) that value.  `ws` holds argmax_workspace_size bytes.
size_t argmax_workspace_size(int64_t m, int64_t n);
hipError_t launch_argmax(const float* y, int64_t m, int64_t n, int64_t ldy, int32_t* idx, float* val, void* ws,
                         hipStream_t s);

// Greedy selection fused into the product.  Where gemv_argmax_supported
// (one input row, iq_gemv.hip), launch_gemv_argmax computes y = x . W^T as
// launch_gemv does (the same bits) and also leaves each wave's largest
// (argmax key, logit) pair of its rows in keys / vals, *nparts of them (at
// most gemv_argmax_parts).  Where dense_argmax_supported (2..8 input rows on
// the pair-lane MFMA tile, iq_dense_mfma.hip), launch_dense_argmax does the
// same per workgroup and input row: pair (r, b) at r * dense_argmax_parts +
// b, with `ws` as launch_dense_mfma's.  launch_argmax_kv (iq_argmax.hip)
// then reduces m rows of nparts pairs to each row's index and value, as
// launch_argmax would from y.
bool gemv_argmax_supported(const WeightView& w);
int64_t gemv_argmax_parts(const WeightView& w);
hipError_t launch_gemv_argmax(const WeightView& w, const float* x, float* y, uint64_t* keys, float* vals, int* nparts,
                              hipStream_t s);
bool dense_argmax_supported(const WeightView& w, int64_t m);
int64_t dense_argmax_parts(const WeightView& w);
hipError_t launch_dense_argmax(const WeightView& w, const float* x, int64_t m, float* y, void* ws, uint64_t* keys,
                               float* vals, hipStream_t s);
hipError_t launch_argmax_kv(const uint64_t* keys, const float* vals, int64_t m, int nparts, int32_t* idx, float* val,
                            hipStream_t s);

}  // namespace iq
