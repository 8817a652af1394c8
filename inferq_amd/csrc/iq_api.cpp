// iq_api.cpp -- the C ABI (include/iq_qgemm.h): handles, validation that
// mirrors the reference's load- and call-time checks, workspaces and
// dispatch to the kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstddef>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/iq_qgemm.h"
#include "iq_api_internal.h"
#include "iq_internal.h"

#define IQ_API extern "C" __attribute__((visibility("default")))

namespace iq {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(IQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

const char* dtype_name(int dtype) {
    switch (dtype) {
    case kF32: return "F32";
    case kBF16: return "BF16";
    case kQ4_K: return "Q4K";
    case kQ5_K: return "Q5K";
    case kQ6_K: return "Q6K";
    case kQ8_0: return "Q8_0";
    default: return "unknown";
    }
}

bool float_dtype(int dtype) { return dtype == kF32 || dtype == kBF16; }
int64_t block_elems(int dtype) { return float_dtype(dtype) ? 1 : dtype == kQ8_0 ? 32 : 256; }
int64_t block_bytes(int dtype) {
    return dtype == kF32 ? 4 : dtype == kBF16 ? 2 : dtype == kQ4_K ? 144 : dtype == kQ5_K ? 176 : dtype == kQ6_K ? 210 : 34;
}
bool dtype_ok(int dtype) {
    return dtype == kQ4_K || dtype == kQ5_K || dtype == kQ6_K || dtype == kQ8_0 || float_dtype(dtype);
}
bool moe_dtype_ok(int dtype) { return dtype == kQ4_K || dtype == kQ5_K || dtype == kQ6_K || dtype == kQ8_0; }

namespace {

std::mutex g_ws_mu;
struct Workspace {
    int device = -1;
    hipStream_t stream = nullptr;
    void* p = nullptr;
    size_t bytes = 0;
    // Buffers this workspace outgrew.  Graphs captured on the stream keep
    // their addresses, so they stay allocated until iq_workspace_release.
    std::vector<void*> retired;
};
std::vector<Workspace> g_ws;

int current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    return IQ_OK;
}

}  // namespace

int WsLease::acquire(size_t bytes, hipStream_t stream) {
    int dev;
    if (int rc = current_device(&dev)) return rc;
    lock_ = std::unique_lock<std::mutex>(g_ws_mu);
    Workspace* w = nullptr;
    for (Workspace& c : g_ws)
        if (c.device == dev && c.stream == stream) w = &c;
    if (!w) {
        g_ws.push_back(Workspace{dev, stream, nullptr, 0, {}});
        w = &g_ws.back();
    }
    if (w->bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return fail(IQ_ERR_INVALID,
                        "the library workspace of this stream must grow to %zu bytes, which cannot happen during "
                        "graph capture: call iq_matmul_reserve (or make one eager call of the same size) on the "
                        "stream first, or pass a workspace (iq_matmul_ws)",
                        bytes);
        // at least 1 MiB, and at least double the old size, so that a run of
        // growing calls retires few buffers
        size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
        if (w->bytes && want < 2 * w->bytes) want = 2 * w->bytes;
        void* np = nullptr;
        e = hipMalloc(&np, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            if (want > bytes) e = hipMalloc(&np, want = bytes);  // doubling may not fit where the need does
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return fail(IQ_ERR_OOM, "workspace allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
            }
        }
        // earlier launches (and captured graphs) may still read the old
        // buffer: it is retired, not freed
        if (w->p) w->retired.push_back(w->p);
        w->p = np;
        w->bytes = want;
    }
    p_ = w->p;
    return IQ_OK;
}

// Free the workspaces of `stream` on the current device (the live one and
// every retired one), after the stream's work has finished.
int release_workspace(hipStream_t stream) {
    int dev;
    if (int rc = current_device(&dev)) return rc;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (size_t i = 0; i < g_ws.size(); i++) {
        Workspace& w = g_ws[i];
        if (w.device != dev || w.stream != stream) continue;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return fail(IQ_ERR_INVALID, "a stream's workspace cannot be released during graph capture");
        e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        if (w.p) (void)hipFree(w.p);
        for (void* r : w.retired) (void)hipFree(r);
        g_ws.erase(g_ws.begin() + (std::ptrdiff_t)i);
        return IQ_OK;
    }
    return IQ_OK;
}

// ---- allocation-free products (iq_matmul_noalloc) ----
// A fixed device array serves as the workspace of iq_matmul_noalloc, for
// callers that must not allocate (graph capture, serving loops).  Each
// device holds its own copy for the life of the process; its address on a
// device comes from hipGetSymbolAddress with that device current (the
// array's name is not a device address in host code).  Every call on a
// device shares its copy: such calls must not overlap in time on one device.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device, null until resolved
}  // namespace

// Resolve (once per device) the current device's address of `scratch`.
int scratch_ptr(void** out) {
    int dev;
    if (int rc = current_device(&dev)) return rc;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((size_t)dev >= g_scratch_ptr.size()) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress (scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return IQ_OK;
}

int check_weight(const iq_weight* w) {
    if (!w || !w->dev) return fail(IQ_ERR_INVALID, "null quantized matrix handle");
    return IQ_OK;
}

WeightView view_of(const iq_weight* w) {
    WeightView v;
    v.w = w->dev;
    v.dtype = w->dtype;
    v.rows = w->rows;
    v.cols = w->cols;
    v.row_bytes = w->row_bytes;
    return v;
}

// Validated shape and size of a GGUF matrix (mirrors QuantizedMatrix::new,
// src/gguf.rs:297-320, and the block-count checks of fused_forward,
// src/gguf.rs:627-646).
int check_matrix(int dtype, int64_t rows, int64_t cols, size_t nbytes, int64_t* row_bytes) {
    if (!dtype_ok(dtype))
        return fail(IQ_ERR_DTYPE,
                    "unsupported executable GGUF matrix dtype %d; expected Q4_K, Q5_K, Q6_K, Q8_0, F32, or BF16", dtype);
    if (rows <= 0 || cols <= 0) return fail(IQ_ERR_SHAPE, "invalid matrix shape [%lld, %lld]", (long long)rows,
                                             (long long)cols);
    if (cols % block_elems(dtype))
        return fail(IQ_ERR_SHAPE, "GGUF matrix width %lld is not divisible by %s block size %lld", (long long)cols,
                    dtype_name(dtype), (long long)block_elems(dtype));
    const int64_t rb = cols / block_elems(dtype) * block_bytes(dtype);
    if ((size_t)(rows * rb) != nbytes)
        return fail(IQ_ERR_SHAPE, "quantized matrix has %zu bytes, expected %lld for [%lld, %lld] %s", nbytes,
                    (long long)(rows * rb), (long long)rows, (long long)cols, dtype_name(dtype));
    *row_bytes = rb;
    return IQ_OK;
}

int alloc_weight(int dtype, int64_t rows, int64_t cols, int64_t row_bytes, iq_weight** out) {
    // 256 zeroed padding bytes keep every vector load of the last block
    // inside the allocation.
    const size_t bytes = (size_t)(rows * row_bytes);
    uint8_t* dev = nullptr;
    hipError_t e = hipMalloc(&dev, bytes + 256);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(IQ_ERR_OOM, "allocation of %zu bytes for a [%lld, %lld] %s matrix failed: %s", bytes,
                    (long long)rows, (long long)cols, dtype_name(dtype), hipGetErrorString(e));
    }
    e = hipMemset(dev + bytes, 0, 256);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "hipMemset");
    }
    iq_weight* w = new iq_weight;
    w->dtype = dtype;
    w->rows = rows;
    w->cols = cols;
    w->row_bytes = row_bytes;
    w->nbytes = bytes;
    w->dev = dev;
    w->owned = true;
    (void)hipGetDevice(&w->device);
    *out = w;
    return IQ_OK;
}

// Quantise m rows of device x for W's activation format into `a`.
int quantize_for(const iq_weight* w, const float* x, int64_t m, const ActView& a, uint8_t* ref, hipStream_t s) {
    hipError_t e = w->dtype == kQ8_0 ? launch_quant_q80(x, w->cols, m, w->cols, a, ref, s)
                                     : launch_quant_q8k(x, w->cols, m, w->cols, a, ref, s);
    if (e != hipSuccess) return hip_fail(e, "activation quantisation launch");
    return IQ_OK;
}

// Device workspace a product of m rows needs (activation quantisation, and
// for the int8-MFMA path its layouts and split-K partial tiles).
size_t matmul_ws_bytes(const iq_weight* w, int64_t m) {
    if (float_dtype(w->dtype)) return 0;  // the f32 product reads x as it is
    const size_t a = act_bytes(m, w->cols), p = prefill_workspace_size(view_of(w), m);
    const size_t d = dense_mfma_workspace_any(view_of(w), m);
    const size_t ap = a > p ? a : p;
    return ap > d ? ap : d;
}

// Greedy selection fused into the product (iq_matmul_argmax): 1 = one row
// on the four-row-item GEMV, 2 = 2..8 rows on the pair-lane MFMA tile, 0 =
// none (the product, then launch_argmax over its logits).
int argmax_fusion(const iq_weight* w, int64_t m) {
    const WeightView v = view_of(w);
    if (m == 1 && gemv_argmax_supported(v)) return 1;
    if (dense_argmax_supported(v, m)) return 2;
    return 0;
}

// (key, logit) pairs per input row of a fused selection.
int64_t argmax_fused_parts(const iq_weight* w, int64_t m) {
    const int f = argmax_fusion(w, m);
    return f == 1 ? gemv_argmax_parts(view_of(w)) : f == 2 ? dense_argmax_parts(view_of(w)) : 0;
}

// Workspace of iq_matmul_argmax: the logits, then either the argmax
// partials and the product's own workspace or, fused, the pairs (keys,
// then logits) and the product's workspace.
size_t argmax_call_bytes(const iq_weight* w, int64_t m) {
    const size_t yb = ((size_t)(m * w->rows) * 4 + 255) & ~(size_t)255;
    const size_t ab = (argmax_workspace_size(m, w->rows) + 255) & ~(size_t)255;
    const size_t rest = ab + matmul_ws_bytes(w, m);
    const size_t P = (size_t)(m * argmax_fused_parts(w, m));
    const size_t fused = P ? ((P * 8 + 255) & ~(size_t)255) + ((P * 4 + 255) & ~(size_t)255) + matmul_ws_bytes(w, m)
                           : 0;
    return yb + (rest > fused ? rest : fused);
}

// Kernel choice of a product (iq_matmul_via's path argument).  Every path
// but IQ_PATH_PREFILL_TILES gives the reference's result bit for bit.
hipError_t launch_path(const iq_weight* w, const float* x, int64_t m, float* y, void* ws, int path, int32_t* isum,
                       int32_t* msum, hipStream_t s) {
    const WeightView v = view_of(w);
    hipError_t e = hipErrorNotSupported;
    // F32 / BF16: one f32 product, no fixed kernel paths (the reference has
    // no multi-row kernel for them either) and no per-block integers
    if (float_dtype(w->dtype))
        return path == IQ_PATH_AUTO && !isum ? launch_float_mm(v, x, w->cols, m, y, w->rows, s) : hipErrorNotSupported;
    if (path == IQ_PATH_AUTO) {
        if (!isum && dense_mfma_supported(v, m)) e = launch_dense_mfma(v, x, w->cols, m, y, w->rows, ws, s);
        if (e == hipErrorNotSupported && !isum && gemv_supported(v, m)) e = launch_gemv(v, x, w->cols, m, y, w->rows, s);
    } else if (path == IQ_PATH_GEMV) {
        e = launch_gemv(v, x, w->cols, m, y, w->rows, s);
    } else if (path == IQ_PATH_LANE_MFMA) {
        e = launch_dense_mfma_any(v, x, w->cols, m, y, w->rows, ws, s);
    } else if (path == IQ_PATH_PREFILL_TILES) {
        e = launch_prefill(v, x, w->cols, m, y, w->rows, ws, nullptr, nullptr, s);
    }
    if (e == hipErrorNotSupported && (path == IQ_PATH_AUTO || path == IQ_PATH_LANES)) {
        ActView a = act_carve(ws, m, w->cols);
        e = w->dtype == kQ8_0 ? launch_quant_q80(x, w->cols, m, w->cols, a, nullptr, s)
                              : launch_quant_q8k(x, w->cols, m, w->cols, a, nullptr, s);
        if (e == hipSuccess) e = launch_matmul_lanes(v, a, y, w->rows, isum, msum, s);
    }
    return e;
}

const char* path_name(int path) {
    switch (path) {
    case IQ_PATH_AUTO: return "auto";
    case IQ_PATH_LANES: return "lanes";
    case IQ_PATH_GEMV: return "gemv";
    case IQ_PATH_LANE_MFMA: return "lane-order MFMA";
    case IQ_PATH_PREFILL_TILES: return "prefill tiles";
    default: return "unknown";
    }
}

int matmul_impl(const iq_weight* w, const float* x, int64_t m, float* y, void* ws, size_t ws_bytes, int path,
                int32_t* isum, int32_t* msum, hipStream_t s) {
    if (int rc = check_weight(w)) return rc;
    if (m < 0) return fail(IQ_ERR_SHAPE, "negative input row count %lld", (long long)m);
    if (path < IQ_PATH_AUTO || path > IQ_PATH_PREFILL_TILES) return fail(IQ_ERR_INVALID, "unknown matmul path %d", path);
    if (m == 0) return IQ_OK;
    if (!x || !y) return fail(IQ_ERR_INVALID, "null input or output pointer");
    const size_t need = matmul_ws_bytes(w, m);
    WsLease lease;  // held until the launches below are enqueued
    if (!ws) {
        if (int rc = lease.acquire(need, s)) return rc;
        ws = lease.ptr();
    } else if (ws_bytes < need) {
        return fail(IQ_ERR_SHAPE, "workspace of %zu bytes is smaller than the %zu bytes needed", ws_bytes, need);
    }
    const hipError_t e = launch_path(w, x, m, y, ws, path, isum, msum, s);
    if (e == hipErrorNotSupported)
        return fail(IQ_ERR_DTYPE, "%s has no %s kernel for %lld input rows of a [%lld, %lld] matrix", dtype_name(w->dtype),
                    path_name(path), (long long)m, (long long)w->rows, (long long)w->cols);
    if (e != hipSuccess) return hip_fail(e, "matmul launch");
    return IQ_OK;
}

}  // namespace iq

using namespace iq;

IQ_API const char* iq_version(void) { return "inferq-amd 0.1 (gfx950)"; }

IQ_API const char* iq_last_error(void) { return g_err.c_str(); }

IQ_API int iq_init(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(IQ_ERR_RANGE, "device %d out of range (%d devices)", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(IQ_ERR_HIP, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    void* sp;
    return scratch_ptr(&sp);  // set-up of the allocation-free entry on this device
}

IQ_API int iq_weights_upload(const void* host_bytes, size_t nbytes, int dtype, int64_t rows, int64_t cols,
                             iq_weight_t* out) {
    if (!host_bytes || !out) return fail(IQ_ERR_INVALID, "null pointer");
    int64_t rb;
    if (int rc = check_matrix(dtype, rows, cols, nbytes, &rb)) return rc;
    iq_weight* w;
    if (int rc = alloc_weight(dtype, rows, cols, rb, &w)) return rc;
    hipError_t e = hipMemcpy(w->dev, host_bytes, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w->dev);
        delete w;
        return hip_fail(e, "hipMemcpy (weights upload)");
    }
    *out = w;
    return IQ_OK;
}

IQ_API int iq_weights_view(const void* device_bytes, size_t nbytes, int dtype, int64_t rows, int64_t cols,
                           iq_weight_t* out) {
    if (!device_bytes || !out) return fail(IQ_ERR_INVALID, "null pointer");
    if ((uintptr_t)device_bytes & 15u)
        return fail(IQ_ERR_INVALID, "device matrix bytes must be 16-byte aligned");
    int64_t rb;
    if (int rc = check_matrix(dtype, rows, cols, nbytes, &rb)) return rc;
    iq_weight* w = new iq_weight;
    w->dtype = dtype;
    w->rows = rows;
    w->cols = cols;
    w->row_bytes = rb;
    w->nbytes = nbytes;
    w->dev = (uint8_t*)device_bytes;
    w->owned = false;
    (void)hipGetDevice(&w->device);
    *out = w;
    return IQ_OK;
}

IQ_API int iq_weights_free(iq_weight_t w) {
    if (!w) return IQ_OK;
    if (w->owned && w->dev) (void)hipFree(w->dev);
    delete w;
    return IQ_OK;
}

IQ_API int iq_weights_info(iq_weight_t w, int* dtype, int64_t* rows, int64_t* cols, size_t* nbytes,
                           const void** device_bytes) {
    if (int rc = check_weight(w)) return rc;
    if (dtype) *dtype = w->dtype;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (nbytes) *nbytes = w->nbytes;
    if (device_bytes) *device_bytes = w->dev;
    return IQ_OK;
}

IQ_API int iq_weights_concat_rows(iq_weight_t a, iq_weight_t b, iq_weight_t* out) {
    if (int rc = check_weight(a)) return rc;
    if (int rc = check_weight(b)) return rc;
    if (!out) return fail(IQ_ERR_INVALID, "null output handle");
    if (a->dtype != b->dtype)
        return fail(IQ_ERR_DTYPE, "cannot concatenate quantized matrices with dtypes %s and %s", dtype_name(a->dtype),
                    dtype_name(b->dtype));
    if (a->cols != b->cols)
        return fail(IQ_ERR_SHAPE, "cannot concatenate quantized matrices with %lld and %lld columns",
                    (long long)a->cols, (long long)b->cols);
    iq_weight* w;
    if (int rc = alloc_weight(a->dtype, a->rows + b->rows, a->cols, a->row_bytes, &w)) return rc;
    hipError_t e = hipMemcpy(w->dev, a->dev, a->nbytes, hipMemcpyDeviceToDevice);
    if (e == hipSuccess) e = hipMemcpy(w->dev + a->nbytes, b->dev, b->nbytes, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w->dev);
        delete w;
        return hip_fail(e, "hipMemcpy (concatenate_rows)");
    }
    *out = w;
    return IQ_OK;
}

IQ_API int iq_weights_leading_rows(iq_weight_t a, int64_t rows, iq_weight_t* out) {
    if (int rc = check_weight(a)) return rc;
    if (!out) return fail(IQ_ERR_INVALID, "null output handle");
    if (rows <= 0 || rows > a->rows)
        return fail(IQ_ERR_RANGE, "cannot take %lld leading rows of a %lld-row matrix", (long long)rows,
                    (long long)a->rows);
    iq_weight* w;
    if (int rc = alloc_weight(a->dtype, rows, a->cols, a->row_bytes, &w)) return rc;
    hipError_t e = hipMemcpy(w->dev, a->dev, (size_t)(rows * a->row_bytes), hipMemcpyDeviceToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w->dev);
        delete w;
        return hip_fail(e, "hipMemcpy (leading_rows)");
    }
    *out = w;
    return IQ_OK;
}

IQ_API int iq_matmul(iq_weight_t w, const float* x, int64_t m, float* y, iq_stream_t stream) {
    return matmul_impl(w, x, m, y, nullptr, 0, IQ_PATH_AUTO, nullptr, nullptr, (hipStream_t)stream);
}

IQ_API int iq_matmul_via(iq_weight_t w, const float* x, int64_t m, float* y, int path, iq_stream_t stream) {
    return matmul_impl(w, x, m, y, nullptr, 0, path, nullptr, nullptr, (hipStream_t)stream);
}

IQ_API int iq_matmul_noalloc(iq_weight_t w, const float* x, int64_t m, float* y, iq_stream_t stream) {
    if (int rc = check_weight(w)) return rc;
    if (m < 0) return fail(IQ_ERR_SHAPE, "negative input row count %lld", (long long)m);
    if (m == 0) return IQ_OK;
    if (!x || !y) return fail(IQ_ERR_INVALID, "null input or output pointer");
    const size_t need = matmul_ws_bytes(w, m);
    if (need > kScratchBytes)
        return fail(IQ_ERR_RANGE,
                    "%lld input rows of a [%lld, %lld] %s matrix need %zu bytes of scratch; iq_matmul_noalloc has %zu "
                    "(use iq_matmul or iq_matmul_ws, or split the rows)",
                    (long long)m, (long long)w->rows, (long long)w->cols, dtype_name(w->dtype), need, kScratchBytes);
    void* ws;
    if (int rc = scratch_ptr(&ws)) return rc;
    // every kernel of the dispatch writes the scratch it reads (quantised
    // activations, scales, sums) before reading it: nothing needs clearing
    const hipError_t e = launch_path(w, x, m, y, ws, IQ_PATH_AUTO, nullptr, nullptr, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "matmul launch");
    return IQ_OK;
}

IQ_API size_t iq_matmul_noalloc_max_bytes(void) { return kScratchBytes; }

IQ_API int iq_matmul_reserve(iq_weight_t w, int64_t m, iq_stream_t stream) {
    if (int rc = check_weight(w)) return rc;
    if (m < 0) return fail(IQ_ERR_SHAPE, "negative input row count %lld", (long long)m);
    if (m == 0) return IQ_OK;
    // the widest of the entries that use the stream's workspace for W
    const size_t need = std::max(matmul_ws_bytes(w, m), m <= 65535 ? argmax_call_bytes(w, m) : 0);
    WsLease lease;
    return lease.acquire(need, (hipStream_t)stream);
}

IQ_API int iq_workspace_release(iq_stream_t stream) { return release_workspace((hipStream_t)stream); }

IQ_API size_t iq_matmul_workspace_size(iq_weight_t w, int64_t m) {
    if (!w || m <= 0) return 0;
    return matmul_ws_bytes(w, m);
}

IQ_API int iq_matmul_ws(iq_weight_t w, const float* x, int64_t m, float* y, void* workspace_ptr,
                        size_t workspace_bytes, iq_stream_t stream) {
    if (!workspace_ptr) return fail(IQ_ERR_INVALID, "null workspace");
    return matmul_impl(w, x, m, y, workspace_ptr, workspace_bytes, IQ_PATH_AUTO, nullptr, nullptr,
                       (hipStream_t)stream);
}

IQ_API int iq_matmul_host(iq_weight_t w, const float* x_host, int64_t m, float* y_host) {
    if (int rc = check_weight(w)) return rc;
    if (m <= 0) return m == 0 ? IQ_OK : fail(IQ_ERR_SHAPE, "negative input row count");
    if (!x_host || !y_host) return fail(IQ_ERR_INVALID, "null input or output pointer");
    const size_t xb = (size_t)(m * w->cols) * 4, yb = (size_t)(m * w->rows) * 4;
    const size_t xo = 0, yo = (xb + 255) & ~(size_t)255, ao = yo + ((yb + 255) & ~(size_t)255);
    const size_t need = ao + matmul_ws_bytes(w, m);
    WsLease lease;
    if (int rc = lease.acquire(need, nullptr)) return rc;
    uint8_t* base = (uint8_t*)lease.ptr();
    hipError_t e = hipMemcpy(base + xo, x_host, xb, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (input)");
    if (int rc = matmul_impl(w, (const float*)(base + xo), m, (float*)(base + yo), base + ao, need - ao, IQ_PATH_AUTO,
                             nullptr, nullptr, nullptr))
        return rc;
    e = hipMemcpy(y_host, base + yo, yb, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (output)");
    return IQ_OK;
}

static int quantize_entry(int dtype, const float* x, int64_t m, int64_t k, void* blocks_out, hipStream_t s) {
    if (!x || !blocks_out) return fail(IQ_ERR_INVALID, "null pointer");
    const int64_t be = dtype == kQ8_0 ? 32 : 256;
    if (m < 0 || k <= 0 || k % be)
        return fail(IQ_ERR_SHAPE, "quantize_row_%s: %lld is not divisible by %lld", dtype == kQ8_0 ? "q8_0" : "q8k",
                    (long long)k, (long long)be);
    if (m == 0) return IQ_OK;
    WsLease lease;
    if (int rc = lease.acquire(act_bytes(m, k), s)) return rc;
    ActView a = act_carve(lease.ptr(), m, k);
    hipError_t e = dtype == kQ8_0 ? launch_quant_q80(x, k, m, k, a, (uint8_t*)blocks_out, s)
                                  : launch_quant_q8k(x, k, m, k, a, (uint8_t*)blocks_out, s);
    if (e != hipSuccess) return hip_fail(e, "quantisation launch");
    return IQ_OK;
}

IQ_API int iq_quantize_q8k(const float* x, int64_t m, int64_t k, void* blocks_out, iq_stream_t stream) {
    return quantize_entry(kQ4_K, x, m, k, blocks_out, (hipStream_t)stream);
}

IQ_API int iq_quantize_q80(const float* x, int64_t m, int64_t k, void* blocks_out, iq_stream_t stream) {
    return quantize_entry(kQ8_0, x, m, k, blocks_out, (hipStream_t)stream);
}

IQ_API int iq_prefill_block_sums(iq_weight_t w, const float* x, int64_t m, float* y, int32_t* isum, int32_t* msum,
                                 iq_stream_t stream) {
    if (int rc = check_weight(w)) return rc;
    if (!x || !y || !isum || !msum) return fail(IQ_ERR_INVALID, "null input, output or integer buffer");
    if (!prefill_supported(view_of(w), m))
        return fail(IQ_ERR_SHAPE, "the int8-MFMA path covers Q4_K matrices at %lld or more input rows (got %s, %lld)",
                    (long long)kPrefillMinRows, dtype_name(w->dtype), (long long)m);
    WsLease lease;
    if (int rc = lease.acquire(prefill_workspace_size(view_of(w), m), (hipStream_t)stream)) return rc;
    hipError_t e = launch_prefill(view_of(w), x, w->cols, m, y, w->rows, lease.ptr(), isum, msum, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return IQ_OK;
}

IQ_API int iq_argmax_rows(const float* y, int64_t m, int64_t n, int32_t* idx, float* val, iq_stream_t stream) {
    if (m < 0 || n < 0) return fail(IQ_ERR_SHAPE, "negative logit shape [%lld, %lld]", (long long)m, (long long)n);
    if (m == 0) return IQ_OK;
    if (!y || !idx) return fail(IQ_ERR_INVALID, "null logits or index buffer");
    if (n == 0 || n > INT32_MAX || m > 65535)
        return fail(IQ_ERR_SHAPE, "argmax covers 1..%d logits per row and up to 65535 rows (got [%lld, %lld])",
                    INT32_MAX, (long long)m, (long long)n);
    hipStream_t s = (hipStream_t)stream;
    WsLease lease;
    if (int rc = lease.acquire(argmax_workspace_size(m, n), s)) return rc;
    hipError_t e = launch_argmax(y, m, n, n, idx, val, lease.ptr(), s);
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    return IQ_OK;
}

IQ_API int iq_matmul_argmax(iq_weight_t w, const float* x, int64_t m, int32_t* idx, float* val, iq_stream_t stream) {
    if (int rc = check_weight(w)) return rc;
    if (m < 0) return fail(IQ_ERR_SHAPE, "negative input row count %lld", (long long)m);
    if (m == 0) return IQ_OK;
    if (!x || !idx) return fail(IQ_ERR_INVALID, "null input or index buffer");
    if (m > 65535) return fail(IQ_ERR_SHAPE, "argmax covers up to 65535 rows (got %lld)", (long long)m);
    hipStream_t s = (hipStream_t)stream;
    const size_t yb = ((size_t)(m * w->rows) * 4 + 255) & ~(size_t)255;
    const size_t ab = (argmax_workspace_size(m, w->rows) + 255) & ~(size_t)255;
    WsLease lease;
    if (int rc = lease.acquire(argmax_call_bytes(w, m), s)) return rc;
    uint8_t* base = (uint8_t*)lease.ptr();
    float* y = (float*)base;
    if (const int f = argmax_fusion(w, m)) {
        // the product reduces its outputs as it writes them (per wave, or
        // per workgroup and row), and one small launch joins the pairs
        const int64_t parts = argmax_fused_parts(w, m);
        const size_t P = (size_t)(m * parts);
        const size_t kb = (P * 8 + 255) & ~(size_t)255, vb = (P * 4 + 255) & ~(size_t)255;
        uint64_t* keys = (uint64_t*)(base + yb);
        float* vals = (float*)(base + yb + kb);
        int nparts = (int)parts;
        hipError_t e = f == 1 ? launch_gemv_argmax(view_of(w), x, y, keys, vals, &nparts, s)
                              : launch_dense_argmax(view_of(w), x, m, y, base + yb + kb + vb, keys, vals, s);
        if (e != hipSuccess) return hip_fail(e, "matmul launch");
        e = launch_argmax_kv(keys, vals, m, nparts, idx, val, s);
        if (e != hipSuccess) return hip_fail(e, "argmax launch");
        return IQ_OK;
    }
    hipError_t e = launch_path(w, x, m, y, base + yb + ab, IQ_PATH_AUTO, nullptr, nullptr, s);
    if (e != hipSuccess) return hip_fail(e, "matmul launch");
    e = launch_argmax(y, m, w->rows, w->rows, idx, val, base + yb, s);
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    return IQ_OK;
}

IQ_API int iq_block_sums(iq_weight_t w, const float* x, int64_t m, float* y, int32_t* isum, int32_t* msum,
                         iq_stream_t stream) {
    if (!isum) return fail(IQ_ERR_INVALID, "null isum buffer");
    if (w && (w->dtype == kQ4_K || w->dtype == kQ5_K) && !msum)
        return fail(IQ_ERR_INVALID, "%s needs an msum buffer", dtype_name(w->dtype));
    return matmul_impl(w, x, m, y, nullptr, 0, IQ_PATH_LANES, isum, msum, (hipStream_t)stream);
}
