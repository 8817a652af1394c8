// iq_api_internal.h -- handle types and helpers shared by the C-ABI sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "iq_internal.h"

struct iq_weight {
    int dtype = 0;
    int64_t rows = 0, cols = 0, row_bytes = 0;
    size_t nbytes = 0;
    uint8_t* dev = nullptr;
    bool owned = false;
    int device = 0;
};

namespace iq {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
const char* dtype_name(int dtype);
int64_t block_elems(int dtype);
int64_t block_bytes(int dtype);
bool dtype_ok(int dtype);
bool moe_dtype_ok(int dtype);  // expert formats of the MoE layer
// Library-owned device workspace of one (device, stream) pair.  A lease
// holds the library's workspace lock until it is destroyed, so a caller
// keeps it across every launch that uses the memory: another thread can
// neither grow (free) the buffer under those launches nor interleave its own
// launches on the same memory.  Workspaces of different streams are
// distinct, so calls on different streams never share memory.  Growing a
// workspace synchronises its stream (its earlier work may still read the old
// buffer) and is refused while the stream is being captured into a graph.
class WsLease {
  public:
    WsLease() = default;
    WsLease(const WsLease&) = delete;
    WsLease& operator=(const WsLease&) = delete;
    // Acquire at least `bytes` for `stream` on the current device.
    int acquire(size_t bytes, hipStream_t stream);
    void* ptr() const { return p_; }

  private:
    std::unique_lock<std::mutex> lock_;
    void* p_ = nullptr;
};
int check_weight(const iq_weight* w);
// y = x . W^T through the dispatch (or a fixed path), with the caller's
// workspace when ws is not null (ws_bytes >= matmul_ws_bytes(w, m)).
size_t matmul_ws_bytes(const iq_weight* w, int64_t m);
int matmul_impl(const iq_weight* w, const float* x, int64_t m, float* y, void* ws, size_t ws_bytes, int path,
                int32_t* isum, int32_t* msum, hipStream_t s);
WeightView view_of(const iq_weight* w);
// Shape and size checks of a GGUF matrix (QuantizedMatrix::new); row bytes out.
int check_matrix(int dtype, int64_t rows, int64_t cols, size_t nbytes, int64_t* row_bytes);
// A library-owned device matrix of that shape (256 zeroed bytes past the end).
int alloc_weight(int dtype, int64_t rows, int64_t cols, int64_t row_bytes, iq_weight** out);

}  // namespace iq
