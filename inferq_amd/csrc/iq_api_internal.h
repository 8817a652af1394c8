// iq_api_internal.h -- handle types and helpers shared by the C-ABI sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
int workspace(size_t bytes, void** out);
int check_weight(const iq_weight* w);
WeightView view_of(const iq_weight* w);

}  // namespace iq
