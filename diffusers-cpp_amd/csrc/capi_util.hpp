// capi_util.hpp -- status codes, thread-local error text and launch checks
// shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dit_hip.h"

namespace dit {

// Records a formatted message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; DT_OK or DT_ERR_HIP.
int check_launch(const char* what);

// Multiprocessor (CU) count of the current device, cached per device.
int cu_count();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int elem_size(int32_t type) {
    switch (type) {
        case DT_TYPE_F32: return 4;
        case DT_TYPE_I32: return 4;
        case DT_TYPE_F16: return 2;
        case DT_TYPE_BF16: return 2;
        default: return 0;
    }
}

inline bool is_io_type(int32_t t) { return t == DT_TYPE_F32 || t == DT_TYPE_BF16; }

}  // namespace dit

#define DT_REQUIRE(cond, ...)                                         \
    do {                                                              \
        if (!(cond)) return ::dit::fail(DT_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)
