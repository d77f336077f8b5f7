// hai_common.h -- host-side helpers shared by the kernel translation units
// (argument checks, error text, launch status).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/hai_kernels.h"

namespace hai {

void set_error(const std::string& message);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int invalid(const char* what) {
    set_error(std::string("invalid argument: ") + what);
    return HAI_ERR_INVALID_ARGUMENT;
}

inline int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return HAI_OK;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return HAI_ERR_BACKEND;
}

inline int launched(const char* what) { return check_hip(hipGetLastError(), what); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace hai
