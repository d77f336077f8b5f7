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

// Opt-in host-side operand check (environment HAI_CHECK_BOUNDS=1, read once
// per process; the tests set it).  The kernels size their buffer
// descriptors and strides from the shapes they are given, not from the
// allocations, so an operand smaller than its shape implies would be read
// or written past its end on the GPU.  With the check on, every launcher
// that calls check_extent verifies before launching that [p, p + bytes)
// lies inside one device allocation (hipMemGetAddressRange) and returns
// HAI_ERR_INVALID_ARGUMENT otherwise.  Off, it costs one branch.
bool bounds_checking();
int check_extent(const void* p, size_t bytes, const char* what);

// Bytes spanned by `rows` rows of `cols` elements at row pitch `ld`.
inline size_t rows_extent(int64_t rows, int64_t cols, int64_t ld, size_t elem) {
    return rows <= 0 || cols <= 0 ? 0 : static_cast<size_t>((rows - 1) * ld + cols) * elem;
}

// The operands of a linear layer Y[M, N] = X[M, K] . W[N, K]^T (w_elem bytes
// per weight) with the given epilogue (SwiGLU writes N / 2 columns, the
// residual epilogue reads res[M, N]); HAI_OK when unchecked.
inline int check_gemm_extents(const void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, size_t w_elem,
                              int64_t M, int64_t N, int64_t K, int epilogue, const void* res, int64_t ldres) {
    if (!bounds_checking()) return HAI_OK;
    const int epi = epilogue & 0xff;
    int rc = check_extent(x, rows_extent(M, K, ldx, 2), "gemm x");
    if (rc == HAI_OK) rc = check_extent(w, static_cast<size_t>(N) * static_cast<size_t>(K) * w_elem, "gemm w");
    if (rc == HAI_OK)
        rc = check_extent(y, rows_extent(M, epi == HAI_EPI_SILU_MUL ? N / 2 : N, ldy, 2), "gemm y");
    if (rc == HAI_OK && epi == HAI_EPI_RESIDUAL) rc = check_extent(res, rows_extent(M, N, ldres, 2), "gemm res");
    return rc;
}

}  // namespace hai
