// hai_gemm_blaslt.hip -- prompt-chunk linear layers through hipBLASLt: the
// plain GEMM Y[M, N] = X[M, K] . W[N, K]^T (bf16 in, fp32 accumulate) of the
// fast prefill, with the prefill's epilogues (store, residual add, SwiGLU of
// interleaved gate / up rows), replacing rocblas_gemm_ex in HipBackend::gemm
// (hip_backend.cc:697-809) for prompt-sized row counts.
//
// These are plain library GEMMs: at 1024-4096 rows the layer is compute
// bound, and hipBLASLt's tuned gfx950 kernels run 1.07-1.41 PFLOP/s on the
// 27B prefill shapes against 0.53-0.83 for the hand-written tiled kernel
// (measured on MI355X).  The decode path (verify rows, corrections, drafts)
// does not come here.
//   * row-major Y = X W^T is column-major Y^T = W X^T: A = W (K x N,
//     transposed), B = X (K x M), D = Y (N x M, leading dimension ldy);
//   * the residual epilogue is beta = 1 with C = the residual rows;
//   * SwiGLU: the GEMM writes the interleaved (gate_f, up_f) columns to a
//     scratch in the caller's workspace, and swiglu_pairs_kernel forms
//     y = bf16(silu(g) * u) with the rounding points of the other GEMMs'
//     SwiGLU epilogue;
//   * one hipBLASLt handle per device and one heuristic choice per shape,
//     cached; the algorithm's workspace comes from the caller.
// Tolerance mode, as the other matrix-core GEMMs.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr size_t kAlgoWorkspace = size_t{64} << 20;  // bytes offered to the algorithm
constexpr int kMaxDevices = 64;

// y[m][f] = bf16(silu(bf16 g) * bf16 u) for the interleaved pairs (g, u) =
// (p[m][2f], p[m][2f + 1]) of the bf16 product; 8 outputs per thread.
__global__ __launch_bounds__(256) void swiglu_pairs_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                           const uint16_t* __restrict__ p, int64_t ldp, int64_t M,
                                                           int64_t F) {
    const int64_t groups = (F + 7) / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= M * groups) return;
    const int64_t m = i / groups;
    const int64_t f0 = (i - m * groups) * 8;
    const uint16_t* pr = p + m * ldp + 2 * f0;
    uint16_t* yr = y + m * ldy + f0;
    if (f0 + 8 <= F) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(pr);
        const u32x4 b = *reinterpret_cast<const u32x4*>(pr + 8);
        const uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            o[q] = f2bf2(csilu(lo_bf(w[2 * q])) * hi_bf(w[2 * q]),
                         csilu(lo_bf(w[2 * q + 1])) * hi_bf(w[2 * q + 1]));
        }
        if ((reinterpret_cast<uintptr_t>(yr) & 15u) == 0) {
            *reinterpret_cast<u32x4*>(yr) = u32x4{o[0], o[1], o[2], o[3]};
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                yr[2 * q] = static_cast<uint16_t>(o[q]);
                yr[2 * q + 1] = static_cast<uint16_t>(o[q] >> 16);
            }
        }
    } else {
        for (int64_t f = f0; f < F; ++f) y[m * ldy + f] = f2bf(csilu(bf2f(p[m * ldp + 2 * f])) * bf2f(p[m * ldp + 2 * f + 1]));
    }
}

struct Device {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t, int>, hipblasLtMatmulAlgo_t> algos;
};
Device g_dev[kMaxDevices];
std::mutex g_mu;

int status(hipblasStatus_t s, const char* what) {
    if (s == HIPBLAS_STATUS_SUCCESS) return HAI_OK;
    set_error(std::string(what) + ": hipBLASLt status " + std::to_string(static_cast<int>(s)));
    return HAI_ERR_BACKEND;
}

// Descriptors of one call; destroyed with the object.
struct Call {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr, ld = nullptr;
    ~Call() {
        if (la) hipblasLtMatrixLayoutDestroy(la);
        if (lb) hipblasLtMatrixLayoutDestroy(lb);
        if (lc) hipblasLtMatrixLayoutDestroy(lc);
        if (ld) hipblasLtMatrixLayoutDestroy(ld);
        if (op) hipblasLtMatmulDescDestroy(op);
    }
    int make(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldc, int64_t ldd) {
        int rc = status(hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul desc");
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        if (rc == HAI_OK)
            rc = status(hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)), "transa");
        if (rc == HAI_OK)
            rc = status(hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)), "transb");
        if (rc == HAI_OK) rc = status(hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, K, N, K), "layout A");
        if (rc == HAI_OK) rc = status(hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, K, M, ldx), "layout B");
        if (rc == HAI_OK) rc = status(hipblasLtMatrixLayoutCreate(&lc, HIP_R_16BF, N, M, ldc), "layout C");
        if (rc == HAI_OK) rc = status(hipblasLtMatrixLayoutCreate(&ld, HIP_R_16BF, N, M, ldd), "layout D");
        return rc;
    }
};

// Creates the device's handle (hipBLASLt loads its kernel libraries here:
// seconds, once per process and device).  Called with g_mu held.
int ensure_handle(Device& D) {
    if (D.handle != nullptr) return HAI_OK;
    return status(hipblasLtCreate(&D.handle), "hipblasLtCreate");
}

size_t scratch_bytes(int64_t M, int64_t N, int epi) {
    return epi == HAI_EPI_SILU_MUL ? static_cast<size_t>(M * N) * 2 : 0;
}

}  // namespace

extern "C" int hai_gemm_bf16_blaslt_prepare(void* workspace, size_t workspace_bytes, void* stream) {
    // a 64 x 64 x 64 GEMM inside the workspace: its operands and output take
    // the first 24 KB, its algorithm workspace the rest of the algorithm part;
    // the values are whatever the workspace holds and the output is discarded
    if (workspace == nullptr || workspace_bytes < kAlgoWorkspace || !aligned16(workspace))
        return invalid("gemm_bf16_blaslt_prepare: workspace below the algorithm workspace");
    {
        const int rc = check_extent(workspace, workspace_bytes, "gemm_bf16_blaslt_prepare workspace");
        if (rc != HAI_OK) return rc;
    }
    char* base = static_cast<char*>(workspace);
    constexpr int64_t n = 64;
    constexpr size_t kOperands = size_t{1} << 20;  // operands of the tiny GEMM, then its algorithm workspace
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != HAI_OK) return rc;
    if (dev < 0 || dev >= kMaxDevices) return invalid("gemm_bf16_blaslt: device ordinal above 63");
    std::lock_guard<std::mutex> lock(g_mu);
    Device& D = g_dev[dev];
    rc = ensure_handle(D);
    if (rc != HAI_OK) return rc;
    Call call;
    rc = call.make(n, n, n, n, n, n);
    hipblasLtMatmulPreference_t pref = nullptr;
    if (rc == HAI_OK) rc = status(hipblasLtMatmulPreferenceCreate(&pref), "preference");
    const uint64_t wsz = kAlgoWorkspace - kOperands;
    if (rc == HAI_OK)
        rc = status(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                          sizeof(wsz)),
                    "preference workspace");
    hipblasLtMatmulHeuristicResult_t res1[1];
    int found = 0;
    if (rc == HAI_OK)
        rc = status(hipblasLtMatmulAlgoGetHeuristic(D.handle, call.op, call.la, call.lb, call.lc, call.ld, pref, 1, res1,
                                                    &found),
                    "heuristic");
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (rc != HAI_OK) return rc;
    if (found < 1) return HAI_OK;  // nothing to load ahead; the first real call loads it
    const float alpha = 1.0f, beta = 0.0f;
    const void* w = base;
    const void* x = base + 8192;
    void* y = base + 16384;
    return status(hipblasLtMatmul(D.handle, call.op, &alpha, w, call.la, x, call.lb, &beta, y, call.lc, y, call.ld,
                                  &res1[0].algo, base + kOperands, wsz, as_stream(stream)),
                  "hipblasLtMatmul (prepare)");
}

extern "C" size_t hai_gemm_bf16_blaslt_workspace_bytes(int64_t M, int64_t N, int epilogue) {
    if (M <= 0 || N <= 0) return 0;
    return kAlgoWorkspace + ((scratch_bytes(M, N, epilogue & 0xff) + 255) & ~size_t{255});
}

extern "C" int hai_gemm_bf16_blaslt(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t M,
                                    int64_t N, int64_t K, int epilogue, const void* res, int64_t ld_res,
                                    void* workspace, size_t workspace_bytes, void* stream) {
    if (y == nullptr || x == nullptr || w == nullptr || workspace == nullptr)
        return invalid("gemm_bf16_blaslt: null pointer");
    if (M < 0 || N <= 0 || K <= 0 || ldx < K || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
        return invalid("gemm_bf16_blaslt: shape");
    const int epi = epilogue & 0xff;
    if (epi != HAI_EPI_STORE && epi != HAI_EPI_RESIDUAL && epi != HAI_EPI_SILU_MUL)
        return invalid("gemm_bf16_blaslt: unknown epilogue");
    if (epi == HAI_EPI_SILU_MUL ? (N % 2 != 0 || ldy < N / 2) : ldy < N) return invalid("gemm_bf16_blaslt: ldy");
    if (epi == HAI_EPI_RESIDUAL && (res == nullptr || ld_res < N)) return invalid("gemm_bf16_blaslt: residual");
    if (workspace_bytes < hai_gemm_bf16_blaslt_workspace_bytes(M, N, epi))
        return invalid("gemm_bf16_blaslt: workspace below hai_gemm_bf16_blaslt_workspace_bytes");
    if (!aligned16(workspace)) return invalid("gemm_bf16_blaslt: workspace alignment");
    {
        int rc = check_gemm_extents(y, ldy, x, ldx, w, 2, M, N, K, epilogue, res, ld_res);
        if (rc == HAI_OK) rc = check_extent(workspace, workspace_bytes, "gemm_bf16_blaslt workspace");
        if (rc != HAI_OK) return rc;
    }
    if (M == 0) return HAI_OK;
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != HAI_OK) return rc;
    if (dev < 0 || dev >= kMaxDevices) return invalid("gemm_bf16_blaslt: device ordinal above 63");

    char* scratch = static_cast<char*>(workspace) + kAlgoWorkspace;
    uint16_t* d = epi == HAI_EPI_SILU_MUL ? reinterpret_cast<uint16_t*>(scratch) : static_cast<uint16_t*>(y);
    const int64_t ldd = epi == HAI_EPI_SILU_MUL ? N : ldy;
    const void* c = epi == HAI_EPI_RESIDUAL ? res : static_cast<const void*>(d);
    const int64_t ldc = epi == HAI_EPI_RESIDUAL ? ld_res : ldd;
    const float alpha = 1.0f, beta = epi == HAI_EPI_RESIDUAL ? 1.0f : 0.0f;

    Call call;
    rc = call.make(M, N, K, ldx, ldc, ldd);
    if (rc != HAI_OK) return rc;
    hipblasLtMatmulAlgo_t algo;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        Device& D = g_dev[dev];
        rc = ensure_handle(D);
        if (rc != HAI_OK) return rc;
        const auto key = std::make_tuple(M, N, K, ldx, ldd * (int64_t{1} << 32) + ldc, epi);
        auto it = D.algos.find(key);
        if (it == D.algos.end()) {
            hipblasLtMatmulPreference_t pref = nullptr;
            rc = status(hipblasLtMatmulPreferenceCreate(&pref), "preference");
            const uint64_t wsz = kAlgoWorkspace;
            if (rc == HAI_OK)
                rc = status(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                                  sizeof(wsz)),
                            "preference workspace");
            hipblasLtMatmulHeuristicResult_t res1[1];
            int n = 0;
            if (rc == HAI_OK)
                rc = status(hipblasLtMatmulAlgoGetHeuristic(D.handle, call.op, call.la, call.lb, call.lc, call.ld, pref, 1,
                                                            res1, &n),
                            "heuristic");
            if (pref) hipblasLtMatmulPreferenceDestroy(pref);
            if (rc != HAI_OK) return rc;
            if (n < 1 || res1[0].workspaceSize > kAlgoWorkspace) {
                set_error("gemm_bf16_blaslt: no hipBLASLt algorithm for this shape");
                return HAI_ERR_NOT_IMPLEMENTED;
            }
            it = D.algos.emplace(key, res1[0].algo).first;
        }
        algo = it->second;
        rc = status(hipblasLtMatmul(D.handle, call.op, &alpha, w, call.la, x, call.lb, &beta, c, call.lc, d, call.ld,
                                    &algo, workspace, kAlgoWorkspace, as_stream(stream)),
                    "hipblasLtMatmul");
    }
    if (rc != HAI_OK) return rc;
    if (epi != HAI_EPI_SILU_MUL) return HAI_OK;
    const int64_t F = N / 2;
    const int64_t threads = M * ((F + 7) / 8);
    swiglu_pairs_kernel<<<dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(y), ldy, d, N, M, F);
    return launched("swiglu_pairs_kernel");
}
