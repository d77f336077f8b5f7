// hai_gemm_mfma.hip -- batched-verify linear layer on the gfx950 matrix cores:
// Y[M, N] = X[M, K] . W[N, K]^T for M = (k+1) tokens x batch rows beyond the
// skinny kernel's 16 (the C4 / C5 batches: 32-64 rows), replacing
// rocblas_gemm_ex in HipBackend::gemm (hip_backend.cc:697-809) for that case.
//
// Tolerance mode: v_mfma_f32_16x16x32_bf16 sums each 32-product group with
// its own internal rounding, so results match the canonical fp32 order to
// ~1e-6 relative before the bf16 output rounding, not bit for bit.  The
// bit-exact path (hai_gemm_bf16) stays the one for M <= 16.
//
// Design (weight-streaming bound: 2M flop per weight pair of bytes, far below
// the MFMA ridge even at M = 128):
//   * A block owns 16 * NT consecutive weight rows; its KS waves split K by
//     512-element chunks (wave w takes chunks w, w + KS, ...), so every weight
//     byte is read once and narrow layers still get KS waves per row tile.
//   * Operands come straight from global memory in the MFMA register layout:
//     lane l supplies row (l % 16) and the 8 consecutive k of slab l / 16.
//     Any K order works if A and B use the same one; within a 512-element
//     chunk, slab g of step j is k = 32 j + 8 g, so the four lanes of a row
//     read 64 contiguous bytes per load instruction (16 rows x 64 B per
//     instruction; 16-byte non-temporal loads).
//   * The KS partial tiles meet in LDS and are summed in wave order (the
//     result does not depend on timing), then one epilogue writes bf16 with
//     the skinny GEMM's epilogues (store, residual add, SwiGLU over
//     interleaved gate/up rows).
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxMfmaRows = 128;

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

template <int MT, int NT, int KS, int JG, int EPI>
__global__ __launch_bounds__(64 * KS) void gemm_bf16_mfma_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                                 const uint16_t* __restrict__ x, int64_t ldx,
                                                                 const uint16_t* __restrict__ w, const uint16_t* res,
                                                                 int64_t ldres, int M, int N, int K) {
    __shared__ f32x4 part[KS][NT][MT][64];
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int64_t row_base = static_cast<int64_t>(blockIdx.x) * (16 * NT);

    // Byte offsets fit 32 bits: the caller bounds N*K*2 and M*ldx*2 below 4 GiB.
    // Rows past N or M start at or past the buffer end and read zeros.
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    uint32_t woff[NT], xoff[MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
        woff[t] = static_cast<uint32_t>(((row_base + 16 * t + li) * static_cast<int64_t>(K) + 8 * kg) * 2);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        xoff[mt] = static_cast<uint32_t>((static_cast<int64_t>(16 * mt + li) * ldx + 8 * kg) * 2);

    f32x4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nck = (K + 511) / 512;
    const int nfull = K / 512;
    for (int c = wave; c < nck; c += KS) {
        const bool full = c < nfull;
#pragma unroll
        for (int j0 = 0; j0 < 16; j0 += JG) {
            u32x4 bw[JG][NT], ax[JG][MT];
#pragma unroll
            for (int jj = 0; jj < JG; ++jj) {
                const int j = j0 + jj;
                const uint32_t koff = static_cast<uint32_t>(c) * 1024u + static_cast<uint32_t>(j) * 64u;
                // ragged chunk: this lane's 8 elements are all in range or all
                // out (K % 8 == 0)
                const bool ok = full || (c * 512 + 32 * j + 8 * kg < K);
                const ChunkOffset co(full, ok, koff);
#pragma unroll
                for (int t = 0; t < NT; ++t) bw[jj][t] = bload_w(rw, co.v(woff[t]), co.s);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) ax[jj][mt] = bload(rx, co.v(xoff[mt]), co.s);
            }
#pragma unroll
            for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma16(ax[jj][mt], bw[jj][t], acc[t][mt]);
        }
    }

#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) part[wave][t][mt][lane] = acc[t][mt];
    __syncthreads();

    // Tiles (t, mt) are finished by the waves in turn; partials summed in wave
    // order.  Lane l holds D rows 16 mt + 4 (l / 16) + i, column n = l % 16 of
    // tile t.
    for (int tile = wave; tile < NT * MT; tile += KS) {
        const int t = tile / MT;
        const int mt = tile - t * MT;
        f32x4 s = part[0][t][mt][lane];
#pragma unroll
        for (int q = 1; q < KS; ++q) {
            const f32x4 p = part[q][t][mt][lane];
            s = f32x4{s[0] + p[0], s[1] + p[1], s[2] + p[2], s[3] + p[3]};
        }
        const int64_t n = row_base + 16 * t + li;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * mt + 4 * kg + i;
            if (EPI == HAI_EPI_SILU_MUL) {
                // rows (2f, 2f+1) = (gate_f, up_f) sit in lanes (2p, 2p+1)
                const float g = bfr(s[i]);
                const float u = __shfl_xor(g, 1);
                if ((li & 1) == 0 && m < M && n + 1 < N) y[static_cast<int64_t>(m) * ldy + n / 2] = f2bf(csilu(g) * u);
            } else if (m < M && n < N) {
                float v = bfr(s[i]);
                if (EPI == HAI_EPI_RESIDUAL) v = bf2f(res[static_cast<int64_t>(m) * ldres + n]) + v;
                y[static_cast<int64_t>(m) * ldy + n] = f2bf(v);
            }
        }
    }
}

struct MfmaArgs {
    uint16_t* y;
    int64_t ldy;
    const uint16_t* x;
    int64_t ldx;
    const uint16_t* w;
    const uint16_t* res;
    int64_t ldres;
    int M, N, K;
};

template <int MT, int EPI>
void launch_mfma(const MfmaArgs& a, hipStream_t s) {
    constexpr int NT = 2, KS = 4, JG = 4;
    const int64_t blocks = (static_cast<int64_t>(a.N) + 16 * NT - 1) / (16 * NT);
    gemm_bf16_mfma_kernel<MT, NT, KS, JG, EPI><<<dim3(static_cast<unsigned>(blocks)), dim3(64 * KS), 0, s>>>(
        a.y, a.ldy, a.x, a.ldx, a.w, a.res, a.ldres, a.M, a.N, a.K);
}

template <int EPI>
void dispatch_mfma(const MfmaArgs& a, hipStream_t s) {
    if (a.M <= 16) launch_mfma<1, EPI>(a, s);
    else if (a.M <= 32) launch_mfma<2, EPI>(a, s);
    else if (a.M <= 64) launch_mfma<4, EPI>(a, s);
    else launch_mfma<8, EPI>(a, s);
}

}  // namespace

extern "C" int hai_gemm_bf16_mfma(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t M,
                                  int64_t N, int64_t K, int epilogue, const void* res, int64_t ld_res,
                                  void* stream) {
    if (y == nullptr || x == nullptr || w == nullptr) return invalid("gemm_mfma: null pointer");
    if (M < 0 || M > kMaxMfmaRows || N < 0 || K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldx < K)
        return invalid("gemm_mfma: shape (need 0<=M<=128, K%8==0, ldx%8==0, ldx>=K)");
    if (N > INT32_MAX || K > INT32_MAX) return invalid("gemm_mfma: dimension too large");
    if ((N + 32) * K * 2 >= (int64_t{1} << 32) || (kMaxMfmaRows + M) * ldx * 2 >= (int64_t{1} << 32))
        return invalid("gemm_mfma: W or X exceeds the 4 GiB buffer-offset range");
    if (!aligned16(x) || !aligned16(w)) return invalid("gemm_mfma: x and w must be 16-byte aligned");
    if (M == 0 || N == 0) return HAI_OK;
    const MfmaArgs a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx,
                     static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(res), ld_res,
                     int(M), int(N), int(K)};
    const hipStream_t s = as_stream(stream);
    switch (epilogue) {
        case HAI_EPI_STORE:
            if (ldy < N) return invalid("gemm_mfma: ldy < N");
            dispatch_mfma<HAI_EPI_STORE>(a, s);
            break;
        case HAI_EPI_RESIDUAL:
            if (res == nullptr || ldy < N || ld_res < N) return invalid("gemm_mfma: residual operands");
            dispatch_mfma<HAI_EPI_RESIDUAL>(a, s);
            break;
        case HAI_EPI_SILU_MUL:
            if (N % 2 != 0 || ldy < N / 2) return invalid("gemm_mfma: silu_mul needs even N and ldy >= N/2");
            dispatch_mfma<HAI_EPI_SILU_MUL>(a, s);
            break;
        default:
            return invalid("gemm_mfma: unknown epilogue");
    }
    return launched("gemm_bf16_mfma_kernel");
}
