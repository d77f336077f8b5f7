// hai_gemm.hip -- skinny BF16 linear layer for the verify step (M = k+1
// tokens x batch, M <= 16 per launch), replacing rocblas_gemm_ex in
// HipBackend::gemm (hip_backend.cc:697-809).
//
// Design (gfx950):
//   * The step is weight-streaming bound: every weight byte is read once, so
//     each wave owns RW consecutive weight rows and streams them with 16-byte
//     loads (8 bf16 per lane, 1 KB per wave instruction), U chunks in flight.
//   * Lane l owns the k-range {512c + 8l + j}; it accumulates with fma in
//     increasing k, and the 64 lane partials are reduced by the xor
//     butterfly.  This "L64 order" is the canonical order the CPU oracle
//     reproduces bit for bit; it does not depend on M, N, grid or tiling, so
//     a row's result is the same whether it is verified in a batch of 2 or
//     replayed alone.
//   * Arithmetic is IEEE fma on the VALU.  The gfx950 bf16 MFMA sums its
//     products with truncation below the group maximum, which no CPU can
//     reproduce, so it is not used on the bit-exact path.
//   * Epilogues fuse the residual add (h = bf16(h + bf16(acc))) and the
//     SwiGLU product for interleaved gate/up rows.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

template <int MB, int RW, int U, int EPI>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(
    uint16_t* __restrict__ y, int64_t ldy, const uint16_t* __restrict__ x, int64_t ldx,
    const uint16_t* __restrict__ w, const uint16_t* res, int64_t ldres, int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * RW;
    if (row0 >= N) return;
    const int nrows = static_cast<int>(min(static_cast<int64_t>(RW), static_cast<int64_t>(N) - row0));

    // Byte offsets fit 32 bits: the caller bounds N*K*2 and M*ldx*2 below 4 GiB.
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    uint32_t woff[RW], xoff[MB];
#pragma unroll
    for (int r = 0; r < RW; ++r)
        woff[r] = static_cast<uint32_t>(((row0 + r) * static_cast<int64_t>(K) + lane * 8) * 2);
#pragma unroll
    for (int m = 0; m < MB; ++m) xoff[m] = static_cast<uint32_t>((static_cast<int64_t>(m) * ldx + lane * 8) * 2);

    float acc[RW][MB];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[r][m] = 0.0f;

    auto body = [&](const u32x4 (&wv)[RW], const u32x4 (&xv)[MB]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float xa[MB], xb[MB];
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                xa[m] = lo_bf(xv[m][q]);
                xb[m] = hi_bf(xv[m][q]);
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const float wa = lo_bf(wv[r][q]);
                const float wb = hi_bf(wv[r][q]);
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    acc[r][m] = fma_(xa[m], wa, acc[r][m]);
                    acc[r][m] = fma_(xb[m], wb, acc[r][m]);
                }
            }
        }
    };

    // Groups of U chunks.  A chunk past K (ragged tail or group padding)
    // reads zeros through an out-of-range offset; fma(0, 0, acc) == acc
    // because acc is never -0 (it starts at +0 and round-to-nearest only
    // produces -0 from (-0) + (-0)), so padding does not change a bit.
    const int nck = (K + 511) / 512;
    const int nfull = K / 512;
    for (int c0 = 0; c0 < nck; c0 += U) {
        u32x4 wv[U][RW];
        u32x4 xv[U][MB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u;
            // full chunk: every lane valid; ragged chunk: lanes past K masked
            const bool ok = c < nfull || (c < nck && c * 512 + lane * 8 < K);
            const uint32_t so = ok ? static_cast<uint32_t>(c) * 1024u : 0u;
#pragma unroll
            for (int r = 0; r < RW; ++r) wv[u][r] = bload(rw, ok ? woff[r] : kOutOfRange, so);
#pragma unroll
            for (int m = 0; m < MB; ++m) xv[u][m] = bload(rx, ok ? xoff[m] : kOutOfRange, so);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) body(wv[u], xv[u]);
    }

#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[r][m] = wave_sum64(acc[r][m]);

    if (EPI == HAI_EPI_SILU_MUL) {
        // rows (2p, 2p+1) = (gate_f, up_f), output column f = row0/2 + p.
#pragma unroll
        for (int p = 0; p < RW / 2; ++p)
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                if (lane == p * MB + m && m < M && 2 * p + 1 < nrows) {
                    const float g = bfr(acc[2 * p][m]);
                    const float u = bfr(acc[2 * p + 1][m]);
                    y[static_cast<int64_t>(m) * ldy + row0 / 2 + p] = f2bf(csilu(g) * u);
                }
            }
    } else {
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                if (lane == r * MB + m && m < M && r < nrows) {
                    const int64_t n = row0 + r;
                    float v = bfr(acc[r][m]);
                    if (EPI == HAI_EPI_RESIDUAL) v = bf2f(res[static_cast<int64_t>(m) * ldres + n]) + v;
                    y[static_cast<int64_t>(m) * ldy + n] = f2bf(v);
                }
            }
    }
}

template <int MB, int RW, int EPI>
void launch_gemm(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 const uint16_t* res, int64_t ldres, int M, int N, int K, hipStream_t s) {
    constexpr int U = MB <= 2 ? 4 : (MB <= 8 ? 2 : 1);
    const int64_t waves = (static_cast<int64_t>(N) + RW - 1) / RW;
    const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
    gemm_bf16_kernel<MB, RW, U, EPI><<<dim3(blocks), dim3(256), 0, s>>>(y, ldy, x, ldx, w, res, ldres, M,
                                                                        N, K);
}

template <int MB, int EPI>
void dispatch_rw(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 const uint16_t* res, int64_t ldres, int M, int N, int K, hipStream_t s) {
    // Two rows per wave keeps the register footprint small enough for eight
    // waves per SIMD, which is what keeps enough bytes in flight on gfx950
    // (measured faster than 4 rows per wave or software-pipelined variants).
    launch_gemm<MB, 2, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
}

template <int EPI>
void dispatch_mb(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 const uint16_t* res, int64_t ldres, int M, int N, int K, hipStream_t s) {
    if (M <= 1) dispatch_rw<1, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
    else if (M <= 2) dispatch_rw<2, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
    else if (M <= 4) dispatch_rw<4, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
    else if (M <= 8) dispatch_rw<8, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
    else dispatch_rw<16, EPI>(y, ldy, x, ldx, w, res, ldres, M, N, K, s);
}

}  // namespace

extern "C" int hai_gemm_bf16(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t M,
                             int64_t N, int64_t K, int epilogue, const void* res, int64_t ld_res,
                             void* stream) {
    if (y == nullptr || x == nullptr || w == nullptr) return invalid("gemm: null pointer");
    if (M < 0 || M > 16 || N < 0 || K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldx < K)
        return invalid("gemm: shape (need 0<=M<=16, K%8==0, ldx%8==0, ldx>=K)");
    if (N > INT32_MAX || K > INT32_MAX) return invalid("gemm: dimension too large");
    if ((N + 4) * K * 2 >= (int64_t{1} << 32) || M * ldx * 2 >= (int64_t{1} << 32))
        return invalid("gemm: W or X exceeds the 4 GiB buffer-offset range");
    if (!aligned16(x) || !aligned16(w)) return invalid("gemm: x and w must be 16-byte aligned");
    if (M == 0 || N == 0) return HAI_OK;
    const auto* xs = static_cast<const uint16_t*>(x);
    const auto* ws = static_cast<const uint16_t*>(w);
    auto* ys = static_cast<uint16_t*>(y);
    const auto* rs = static_cast<const uint16_t*>(res);
    const hipStream_t s = as_stream(stream);
    switch (epilogue) {
        case HAI_EPI_STORE:
            if (ldy < N) return invalid("gemm: ldy < N");
            dispatch_mb<HAI_EPI_STORE>(ys, ldy, xs, ldx, ws, nullptr, 0, int(M), int(N), int(K), s);
            break;
        case HAI_EPI_RESIDUAL:
            if (res == nullptr || ldy < N || ld_res < N) return invalid("gemm: residual operands");
            dispatch_mb<HAI_EPI_RESIDUAL>(ys, ldy, xs, ldx, ws, rs, ld_res, int(M), int(N), int(K), s);
            break;
        case HAI_EPI_SILU_MUL:
            if (N % 2 != 0 || ldy < N / 2) return invalid("gemm: silu_mul needs even N and ldy >= N/2");
            dispatch_mb<HAI_EPI_SILU_MUL>(ys, ldy, xs, ldx, ws, nullptr, 0, int(M), int(N), int(K), s);
            break;
        default:
            return invalid("gemm: unknown epilogue");
    }
    return launched("gemm_bf16_kernel");
}
