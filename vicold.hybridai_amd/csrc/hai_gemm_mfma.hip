// hai_gemm_mfma.hip -- batched-verify linear layer on the gfx950 matrix cores:
// Y[M, N] = X[M, K] . W[N, K]^T for M <= 128 rows of (k+1) tokens x batch
// (the C4 / C5 batches, their drafts and corrections, batched prompt chunks),
// replacing rocblas_gemm_ex in HipBackend::gemm (hip_backend.cc:697-809) for
// that case.
//
// Tolerance mode: v_mfma_f32_16x16x32_bf16 sums each 32-product group with
// its own internal rounding, so results match the canonical fp32 order to
// ~1e-6 relative before the bf16 output rounding, not bit for bit.  The
// bit-exact path (hai_gemm_bf16) stays the one for M <= 16.
//
// Design (weight-streaming bound: 2M flop per pair of weight bytes, far
// below the MFMA ridge even at M = 128):
//   * A block (4 waves) owns 64 consecutive weight rows, 16 per wave, and
//     walks K in 256-element chunks.  Every wave streams its rows with
//     row-contiguous 16-byte loads (two rows per instruction, non-temporal)
//     into its own LDS tile; the chunk's activation rows [M x 256] are loaded
//     once per block, coalesced, into a shared LDS tile.  The next chunk's
//     loads are in flight (registers) while the current one is multiplied.
//   * MFMA operands are read from LDS in the register layout of the 16x16x32
//     instruction: lane l takes row l % 16 and k-slab 8 (l / 16) + 32 j.
//     Rows are padded by 16 bytes, so those reads are bank-conflict free.
//   * Narrow layers (N <= 20480) also split K across 2 or 4 blocks when the
//     caller passes a workspace: the blocks write fp32 partials and a second
//     pass sums them in split order (deterministic) and applies the epilogue.
//     (Folding that pass into the last block of each tile needs a device-scope
//     release per block, an L2 write-back that serialises within an XCD:
//     measured 1.8x slower than the second launch on MI355X.)
//   * Epilogues as in the skinny GEMM: store, residual add, SwiGLU over
//     interleaved (gate_f, up_f) rows.
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "hai_common.h"
#include "hai_device.h"
#include "hai_gemm_common.h"

namespace {

using namespace hai;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxMfmaRows = 128;
constexpr int kChunk = 256;           // k elements per chunk
constexpr int kLdsRow = kChunk + 8;   // padded LDS row, bf16 elements
constexpr int kBlockRows = 64;        // weight rows per block

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
// 32 x 32 x 16: lane l holds A row l % 32 (B column l % 32), k 8 (l / 32) .. +7;
// result element r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4, column
// l % 32.  On MI355X this form issues at 2.1-2.2 PFLOP/s against 0.8-1.3
// for the 16 x 16 x 32 one (register-operand probe, 1-4 blocks per CU).
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Epilogue of one output element pair held by lane (li, kg): value v of row m,
// column n (SwiGLU pairs columns n, n ^ 1 across lanes li, li ^ 1).
template <int EPI>
__device__ __forceinline__ void mfma_store(uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldres, float v,
                                           int m, int64_t n, int M, int N, int li) {
    if (EPI == HAI_EPI_SILU_MUL) {
        const float g = bfr(v);
        const float u = __shfl_xor(g, 1);
        if ((li & 1) == 0 && m < M && n + 1 < N) y[static_cast<int64_t>(m) * ldy + n / 2] = f2bf(csilu(g) * u);
    } else if (m < M && n < N) {
        float o = bfr(v);
        if (EPI == HAI_EPI_RESIDUAL) o = bf2f(res[static_cast<int64_t>(m) * ldres + n]) + o;
        y[static_cast<int64_t>(m) * ldy + n] = f2bf(o);
    }
}

// Stream-K split (sk > 0 blocks): the ntiles x nck (tile, chunk) items are
// cut into sk equal contiguous ranges, block b taking [b I / sk, (b+1) I /
// sk).  Used when the tiles exceed one round of resident blocks, so a block
// takes more than one tile's chunks and a tile spans at most two blocks: the
// block holding its first chunk writes partial plane 0, the other plane 1.
// Tiles inside one block are finished in place.
__host__ __device__ inline int64_t sk_block_of(int64_t item, int64_t items, int64_t sk) {
    return ((item + 1) * sk - 1) / items;
}

// grid (ceil(N / 64), KSB); with KSB > 1 the blocks of split s take chunks
// s, s + KSB, ... and write fp32 partials part[s][m][n].
template <int MT, int EPI, bool SK>
__global__ __launch_bounds__(256) void gemm_bf16_mfma_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                             const uint16_t* __restrict__ x, int64_t ldx,
                                                             const uint16_t* __restrict__ w, const uint16_t* res,
                                                             int64_t ldres, int M, int N, int K,
                                                             float* __restrict__ part, int KSB, int sk) {
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* xs = lds;                          // [16 MT][kLdsRow] activation rows
    uint16_t* ws = lds + 16 * MT * kLdsRow;      // [4 waves][16][kLdsRow] weight rows
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int nck = (K + kChunk - 1) / kChunk;
    const int nfull = K / kChunk;
    // one tile (64 weight rows) over chunks cbeg, cbeg + cstep, ... < cend;
    // plane < 0: finish y, else write partial plane `plane`
    auto piece = [&](int64_t tile, int cbeg, int cend, int cstep, int plane) {
    const int64_t row_base = tile * kBlockRows + wave * 16;

    // Byte offsets fit 32 bits: the caller bounds N*K*2 and M*ldx*2 below 4
    // GiB.  Rows past N or M start at or past the buffer end and read zeros.
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    // weight loads: instruction i covers rows 2i and 2i+1 (lanes 0-31 / 32-63)
    const int w_half = lane >> 5;
    const int w_col = (lane & 31) * 8;
    const uint32_t woff0 = static_cast<uint32_t>(((row_base + w_half) * static_cast<int64_t>(K) + w_col) * 2);
    const uint32_t two_rows = static_cast<uint32_t>(K) * 4u;
    // activation loads: 16 MT rows x 256 elements, 32 lanes per row
    constexpr int XL = 2 * MT;
    uint32_t xoff[XL];
    int xrow[XL], xcol[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int e = tid + 256 * i;
        xrow[i] = e >> 5;
        xcol[i] = (e & 31) * 8;
        xoff[i] = static_cast<uint32_t>((static_cast<int64_t>(xrow[i]) * ldx + xcol[i]) * 2);
    }

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 wv[8], xv[XL];
    auto load = [&](int c) {
        const uint32_t off = static_cast<uint32_t>(c) * (kChunk * 2);
        if (c < nfull) {
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] = bload_w(rw, woff0 + i * two_rows, off);
#pragma unroll
            for (int i = 0; i < XL; ++i) xv[i] = bload(rx, xoff[i], off);
        } else {
            // ragged chunk: a lane's 8 elements are all in K or all past it
            const bool okw = c * kChunk + w_col < K;
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] = bload_w(rw, okw ? woff0 + i * two_rows + off : kOutOfRange, 0u);
#pragma unroll
            for (int i = 0; i < XL; ++i) xv[i] = bload(rx, c * kChunk + xcol[i] < K ? xoff[i] + off : kOutOfRange, 0u);
        }
    };
    int c = cbeg;
    if (c < cend) load(c);
    for (; c < cend; c += cstep) {
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4*>(&ws[(wave * 16 + 2 * i + w_half) * kLdsRow + w_col]) = wv[i];
#pragma unroll
        for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(&xs[xrow[i] * kLdsRow + xcol[i]]) = xv[i];
        __syncthreads();
        if (c + cstep < cend) load(c + cstep);
#pragma unroll
        for (int j = 0; j < kChunk / 32; ++j) {
            const u32x4 b = *reinterpret_cast<const u32x4*>(&ws[(wave * 16 + li) * kLdsRow + 32 * j + 8 * kg]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(&xs[(16 * mt + li) * kLdsRow + 32 * j + 8 * kg]);
                acc[mt] = mfma16(a, b, acc[mt]);
            }
        }
    }

    // D layout: lane (li, kg) holds rows 16 mt + 4 kg + i of column row_base + li
    const int64_t n = row_base + li;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * mt + 4 * kg + i;
            if (plane < 0)
                mfma_store<EPI>(y, ldy, res, ldres, acc[mt][i], m, n, M, N, li);
            else if (m < M && n < N)
                part[(static_cast<int64_t>(plane) * M + m) * N + n] = acc[mt][i];
        }
    };
    if constexpr (!SK) {
        piece(blockIdx.x, blockIdx.y, nck, KSB, KSB == 1 ? -1 : static_cast<int>(blockIdx.y));
        return;
    }
    const int64_t ntiles = (N + kBlockRows - 1) / kBlockRows;
    const int64_t items = ntiles * nck;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * items / sk;
    const int64_t hi = (static_cast<int64_t>(blockIdx.x) + 1) * items / sk;
    for (int64_t it = lo; it < hi;) {
        const int64_t tile = it / nck;
        const int c0 = static_cast<int>(it - tile * nck);
        const int c1 = static_cast<int>(min(hi - tile * nck, static_cast<int64_t>(nck)));
        const int plane = (c0 == 0 && c1 == nck) ? -1 : (sk_block_of(tile * nck, items, sk) == blockIdx.x ? 0 : 1);
        piece(tile, c0, c1, 1, plane);  // (a piece's first chunk waits for the LDS reads of the last one)
        it = tile * nck + c1;
    }
}

// Sums the KSB partials of every element in split order and applies the
// epilogue; one thread per output column pair (n even, n + 1).
template <int EPI>
__global__ void mfma_finalize_kernel(uint16_t* __restrict__ y, int64_t ldy, const float* __restrict__ part, int KSB,
                                     const uint16_t* res, int64_t ldres, int M, int N) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t np = (static_cast<int64_t>(N) + 1) / 2;
    if (i >= static_cast<int64_t>(M) * np) return;
    const int m = static_cast<int>(i / np);
    const int64_t n = (i - m * np) * 2;
    float v[2] = {0.0f, 0.0f};
    for (int e = 0; e < 2; ++e) {
        if (n + e >= N) continue;
        const int64_t at = static_cast<int64_t>(m) * N + n + e;
        float s = part[at];
        for (int q = 1; q < KSB; ++q) s = s + part[static_cast<int64_t>(q) * M * N + at];
        v[e] = s;
    }
    if (EPI == HAI_EPI_SILU_MUL) {
        if (n + 1 < N) y[static_cast<int64_t>(m) * ldy + n / 2] = f2bf(csilu(bfr(v[0])) * bfr(v[1]));
        return;
    }
    for (int e = 0; e < 2; ++e) {
        if (n + e >= N) continue;
        float o = bfr(v[e]);
        if (EPI == HAI_EPI_RESIDUAL) o = bf2f(res[static_cast<int64_t>(m) * ldres + n + e]) + o;
        y[static_cast<int64_t>(m) * ldy + n + e] = f2bf(o);
    }
}

// Stream-K finalize: the tiles that two blocks share get plane 0 + plane 1
// (the order of the K-split pass) and the epilogue; the others were finished
// by their block.
template <int EPI>
__global__ void mfma_sk_finalize_kernel(uint16_t* __restrict__ y, int64_t ldy, const float* __restrict__ part,
                                        const uint16_t* res, int64_t ldres, int M, int N, int nck, int sk) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t np = (static_cast<int64_t>(N) + 1) / 2;
    if (i >= static_cast<int64_t>(M) * np) return;
    const int m = static_cast<int>(i / np);
    const int64_t n = (i - m * np) * 2;
    const int64_t tile = n / kBlockRows;
    const int64_t items = ((static_cast<int64_t>(N) + kBlockRows - 1) / kBlockRows) * nck;
    if (sk_block_of(tile * nck, items, sk) == sk_block_of(tile * nck + nck - 1, items, sk)) return;
    float v[2] = {0.0f, 0.0f};
    for (int e = 0; e < 2; ++e) {
        if (n + e >= N) continue;
        const int64_t at = static_cast<int64_t>(m) * N + n + e;
        v[e] = part[at] + part[static_cast<int64_t>(M) * N + at];
    }
    if (EPI == HAI_EPI_SILU_MUL) {
        if (n + 1 < N) y[static_cast<int64_t>(m) * ldy + n / 2] = f2bf(csilu(bfr(v[0])) * bfr(v[1]));
        return;
    }
    for (int e = 0; e < 2; ++e) {
        if (n + e >= N) continue;
        float o = bfr(v[e]);
        if (EPI == HAI_EPI_RESIDUAL) o = bf2f(res[static_cast<int64_t>(m) * ldres + n + e]) + o;
        y[static_cast<int64_t>(m) * ldy + n + e] = f2bf(o);
    }
}

// The finalize pass of a residual GEMM fused with the RMSNorm(+offset) of
// the same rows: one 256-thread block per row.  Thread t completes the
// 8-column groups t, t + 256, ... (every load issued before the first use):
// h = bf16(res + bf16(sum of the KSB partials in split order)) exactly as
// mfma_finalize_kernel<HAI_EPI_RESIDUAL> writes it.  The row is staged in LDS
// and the first wave takes the sum of squares in L64 order, then every
// thread writes xn = bf16((h * inv) * (w + off)) exactly as rmsnorm_kernel
// computes them (norm_w null: h only).
constexpr int kMaxResidualNormCols = 8192;
template <int G>
__global__ __launch_bounds__(256) void mfma_residual_rmsnorm_kernel(uint16_t* __restrict__ h, int64_t ldh,
                                                                    const float* __restrict__ part, int KSB,
                                                                    int M, int N, const uint16_t* __restrict__ w,
                                                                    float eps, float off, uint16_t* __restrict__ xn,
                                                                    int64_t ldxn) {
    __shared__ __align__(16) uint16_t hs[kMaxResidualNormCols];
    __shared__ float s_inv;
    const int tid = threadIdx.x;
    const int64_t m = blockIdx.x;
    uint16_t* hr = h + m * ldh;
    float4 pa[G][4][2];  // [group][split][half]
    u32x4 r[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int k0 = (tid + 256 * g) * 8;
        if (k0 >= N) continue;
        r[g] = *reinterpret_cast<const u32x4*>(hr + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (q < KSB) {
                const float4* pq = reinterpret_cast<const float4*>(part + (static_cast<int64_t>(q) * M + m) * N + k0);
                pa[g][q][0] = pq[0];
                pa[g][q][1] = pq[1];
            }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int k0 = (tid + 256 * g) * 8;
        if (k0 >= N) continue;
        float v[8] = {pa[g][0][0].x, pa[g][0][0].y, pa[g][0][0].z, pa[g][0][0].w,
                      pa[g][0][1].x, pa[g][0][1].y, pa[g][0][1].z, pa[g][0][1].w};
#pragma unroll
        for (int q = 1; q < 4; ++q)
            if (q < KSB) {
                v[0] = v[0] + pa[g][q][0].x; v[1] = v[1] + pa[g][q][0].y;
                v[2] = v[2] + pa[g][q][0].z; v[3] = v[3] + pa[g][q][0].w;
                v[4] = v[4] + pa[g][q][1].x; v[5] = v[5] + pa[g][q][1].y;
                v[6] = v[6] + pa[g][q][1].z; v[7] = v[7] + pa[g][q][1].w;
            }
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o[e] = f2bf2(lo_bf(r[g][e]) + bfr(v[2 * e]),
                         hi_bf(r[g][e]) + bfr(v[2 * e + 1]));
        }
        const u32x4 hv = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4*>(hr + k0) = hv;
        *reinterpret_cast<u32x4*>(hs + k0) = hv;
    }
    if (w == nullptr) return;
    __syncthreads();
    if (tid < 64) {
        // the rmsnorm_kernel order: lane l takes elements c*512 + 8l .. + 7, c increasing
        float acc = 0.0f;
        for (int k0 = tid * 8; k0 < N; k0 += 512) {
            const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + k0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a = lo_bf(hv[q]);
                const float b = hi_bf(hv[q]);
                acc = fma_(a, a, acc);
                acc = fma_(b, b, acc);
            }
        }
        const float ss = wave_sum64(acc);
        if (tid == 0) s_inv = 1.0f / csqrt(ss / static_cast<float>(N) + eps);
    }
    __syncthreads();
    const float inv = s_inv;
    uint16_t* xr = xn + m * ldxn;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int k0 = (tid + 256 * g) * 8;
        if (k0 >= N) continue;
        const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + k0);
        const u32x4 wd = *reinterpret_cast<const u32x4*>(w + k0);
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            o[q] = f2bf2((lo_bf(hv[q]) * inv) * (lo_bf(wd[q]) + off),
                         (hi_bf(hv[q]) * inv) * (hi_bf(wd[q]) + off));
        }
        *reinterpret_cast<u32x4*>(xr + k0) = u32x4{o[0], o[1], o[2], o[3]};
    }
}

// E4M3 codes (4 per word) -> 4 bf16 of the same values (exact: every E4M3
// value, the reference's +-480 included, has at most 4 significant bits);
// CHECK handles 0x7F / 0xFF, which the hardware conversion maps to NaN.
template <bool CHECK>
__device__ __forceinline__ void e4m3x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    f2v a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
    f2v b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
    if (CHECK && ((((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u) != 0u)) {
        // exact decode of fp8_dequant.cc:12-26 for the word holding a special code
        float f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = (w >> (8 * j)) & 0xffu;
            const uint32_t t = c & 0x7fu;
            float v = t >= 8u ? __uint_as_float((t << 20) + 0x3c000000u)
                              : __uint_as_float((t << 20) + 0x3c800000u) - 0x1p-6f;
            f[j] = (c & 0x80u) ? -v : v;
        }
        a = f2v{f[0], f[1]};
        b = f2v{f[2], f[3]};
    }
    lo = (__float_as_uint(a.x) >> 16) | (__float_as_uint(a.y) & 0xffff0000u);
    hi = (__float_as_uint(b.x) >> 16) | (__float_as_uint(b.y) & 0xffff0000u);
}

// FP8 weights [N, K] with 128x128 fp32 block scales (QuantizedWeight,
// qwen3_weights.cc:131-182): each wave decodes its 16 rows' codes exactly to
// bf16 into its LDS tile, the matrix cores sum every 128-k scale block on
// its own, and the block's scale of the output column (weight row) is
// applied in fp32: y = sum_kb s[sr(n)][kb] * (x . decode(q))_kb.
template <int MT, int EPI, bool CHECK, bool DB, bool SK>
__global__ __launch_bounds__(256) void gemm_fp8_mfma_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                            const uint16_t* __restrict__ x, int64_t ldx,
                                                            const uint8_t* __restrict__ wq,
                                                            const float* __restrict__ scales,
                                                            const int32_t* __restrict__ scale_rows, int paired,
                                                            const uint16_t* res, int64_t ldres, int M, int N, int K,
                                                            float* __restrict__ part, int KSB, int sk) {
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* xs = lds;                          // [16 MT][kLdsRow]
    uint16_t* ws = lds + 16 * MT * kLdsRow;      // [4 waves][16][kLdsRow], decoded bf16
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int nkb = (K + 127) / 128;
    const int nck = (K + kChunk - 1) / kChunk;
    const int nfull = K / kChunk;
    // one tile (64 weight rows) over chunks cbeg, cbeg + cstep, ... < cend;
    // plane < 0: finish y, else write partial plane `plane`
    auto piece = [&](int64_t tile, int cbeg, int cend, int cstep, int plane) {
    const int64_t row_base = tile * kBlockRows + wave * 16;

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq, static_cast<uint32_t>(static_cast<int64_t>(N) * K));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    // code loads: instruction i covers rows 4i .. 4i+3, 16 lanes x 16 codes each
    const int w_quarter = lane >> 4;
    const int w_col = (lane & 15) * 16;
    const uint32_t woff0 = static_cast<uint32_t>((row_base + w_quarter) * static_cast<int64_t>(K) + w_col);
    const uint32_t four_rows = static_cast<uint32_t>(K) * 4u;
    constexpr int XL = 2 * MT;
    uint32_t xoff[XL];
    int xrow[XL], xcol[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int e = tid + 256 * i;
        xrow[i] = e >> 5;
        xcol[i] = (e & 31) * 8;
        xoff[i] = static_cast<uint32_t>((static_cast<int64_t>(xrow[i]) * ldx + xcol[i]) * 2);
    }
    // scale row of this lane's output column (weight row row_base + li)
    const int64_t ncol = min(row_base + li, static_cast<int64_t>(N) - 1);
    const int64_t nsb = ((N >> 1) + 127) / 128;
    const int64_t srow = scale_rows ? scale_rows[ncol] : (paired ? (ncol & 1) * nsb + (ncol >> 1) / 128 : ncol / 128);
    const float* srp = scales + srow * nkb;

    f32x4 tot[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) tot[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 xv[XL];
    // codes of chunk c and the scales of its k-blocks 2c, 2c + 1 (a past-K
    // block gets a finite stand-in; its products are zero)
    auto load_w = [&](u32x4 (&wv)[4], float (&sv)[2], int c) {
        if (c < nfull) {
#pragma unroll
            for (int i = 0; i < 4; ++i) wv[i] = bload_w(rw, woff0 + i * four_rows, static_cast<uint32_t>(c) * kChunk);
        } else {
            const bool okw = c * kChunk + w_col < K;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wv[i] = bload_w(rw, okw ? woff0 + i * four_rows + static_cast<uint32_t>(c) * kChunk : kOutOfRange, 0u);
        }
        sv[0] = srp[min(2 * c, nkb - 1)];
        sv[1] = srp[min(2 * c + 1, nkb - 1)];
    };
    auto load_x = [&](int c) {
        if (c < nfull) {
#pragma unroll
            for (int i = 0; i < XL; ++i) xv[i] = bload(rx, xoff[i], static_cast<uint32_t>(c) * (kChunk * 2));
        } else {
#pragma unroll
            for (int i = 0; i < XL; ++i)
                xv[i] = bload(rx, c * kChunk + xcol[i] < K ? xoff[i] + static_cast<uint32_t>(c) * (kChunk * 2)
                                                           : kOutOfRange, 0u);
        }
    };
    // codes decoded into the wave's LDS tile, activations into the block's
    auto stage = [&](const u32x4 (&wv)[4]) {
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) e4m3x4_to_bf16<CHECK>(wv[i][q], d[2 * q], d[2 * q + 1]);
            uint16_t* dst = &ws[(wave * 16 + 4 * i + w_quarter) * kLdsRow + w_col];
            *reinterpret_cast<u32x4*>(dst) = u32x4{d[0], d[1], d[2], d[3]};
            *reinterpret_cast<u32x4*>(dst + 8) = u32x4{d[4], d[5], d[6], d[7]};
        }
#pragma unroll
        for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(&xs[xrow[i] * kLdsRow + xcol[i]]) = xv[i];
        __syncthreads();
    };
    auto compute = [&](const float s0, const float s1) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 acc[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 4 * kb; j < 4 * kb + 4; ++j) {
                const u32x4 b = *reinterpret_cast<const u32x4*>(&ws[(wave * 16 + li) * kLdsRow + 32 * j + 8 * kg]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(&xs[(16 * mt + li) * kLdsRow + 32 * j + 8 * kg]);
                    acc[mt] = mfma16(a, b, acc[mt]);
                }
            }
            const float sc = kb == 0 ? s0 : s1;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) tot[mt][i] = fma_(sc, acc[mt][i], tot[mt][i]);
        }
    };
    u32x4 wA[4];
    float sA[2];
    int c = cbeg;
    if constexpr (!DB) {
        // one chunk in flight while the current one is multiplied
        if (c < cend) { load_w(wA, sA, c); load_x(c); }
        for (; c < cend; c += cstep) {
            stage(wA);
            const float s0 = sA[0], s1 = sA[1];
            if (c + cstep < cend) { load_w(wA, sA, c + cstep); load_x(c + cstep); }
            compute(s0, s1);
        }
    } else {
        // the codes of two chunks in flight (the activations of one): the
        // next chunk's activations are requested before the codes two ahead,
        // so waiting for them leaves those codes outstanding
        u32x4 wB[4];
        float sB[2];
        if (c < cend) { load_w(wA, sA, c); load_x(c); }
        if (c + cstep < cend) load_w(wB, sB, c + cstep);
        for (; c < cend; c += 2 * cstep) {
            stage(wA);
            const float a0 = sA[0], a1 = sA[1];
            if (c + cstep < cend) load_x(c + cstep);
            if (c + 2 * cstep < cend) load_w(wA, sA, c + 2 * cstep);
            compute(a0, a1);
            if (c + cstep >= cend) break;
            stage(wB);
            const float b0 = sB[0], b1 = sB[1];
            if (c + 2 * cstep < cend) load_x(c + 2 * cstep);
            if (c + 3 * cstep < cend) load_w(wB, sB, c + 3 * cstep);
            compute(b0, b1);
        }
    }

    const int64_t n = row_base + li;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * mt + 4 * kg + i;
            if (plane < 0)
                mfma_store<EPI>(y, ldy, res, ldres, tot[mt][i], m, n, M, N, li);
            else if (m < M && n < N)
                part[(static_cast<int64_t>(plane) * M + m) * N + n] = tot[mt][i];
        }
    };
    if constexpr (!SK) {
        piece(blockIdx.x, blockIdx.y, nck, KSB, KSB == 1 ? -1 : static_cast<int>(blockIdx.y));
        return;
    }
    const int64_t ntiles = (N + kBlockRows - 1) / kBlockRows;
    const int64_t items = ntiles * nck;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * items / sk;
    const int64_t hi = (static_cast<int64_t>(blockIdx.x) + 1) * items / sk;
    for (int64_t it = lo; it < hi;) {
        const int64_t tile = it / nck;
        const int c0 = static_cast<int>(it - tile * nck);
        const int c1 = static_cast<int>(min(hi - tile * nck, static_cast<int64_t>(nck)));
        const int plane = (c0 == 0 && c1 == nck) ? -1 : (sk_block_of(tile * nck, items, sk) == blockIdx.x ? 0 : 1);
        piece(tile, c0, c1, 1, plane);  // (a piece's first chunk waits for the LDS reads of the last one)
        it = tile * nck + c1;
    }
}

// ---------------------------------------------------------------------------
// Register-operand variant of the batched GEMMs (bf16 and FP8 weights, 32 or
// 64 activation rows, K a multiple of 256).  The kernels above pass every
// weight through LDS (written decoded, read back in the MFMA layout) and
// give each wave 16 weight rows, so each activation operand read from LDS
// feeds one MFMA; at 64 rows that is 14 LDS bytes per FP8 code and the
// kernel is LDS-bound.  Here:
//   * weights go straight into the MFMA B-operand registers: one load
//     instruction covers 8 rows x 128 contiguous bytes (lane (li, kg) of
//     load I0 takes row li % 8, 16-byte piece kg + 4 (li >= 8); I1 the rows
//     8..15 with the halves swapped), and a select plus a DPP row rotate by 8
//     lanes turn the pair into the operands of two MFMA k-slices (R0: piece
//     kg of row li, R1: piece kg + 4).  Every instruction reads whole 128-byte
//     lines; an MFMA-layout load (16 rows x 64 bytes per instruction)
//     measured 3.9-4.7 TB/s against 6.1-7.1 for this form on MI355X;
//   * a wave owns 32 weight rows (two MFMA column tiles), so each activation
//     operand read feeds two MFMAs, and one half of every 256-k chunk (for
//     FP8 exactly one 128-k scale block); the two k-halves of a tile meet in
//     LDS at the end, added in a fixed order;
//   * a chunk's activation rows are loaded one chunk ahead (rows past M read
//     zeros) and written to LDS after the current chunk is multiplied, each
//     row's 16-byte pieces XOR-swizzled by the row index so that the 16 rows
//     an operand read touches fall in distinct banks; two chunk buffers, one
//     barrier per chunk.  (Buffer -> LDS copies would save the registers,
//     but the compiler cannot tell which buffer a copy writes and drains
//     every outstanding load before the next LDS read: vmcnt(0) per chunk.)
//   * the weights of the next two chunks are in flight while one is
//     multiplied.
// Same tiles (64 weight rows per block), K splits, stream-K and epilogues as
// the kernels above; tolerance mode as they are.  Used where it measured
// faster (use_rt below).
// ---------------------------------------------------------------------------
constexpr int kRtChunk = 256;  // k per chunk (two 128-k halves)

template <bool FP8>
struct RtLoads {
    static constexpr int kPerTile = FP8 ? 2 : 4;  // 16-byte weight loads per n-tile and chunk half
    static constexpr int kPerChunk = 2 * kPerTile;
};

template <int MT, int EPI, bool FP8, bool CHECK, bool SK>
__global__ __launch_bounds__(256) void gemm_rt_mfma_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                           const uint16_t* __restrict__ x, int64_t ldx,
                                                           const void* w, const float* __restrict__ scales,
                                                           const int32_t* __restrict__ scale_rows, int paired,
                                                           const uint16_t* res, int64_t ldres, int M, int N, int K,
                                                           float* __restrict__ part, int KSB, int sk) {
    constexpr int XR = 16 * MT;              // staged activation rows
    constexpr int XBUF = XR * kRtChunk;      // bf16 elements per chunk buffer
    constexpr int NW = RtLoads<FP8>::kPerChunk;
    constexpr int EB = FP8 ? 1 : 2;          // weight bytes per element
    extern __shared__ __align__(16) uint16_t lds[];  // [2][XR][256], pieces swizzled; then the k-half sums
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int nh = wave & 1;   // rows 32 nh .. 32 nh + 31 of the tile
    const int kh = wave >> 1;  // k-half of every chunk
    const bool low = li < 8;
    const int nck = K / kRtChunk;
    const int nkb = K / 128;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(static_cast<int64_t>(N) * K * EB));
    // activation pieces of a chunk: thread piece e = tid + 256 i is row e / 32,
    // LDS position e % 32, holding the row's piece position ^ (row % 16);
    // rows past M start past the buffer and read zeros
    constexpr int XP = XR / 8;  // pieces per thread and chunk
    uint32_t xoff[XP];
    int xdst[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int e = static_cast<int>(threadIdx.x) + 256 * i;
        const int r = e >> 5;
        const int pos = e & 31;
        xoff[i] = static_cast<uint32_t>((static_cast<int64_t>(r) * ldx + ((pos ^ (r & 15)) * 8)) * 2);
        xdst[i] = r * kRtChunk + pos * 8;
    }
    auto load_x = [&](u32x4 (&xv)[XP], int c) {
#pragma unroll
        for (int i = 0; i < XP; ++i) xv[i] = bload(rx, xoff[i], static_cast<uint32_t>(c) * (kRtChunk * 2));
    };
    auto store_x = [&](const u32x4 (&xv)[XP], int buf) {
#pragma unroll
        for (int i = 0; i < XP; ++i) *reinterpret_cast<u32x4*>(lds + buf * XBUF + xdst[i]) = xv[i];
    };
    // A operand: 8 elements of row 16 mt + li at 16-byte piece p of the chunk
    auto a_op = [&](int buf, int mt, int p) -> u32x4 {
        return *reinterpret_cast<const u32x4*>(lds + buf * XBUF + (16 * mt + li) * kRtChunk + ((p ^ li) * 8));
    };

    auto piece = [&](int64_t tile, int cbeg, int cend, int cstep, int plane) {
        const int64_t row_base = tile * kBlockRows + 32 * nh;
        // per n-tile: byte offsets of loads I0 (rows 0..7) and I1 (rows 8..15) at chunk 0
        uint32_t wo0[2], wo1[2];
        const float* srp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t ra = row_base + 16 * t + (li & 7);
            const int p0 = kg + (low ? 0 : 4), p1 = kg + (low ? 4 : 0);
            wo0[t] = static_cast<uint32_t>((ra * K + kh * 128) * EB + p0 * 16);
            wo1[t] = static_cast<uint32_t>(((ra + 8) * K + kh * 128) * EB + p1 * 16);
            if constexpr (FP8) {
                const int64_t ncol = min(row_base + 16 * t + li, static_cast<int64_t>(N) - 1);
                const int64_t nsb = ((N >> 1) + 127) / 128;
                const int64_t srow =
                    scale_rows ? scale_rows[ncol] : (paired ? (ncol & 1) * nsb + (ncol >> 1) / 128 : ncol / 128);
                srp[t] = scales + srow * nkb + kh;
            } else {
                srp[t] = nullptr;
            }
        }
        f32x4 tot[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) tot[mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        auto load_w = [&](u32x4 (&wv)[NW], int c) {
            const uint32_t off = static_cast<uint32_t>(c) * (kRtChunk * EB);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < NW / 4; ++j) {  // bf16: two 64-k pairs per half, FP8: one
                    wv[(t * (NW / 4) + j) * 2] = bload_w(rw, wo0[t] + j * 128, off);
                    wv[(t * (NW / 4) + j) * 2 + 1] = bload_w(rw, wo1[t] + j * 128, off);
                }
        };
        auto load_s = [&](float (&sv)[2], int c) {
            if constexpr (FP8) {
                sv[0] = srp[0][2 * c];
                sv[1] = srp[1][2 * c];
            }
        };
        // rearranged pair of one load pair: R0 = piece kg of row li, R1 = piece kg + 4
        auto operands = [&](const u32x4& i0, const u32x4& i1, u32x4& r0, u32x4& r1) {
            rows8x128_to_operands(i0, i1, low, r0, r1);
        };
        auto compute = [&](const u32x4 (&wv)[NW], const float (&sv)[2], int buf) {
            if constexpr (FP8) {
                // 128 codes of the wave's half: R0 holds k 16 kg .. + 15, R1 k 64 + 16 kg .. + 15
                u32x4 b[2][4];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    u32x4 r0, r1;
                    operands(wv[2 * t], wv[2 * t + 1], r0, r1);
                    uint32_t d[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        e4m3x4_to_bf16<CHECK>(r0[q], d[2 * q], d[2 * q + 1]);
                        e4m3x4_to_bf16<CHECK>(r1[q], d[8 + 2 * q], d[8 + 2 * q + 1]);
                    }
                    b[t][0] = u32x4{d[0], d[1], d[2], d[3]};
                    b[t][1] = u32x4{d[4], d[5], d[6], d[7]};
                    b[t][2] = u32x4{d[8], d[9], d[10], d[11]};
                    b[t][3] = u32x4{d[12], d[13], d[14], d[15]};
                }
                const int pa = 16 * kh + 2 * kg;
                const int poff[4] = {0, 1, 8, 9};
                f32x4 acc[MT][2];
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const u32x4 a = a_op(buf, mt, pa + poff[s4]);
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            acc[mt][t] = mfma16(a, b[t][s4], s4 == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : acc[mt][t]);
                    }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) tot[mt][t][i] = fma_(sv[t], acc[mt][t][i], tot[mt][t][i]);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    u32x4 b[2][2];
#pragma unroll
                    for (int t = 0; t < 2; ++t) operands(wv[(t * 2 + j) * 2], wv[(t * 2 + j) * 2 + 1], b[t][0], b[t][1]);
                    const int pa = 16 * kh + 8 * j + kg;
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            const u32x4 a = a_op(buf, mt, pa + 4 * h);
#pragma unroll
                            for (int t = 0; t < 2; ++t) tot[mt][t] = mfma16(a, b[t][h], tot[mt][t]);
                        }
                }
            }
        };

        __syncthreads();  // the previous piece's LDS reads are done
        u32x4 wA[NW], wB[NW], wC[NW], xv[XP];
        float sA[2] = {0.0f, 0.0f}, sB[2] = {0.0f, 0.0f}, sC[2] = {0.0f, 0.0f};
        // Loads are issued unconditionally (a chunk past the piece is clamped
        // to the last one and its values are never used), so that the code
        // between the waits is straight-line and the compiler's wait counts
        // stay exact: a load inside a branch makes them drain everything.
        auto clampc = [&](int c) { return min(c, nck - 1); };
        if (cbeg < cend) {
            load_x(xv, cbeg);
            load_s(sA, cbeg);
            load_w(wA, cbeg);
            load_s(sB, clampc(cbeg + cstep));
            load_w(wB, clampc(cbeg + cstep));
            store_x(xv, 0);
        }
        // chunk i (its activations in buffer i % 2): barrier, request the
        // activations of chunk i + 1 and the weights of chunk i + 2, multiply
        // chunk i, write chunk i + 1's activations to the other buffer
        auto step = [&](int i, u32x4 (&cur)[NW], const float (&scur)[2], u32x4 (&pre)[NW], float (&spre)[2]) {
            const int c = cbeg + i * cstep;
            if (c >= cend) return false;
            lds_barrier();
            load_x(xv, clampc(c + cstep));
            load_s(spre, clampc(c + 2 * cstep));
            load_w(pre, clampc(c + 2 * cstep));
            // the requests stay ahead of the multiply (the scheduler would
            // otherwise sink them below it to shorten register lifetimes)
            pin_memory_order();
            __builtin_amdgcn_sched_barrier(0);
            compute(cur, scur, i & 1);
            pin_memory_order();
            __builtin_amdgcn_sched_barrier(0);
            store_x(xv, (i + 1) & 1);
            return true;
        };
        for (int i = 0;; i += 3) {
            if (!step(i, wA, sA, wC, sC)) break;
            if (!step(i + 1, wB, sB, wA, sA)) break;
            if (!step(i + 2, wC, sC, wB, sB)) break;
        }

        // the two k-halves of the tile: half 1 through LDS, added to half 0
        __syncthreads();
        float* red = reinterpret_cast<float*>(lds);  // [2 nh][MT][2][64 lanes] f32x4
        if (kh == 1) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    *reinterpret_cast<f32x4*>(red + (((nh * MT + mt) * 2 + t) * 64 + lane) * 4) = tot[mt][t];
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const f32x4 o = *reinterpret_cast<const f32x4*>(red + (((nh * MT + mt) * 2 + t) * 64 + lane) * 4);
                tot[mt][t] = tot[mt][t] + o;
            }
        // D layout: lane (li, kg) holds rows 16 mt + 4 kg + i of column row_base + 16 t + li
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t n = row_base + 16 * t + li;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 16 * mt + 4 * kg + i;
                    if (plane < 0)
                        mfma_store<EPI>(y, ldy, res, ldres, tot[mt][t][i], m, n, M, N, li);
                    else if (m < M && n < N)
                        part[(static_cast<int64_t>(plane) * M + m) * N + n] = tot[mt][t][i];
                }
        }
    };
    // chunk indices below are in units of kRtChunk == kChunk
    if constexpr (!SK) {
        piece(blockIdx.x, blockIdx.y, nck, KSB, KSB == 1 ? -1 : static_cast<int>(blockIdx.y));
        return;
    }
    const int64_t ntiles = (N + kBlockRows - 1) / kBlockRows;
    const int64_t items = ntiles * nck;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * items / sk;
    const int64_t hi = (static_cast<int64_t>(blockIdx.x) + 1) * items / sk;
    for (int64_t it = lo; it < hi;) {
        const int64_t tile = it / nck;
        const int c0 = static_cast<int>(it - tile * nck);
        const int c1 = static_cast<int>(min(hi - tile * nck, static_cast<int64_t>(nck)));
        const int plane = (c0 == 0 && c1 == nck) ? -1 : (sk_block_of(tile * nck, items, sk) == blockIdx.x ? 0 : 1);
        piece(tile, c0, c1, 1, plane);
        it = tile * nck + c1;
    }
}

// ---------------------------------------------------------------------------
// Copy-staged variant for FP8 weights on the wide layers at 17-64 rows: the
// register-operand kernel's tile, roles and arithmetic (a wave owns 32
// weight rows and one 128-k half of every 256-k chunk, codes decoded
// exactly to bf16 in its B operands, scale blocks applied in fp32), with
// every operand staged by global -> LDS copies instead of registers, so
// that the weight bytes in flight are bounded by LDS rather than by VGPRs:
//   * three weight stages (64 rows x 256 codes, 16 KB, and behind them the
//     chunk's scales, one 4-byte copy per lane and n-tile) and three
//     activation stages (16 MT rows x 256 bf16); the weights, scales and
//     activations of chunk i + 2 are requested before chunk i is
//     multiplied, and one s_waitcnt counts them;
//   * the stages are read by inline ds_read instructions that wait for
//     their own results: the compiler's wait insertion cannot tell a copy
//     into one stage from a read of another and would otherwise drain every
//     outstanding copy (s_waitcnt vmcnt(0)) before each LDS read;
//   * a wave copies and reads only its own weight region (32 rows x 128
//     bytes, row r's 16-byte piece p at slot p ^ (r & 7)); the activation
//     stages are filled by all four waves (row r's piece p at slot
//     p ^ (r & 15), as the register-operand kernel stores them) and read by
//     all behind a barrier.
// Weight rows past N and activation rows past M are read from the last row
// (their results are never stored); chunks past K from the last chunk
// (never used).
// ---------------------------------------------------------------------------
// One global -> LDS copy per lane of 16 bytes (to lds + 16 * lane) or 4
// bytes (to lds + 4 * lane).  __device__ functions rather than calls inside
// the kernel's lambdas: the host pass instantiates those lambdas too, and
// the builtin there made it drop the kernel's host stub.
__device__ __forceinline__ void copy16_to_lds(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void copy4_to_lds(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
// Reads of the copy-staged kernel, each group complete when its asm ends.
__device__ __forceinline__ void lds_b128x4_b32x2(const uint32_t (&a)[4], const uint32_t (&sa)[2], u32x4 (&r)[4],
                                                 float (&f)[2]) {
    asm volatile(
        "ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\tds_read_b128 %2, %8\n\tds_read_b128 %3, %9\n\t"
        "ds_read_b32 %4, %10\n\tds_read_b32 %5, %11\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(f[0]), "=&v"(f[1])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(sa[0]), "v"(sa[1])
        : "memory");
}
__device__ __forceinline__ void lds_b128x4(const uint32_t (&a)[4], u32x4 (&r)[4]) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
        : "memory");
}
__device__ __forceinline__ void lds_b128x8(const uint32_t (&a)[8], u32x4 (&r)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\tds_read_b128 %2, %10\n\tds_read_b128 %3, %11\n\t"
        "ds_read_b128 %4, %12\n\tds_read_b128 %5, %13\n\tds_read_b128 %6, %14\n\tds_read_b128 %7, %15\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7])
        : "memory");
}

// One block per 64-row tile over the whole K (the grid is the tiles).
template <int MT, int EPI, bool CHECK>
__global__ __launch_bounds__(256) void gemm_dma_mfma_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                            const uint16_t* __restrict__ x, int64_t ldx,
                                                            const uint8_t* w, const float* __restrict__ scales,
                                                            const int32_t* __restrict__ scale_rows, int paired,
                                                            const uint16_t* res, int64_t ldres, int M, int N,
                                                            int K) {
    static_assert(MT == 2 || MT == 4, "32 or 64 activation rows");
    constexpr int XR = 16 * MT;                // staged activation rows
    constexpr int XE = XR * kRtChunk;          // bf16 elements per activation stage
    constexpr int WB = kBlockRows * kRtChunk;  // weight bytes per stage
    constexpr int WS = WB + 4 * 2 * 256;       // + the scales: [wave][n-tile][64 lanes] floats
    constexpr int XOPS = 2 * MT;               // 1 KB activation copies per wave and chunk
    constexpr int kAhead = 12 + 4 * MT;        // requests issued after a chunk's activations
    __shared__ __align__(16) uint16_t xs0[XE], xs1[XE], xs2[XE];
    __shared__ __align__(16) uint8_t ws0[WS], ws1[WS], ws2[WS];
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int nh = wave & 1;
    const int kh = wave >> 1;
    const int nck = K / kRtChunk;
    const int nkb = K / 128;

    // activation copies: piece e = (wave * XOPS + i) * 64 + lane is row e / 32,
    // slot e % 32, holding the row's piece slot ^ (row % 16)
    const uint16_t* xsrc[XOPS];
#pragma unroll
    for (int i = 0; i < XOPS; ++i) {
        const int e = (wave * XOPS + i) * 64 + lane;
        const int r = e >> 5;
        const int pos = e & 31;
        xsrc[i] = x + static_cast<int64_t>(min(r, M - 1)) * ldx + (pos ^ (r & 15)) * 8;
    }
    auto copy_x = [&](uint16_t* st, int c) {
#pragma unroll
        for (int i = 0; i < XOPS; ++i)
            copy16_to_lds(xsrc[i] + c * kRtChunk, st + (wave * XOPS + i) * 512);
    };
    // LDS byte offsets of the A operands within a stage: 8 elements of row
    // 16 mt + li at 16-byte piece pa + poff[s4]
    const int pa = 16 * kh + 2 * kg;
    const int poff[4] = {0, 1, 8, 9};
    uint32_t aoff[4][MT];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            aoff[s4][mt] = static_cast<uint32_t>(((16 * mt + li) * kRtChunk + (((pa + poff[s4]) ^ li) * 8)) * 2);
    // B operands: row 16 t + li of the wave's region, pieces kg and kg + 4
    uint32_t boff[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        boff[2 * t] = static_cast<uint32_t>(wave * 4096 + (16 * t + li) * 128 + ((kg ^ (li & 7)) * 16));
        boff[2 * t + 1] = static_cast<uint32_t>(wave * 4096 + (16 * t + li) * 128 + (((kg + 4) ^ (li & 7)) * 16));
    }
    const uint32_t soff[2] = {static_cast<uint32_t>(WB + (wave * 2 + 0) * 256 + lane * 4),
                              static_cast<uint32_t>(WB + (wave * 2 + 1) * 256 + lane * 4)};

    {
        const int64_t row_base = static_cast<int64_t>(blockIdx.x) * kBlockRows + 32 * nh;
        // weight copies j = 0..3 of the wave's region: rows 8 j + lane / 8,
        // slot lane % 8 holding piece slot ^ (lane / 8)
        const uint8_t* wsrc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t row = min(row_base + 8 * j + (lane >> 3), static_cast<int64_t>(N) - 1);
            wsrc[j] = w + row * K + kh * 128 + (((lane & 7) ^ (lane >> 3)) * 16);
        }
        const float* srp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t ncol = min(row_base + 16 * t + li, static_cast<int64_t>(N) - 1);
            const int64_t nsb = ((N >> 1) + 127) / 128;
            const int64_t srow =
                scale_rows ? scale_rows[ncol] : (paired ? (ncol & 1) * nsb + (ncol >> 1) / 128 : ncol / 128);
            srp[t] = scales + srow * nkb + kh;
        }
        // the chunk's weights, then its two scales (copies of 16 and 4 bytes)
        auto copy_w = [&](uint8_t* st, int c) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                copy16_to_lds(wsrc[j] + c * kRtChunk, st + wave * 4096 + j * 1024);
#pragma unroll
            for (int t = 0; t < 2; ++t)
                copy4_to_lds(srp[t] + 2 * c, st + WB + (wave * 2 + t) * 256);
        };
        f32x4 tot[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) tot[mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        auto compute = [&](const uint8_t* wst, const uint16_t* xst) {
            const uint32_t wb = lds_addr(wst), xb = lds_addr(xst);
            // the B operands, the scales and the A operands of the first two k-steps
            u32x4 rw[4];
            float sv[2];
            const uint32_t ba[4] = {wb + boff[0], wb + boff[1], wb + boff[2], wb + boff[3]};
            const uint32_t sa[2] = {wb + soff[0], wb + soff[1]};
            u32x4 av[4][MT];
            if constexpr (MT == 4) {
                lds_b128x4_b32x2(ba, sa, rw, sv);
                const uint32_t aa[8] = {xb + aoff[0][0], xb + aoff[0][1], xb + aoff[0][2], xb + aoff[0][3],
                                        xb + aoff[1][0], xb + aoff[1][1], xb + aoff[1][2], xb + aoff[1][3]};
                u32x4 ar[8];
                lds_b128x8(aa, ar);
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i / 4][i % 4] = ar[i];
            } else {
                lds_b128x4_b32x2(ba, sa, rw, sv);
                const uint32_t aa[4] = {xb + aoff[0][0], xb + aoff[0][1], xb + aoff[1][0], xb + aoff[1][1]};
                u32x4 ar[4];
                lds_b128x4(aa, ar);
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i / 2][i % 2] = ar[i];
            }
            // 128 codes of the wave's half per row: piece kg holds k 16 kg .. + 15,
            // piece kg + 4 k 64 + 16 kg .. + 15
            u32x4 b[2][4];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint32_t d[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    e4m3x4_to_bf16<CHECK>(rw[2 * t][q], d[2 * q], d[2 * q + 1]);
                    e4m3x4_to_bf16<CHECK>(rw[2 * t + 1][q], d[8 + 2 * q], d[8 + 2 * q + 1]);
                }
                b[t][0] = u32x4{d[0], d[1], d[2], d[3]};
                b[t][1] = u32x4{d[4], d[5], d[6], d[7]};
                b[t][2] = u32x4{d[8], d[9], d[10], d[11]};
                b[t][3] = u32x4{d[12], d[13], d[14], d[15]};
            }
            f32x4 acc[MT][2];
#pragma unroll
            for (int s4 = 0; s4 < 2; ++s4)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        acc[mt][t] = mfma16(av[s4][mt], b[t][s4], s4 == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : acc[mt][t]);
            // the A operands of the last two k-steps, read while those run
            if constexpr (MT == 4) {
                const uint32_t aa[8] = {xb + aoff[2][0], xb + aoff[2][1], xb + aoff[2][2], xb + aoff[2][3],
                                        xb + aoff[3][0], xb + aoff[3][1], xb + aoff[3][2], xb + aoff[3][3]};
                u32x4 ar[8];
                lds_b128x8(aa, ar);
#pragma unroll
                for (int i = 0; i < 8; ++i) av[2 + i / 4][i % 4] = ar[i];
            } else {
                const uint32_t aa[4] = {xb + aoff[2][0], xb + aoff[2][1], xb + aoff[3][0], xb + aoff[3][1]};
                u32x4 ar[4];
                lds_b128x4(aa, ar);
#pragma unroll
                for (int i = 0; i < 4; ++i) av[2 + i / 2][i % 2] = ar[i];
            }
#pragma unroll
            for (int s4 = 2; s4 < 4; ++s4)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t) acc[mt][t] = mfma16(av[s4][mt], b[t][s4], acc[mt][t]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) tot[mt][t][i] = fma_(sv[t], acc[mt][t][i], tot[mt][t][i]);
        };

        auto clampc = [&](int c) { return min(c, nck - 1); };
        // order (weights, then activations, per chunk): a chunk's activations
        // are followed by exactly kAhead requests when its step waits
        copy_w(ws0, 0);
        copy_x(xs0, 0);
        copy_w(ws1, clampc(1));
        copy_x(xs1, clampc(1));
        // chunk i: barrier (every wave is done with chunk i - 1), request the
        // weights, scales and activations of chunk i + 2 into the stages
        // chunk i - 1 used, wait for chunk i's copies, barrier (all waves'
        // activation copies landed), multiply
        auto step = [&](int i, const uint8_t* wcur, const uint16_t* xcur, uint8_t* wnext, uint16_t* xnext) {
            if (i >= nck) return false;
            lds_barrier();
            pin_memory_order();
            __builtin_amdgcn_sched_barrier(0);
            copy_w(wnext, clampc(i + 2));
            copy_x(xnext, clampc(i + 2));
            pin_memory_order();
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<kAhead>();
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            compute(wcur, xcur);
            return true;
        };
        for (int i = 0;; i += 3) {
            if (!step(i, ws0, xs0, ws2, xs2)) break;
            if (!step(i + 1, ws1, xs1, ws0, xs0)) break;
            if (!step(i + 2, ws2, xs2, ws1, xs1)) break;
        }

        // the two k-halves of the tile: half 1 through LDS, added to half 0
        wait_vmcnt<0>();
        __syncthreads();
        float* red = reinterpret_cast<float*>(xs0);  // [2 nh][MT][2][64 lanes] f32x4
        if (kh == 1) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    *reinterpret_cast<f32x4*>(red + (((nh * MT + mt) * 2 + t) * 64 + lane) * 4) = tot[mt][t];
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const f32x4 o = *reinterpret_cast<const f32x4*>(red + (((nh * MT + mt) * 2 + t) * 64 + lane) * 4);
                    tot[mt][t] = tot[mt][t] + o;
                }
            // D layout: lane (li, kg) holds rows 16 mt + 4 kg + i of column row_base + 16 t + li
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int64_t n = row_base + 16 * t + li;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        mfma_store<EPI>(y, ldy, res, ldres, tot[mt][t][i], 16 * mt + 4 * kg + i, n, M, N, li);
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
    float* part;
    int KSB;
    // FP8 weights (wq != nullptr)
    const uint8_t* wq = nullptr;
    const float* scales = nullptr;
    const int32_t* scale_rows = nullptr;
    int paired = 0;
    bool check = true;
    bool keep = false;  // leave the K-split partials for hai_mfma_residual_rmsnorm_bf16
    size_t ws_bytes = 0;
};

int device_cus();

// LDS above the 64 KB default needs the attribute, once per kernel instance.
int allow_lds(const void* kern, size_t shmem, bool* done) {
    if (*done) return HAI_OK;
    const int rc = check_hip(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(shmem)),
                             "hipFuncSetAttribute");
    if (rc == HAI_OK) *done = true;
    return rc;
}

// Stream-K when the plain grid would load the CUs unevenly.  The time of a
// matrix-core GEMM follows its busiest CU: 544 tiles of 64 rows on 256 CUs
// put 3 blocks on 32 CUs and 2 on the rest, and those take 1.5x as long
// (MI355X, M = 32: 512 tiles 56 us, 544 tiles 74 us; at M = 64, two
// resident blocks per CU, the 32 extra tiles even form a second round: 63 ->
// 94 us).  With ntiles = (k + f) x CUs, 1 <= k <= the blocks a CU holds and
// 0 < f <= 0.25, stream-K runs k x CUs blocks of (k + f) / k tiles each
// (544 tiles: M = 64 FP8 94 -> 80 us, M = 32 bf16 74 -> 70 us, with the
// finalize pass); every tile then spans at most two blocks.  At f = 0.5 (640
// tiles) or more than k blocks per CU the plain grid measured as fast or
// faster.
int sk_blocks(const void* kern, size_t shmem, const MfmaArgs& a) {
    if (a.KSB != 1 || a.keep || a.part == nullptr ||
        a.ws_bytes < static_cast<size_t>(2) * a.M * a.N * sizeof(float))
        return 0;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 0;
    const int64_t ntiles = (static_cast<int64_t>(a.N) + kBlockRows - 1) / kBlockRows;
    const int64_t per_cu = resident_blocks(kern, shmem) / cus;
    const int64_t k = ntiles / cus;
    const int64_t rem = ntiles - k * cus;  // f x CUs
    if (k < 1 || k > per_cu || rem == 0 || 4 * rem > cus) return 0;
    return static_cast<int>(k * cus);
}

// The register-operand kernels serve K % 256 == 0 and up to 64 rows; the
// environment variable HAI_MFMA_RT (read once per process) selects them for
// the shapes use_rt names (unset or 1), never (0), or for every eligible
// shape (2, for measurements).
int rt_mode() {
    static const int mode = [] {
        const char* e = std::getenv("HAI_MFMA_RT");
        return e == nullptr ? 1 : (e[0] == '0' ? 0 : (e[0] == '2' ? 2 : 1));
    }();
    return mode;
}

template <int MT, int EPI>
int launch_rt(const MfmaArgs& a, hipStream_t s) {
    const size_t shmem = static_cast<size_t>(2) * 16 * MT * kRtChunk * 2;
    const dim3 grid(static_cast<unsigned>((a.N + kBlockRows - 1) / kBlockRows), static_cast<unsigned>(a.KSB));
    const void* w = a.wq != nullptr ? static_cast<const void*>(a.wq) : static_cast<const void*>(a.w);
    using Kern = void (*)(uint16_t*, int64_t, const uint16_t*, int64_t, const void*, const float*, const int32_t*,
                          int, const uint16_t*, int64_t, int, int, int, float*, int, int);
    Kern kern, kern_sk;
    int slot;
    if (a.wq == nullptr) {
        kern = gemm_rt_mfma_kernel<MT, EPI, false, false, false>;
        kern_sk = gemm_rt_mfma_kernel<MT, EPI, false, false, true>;
        slot = 0;
    } else if (a.check) {
        kern = gemm_rt_mfma_kernel<MT, EPI, true, true, false>;
        kern_sk = gemm_rt_mfma_kernel<MT, EPI, true, true, true>;
        slot = 1;
    } else {
        kern = gemm_rt_mfma_kernel<MT, EPI, true, false, false>;
        kern_sk = gemm_rt_mfma_kernel<MT, EPI, true, false, true>;
        slot = 2;
    }
    static bool attr[6] = {false, false, false, false, false, false};
    int rc = allow_lds(reinterpret_cast<const void*>(kern), shmem, &attr[2 * slot]);
    if (rc == HAI_OK) rc = allow_lds(reinterpret_cast<const void*>(kern_sk), shmem, &attr[2 * slot + 1]);
    if (rc != HAI_OK) return rc;
    const int sk = sk_blocks(reinterpret_cast<const void*>(kern_sk), shmem, a);
    if (sk)
        kern_sk<<<dim3(static_cast<unsigned>(sk)), dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, w, a.scales,
                                                                         a.scale_rows, a.paired, a.res, a.ldres, a.M,
                                                                         a.N, a.K, a.part, a.KSB, sk);
    else
        kern<<<grid, dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, w, a.scales, a.scale_rows, a.paired, a.res,
                                            a.ldres, a.M, a.N, a.K, a.part, a.KSB, 0);
    rc = launched("gemm_rt_mfma_kernel");
    if (rc != HAI_OK) return rc;
    const int64_t n = static_cast<int64_t>(a.M) * ((a.N + 1) / 2);
    if (sk) {
        mfma_sk_finalize_kernel<EPI><<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(
            a.y, a.ldy, a.part, a.res, a.ldres, a.M, a.N, (a.K + kChunk - 1) / kChunk, sk);
        return launched("mfma_sk_finalize_kernel");
    }
    if (a.KSB == 1 || a.keep) return HAI_OK;
    mfma_finalize_kernel<EPI><<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(
        a.y, a.ldy, a.part, a.KSB, a.res, a.ldres, a.M, a.N);
    return launched("mfma_finalize_kernel");
}

// The copy-staged FP8 kernel: one block per 64-row tile (150 KB of LDS at
// 64 rows, one block per CU), K not split.
template <int MT, int EPI>
int launch_dma(const MfmaArgs& a, hipStream_t s) {
    auto* kern = a.check ? gemm_dma_mfma_kernel<MT, EPI, true> : gemm_dma_mfma_kernel<MT, EPI, false>;
    const int64_t ntiles = (static_cast<int64_t>(a.N) + kBlockRows - 1) / kBlockRows;
    kern<<<dim3(static_cast<unsigned>(ntiles)), dim3(256), 0, s>>>(a.y, a.ldy, a.x, a.ldx, a.wq, a.scales,
                                                                  a.scale_rows, a.paired, a.res, a.ldres, a.M, a.N,
                                                                  a.K);
    return launched("gemm_dma_mfma_kernel");
}

template <int MT, int EPI>
int launch_mfma(const MfmaArgs& a, hipStream_t s) {
    const size_t shmem = static_cast<size_t>(16 * MT + 4 * 16) * kLdsRow * 2;
    const dim3 grid(static_cast<unsigned>((a.N + kBlockRows - 1) / kBlockRows), static_cast<unsigned>(a.KSB));
    int rc;
    int sk = 0;
    if (a.wq != nullptr) {
        // two chunks of codes in flight from 64 rows (measured on MI355X at
        // M = 64: gate/up 108 -> 90 us; at M = 32 one chunk is faster)
        constexpr bool kDB = MT >= 4;
        auto* kern = a.check ? gemm_fp8_mfma_kernel<MT, EPI, true, kDB, false>
                             : gemm_fp8_mfma_kernel<MT, EPI, false, kDB, false>;
        auto* kern_sk = a.check ? gemm_fp8_mfma_kernel<MT, EPI, true, kDB, true>
                                : gemm_fp8_mfma_kernel<MT, EPI, false, kDB, true>;
        static bool attr[4] = {false, false, false, false};
        rc = allow_lds(reinterpret_cast<const void*>(kern), shmem, &attr[a.check ? 1 : 0]);
        if (rc == HAI_OK) rc = allow_lds(reinterpret_cast<const void*>(kern_sk), shmem, &attr[a.check ? 3 : 2]);
        if (rc != HAI_OK) return rc;
        sk = sk_blocks(reinterpret_cast<const void*>(kern_sk), shmem, a);
        if (sk)
            kern_sk<<<dim3(static_cast<unsigned>(sk)), dim3(256), shmem, s>>>(
                a.y, a.ldy, a.x, a.ldx, a.wq, a.scales, a.scale_rows, a.paired, a.res, a.ldres, a.M, a.N, a.K, a.part,
                a.KSB, sk);
        else
            kern<<<grid, dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, a.wq, a.scales, a.scale_rows, a.paired,
                                                a.res, a.ldres, a.M, a.N, a.K, a.part, a.KSB, 0);
        rc = launched("gemm_fp8_mfma_kernel");
    } else {
        auto* kern = gemm_bf16_mfma_kernel<MT, EPI, false>;
        auto* kern_sk = gemm_bf16_mfma_kernel<MT, EPI, true>;
        static bool attr[2] = {false, false};
        rc = allow_lds(reinterpret_cast<const void*>(kern), shmem, &attr[0]);
        if (rc == HAI_OK) rc = allow_lds(reinterpret_cast<const void*>(kern_sk), shmem, &attr[1]);
        if (rc != HAI_OK) return rc;
        sk = sk_blocks(reinterpret_cast<const void*>(kern_sk), shmem, a);
        if (sk)
            kern_sk<<<dim3(static_cast<unsigned>(sk)), dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, a.w, a.res,
                                                                             a.ldres, a.M, a.N, a.K, a.part, a.KSB,
                                                                             sk);
        else
            kern<<<grid, dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, a.w, a.res, a.ldres, a.M, a.N, a.K, a.part,
                                                a.KSB, 0);
        rc = launched("gemm_bf16_mfma_kernel");
    }
    if (rc != HAI_OK) return rc;
    const int64_t n = static_cast<int64_t>(a.M) * ((a.N + 1) / 2);
    if (sk) {
        mfma_sk_finalize_kernel<EPI><<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(
            a.y, a.ldy, a.part, a.res, a.ldres, a.M, a.N, (a.K + kChunk - 1) / kChunk, sk);
        return launched("mfma_sk_finalize_kernel");
    }
    if (a.KSB == 1 || a.keep) return HAI_OK;
    mfma_finalize_kernel<EPI><<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(
        a.y, a.ldy, a.part, a.KSB, a.res, a.ldres, a.M, a.N);
    return launched("mfma_finalize_kernel");
}

// Where the register-operand kernels run: FP8 weights, 17-64 rows, the
// narrow (N <= 8192, K-split) layers.  Measured on MI355X against the
// LDS-staged kernels (C5 shapes): down 46.9 -> 37.3 us at M = 64 and 38.1
// -> 27.1 us at M = 32, out / o 21.8 -> 19.9 and 16.9 -> 13.9 us.  The wide
// layers (one tile per block over the whole K) lost with them (gate|up at
// M = 64 83 -> 114 us: two resident blocks per CU keep too few weight
// bytes in flight), and so did bf16 weights at 32 rows; those keep the
// LDS-staged kernels.
// The copy-staged kernel: FP8 weights, 17-64 rows, layers wider than 8192
// rows with at most one 64-row tile per CU (in_proj qkv|z and q|gate|k|v
// at the 27B shapes; measured on MI355X at M = 64: 39.7 -> 33.8 us and
// 37.5 -> 32.9 us per call including the K-split finalize the other kernel
// needs, at M = 32 in_proj 25.3 -> 21.5 us).  gate|up (544
// tiles) keeps the LDS-staged kernel with stream-K: there a block takes
// parts of three tiles and refills the copy pipeline for each (84.8 us
// against 94.9).  HAI_MFMA_DMA=0 keeps the LDS-staged kernels everywhere.
bool use_dma(const MfmaArgs& a) {
    static const bool on = [] {
        const char* e = std::getenv("HAI_MFMA_DMA");
        return e == nullptr || e[0] != '0';
    }();
    const int64_t ntiles = (static_cast<int64_t>(a.N) + kBlockRows - 1) / kBlockRows;
    return on && a.wq != nullptr && a.K % kRtChunk == 0 && a.M > 16 && a.M <= 64 && a.N > 8192 && !a.keep &&
           ntiles <= device_cus();
}

bool use_rt(const MfmaArgs& a) {
    if (a.K % kRtChunk != 0 || a.M > 64) return false;
    const int mode = rt_mode();
    if (mode == 2) return true;  // measurement: every eligible shape
    return mode == 1 && a.wq != nullptr && a.M > 16 && a.N <= 8192;
}

template <int EPI>
int dispatch_mfma(const MfmaArgs& a, hipStream_t s) {
    if (use_dma(a)) {
        if (a.M <= 32) return launch_dma<2, EPI>(a, s);
        return launch_dma<4, EPI>(a, s);
    }
    if (use_rt(a)) {
        if (a.M <= 16) return launch_rt<1, EPI>(a, s);
        if (a.M <= 32) return launch_rt<2, EPI>(a, s);
        return launch_rt<4, EPI>(a, s);
    }
    if (a.M <= 16) return launch_mfma<1, EPI>(a, s);
    if (a.M <= 32) return launch_mfma<2, EPI>(a, s);
    if (a.M <= 64) return launch_mfma<4, EPI>(a, s);
    return launch_mfma<8, EPI>(a, s);
}

}  // namespace

extern "C" size_t hai_gemm_mfma_workspace_bytes(int64_t M, int64_t N) {
    // largest split the dispatcher picks for this shape (4 at N <= 8192, 2 at
    // N <= 20480), or the two stream-K planes of the wider layers that need
    // between one and two rounds of blocks (N up to 2 x 1024 tiles of 64)
    const int64_t ksb = N <= 8192 ? 4 : (N <= 20480 ? 2 : (N <= 131072 ? 2 : 1));
    return ksb > 1 ? static_cast<size_t>(ksb * M * N) * sizeof(float) : 0;
}

namespace {

// K split across blocks for narrow layers (measured on MI355X at M = 32:
// N = 5120 4 splits +115 %, N = 16384 2 splits +9 %), if the workspace holds
// the partials and every split gets at least two chunks.  For N <= 8192 the
// split count is the one that loads the busiest CU least (tiles x splits
// blocks on the CUs, ties to more splits): the time of these launches
// follows their busiest CU, so N = 5120 (80 tiles) takes 3 splits, 240
// blocks, rather than 4, whose 320 blocks double up on 64 CUs.
int device_cus() {
    static std::atomic<int> cached{0};  // one GPU model per process; retried until a device answers
    const int known = cached.load(std::memory_order_relaxed);
    if (known > 0) return known;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
        cached.store(cus, std::memory_order_relaxed);
        return cus;
    }
    return 256;  // MI355X
}

int choose_splits(int64_t M, int64_t N, int64_t K, const void* workspace, size_t workspace_bytes) {
    const int64_t nck = (K + kChunk - 1) / kChunk;
    auto fits = [&](int64_t ksb) {
        return nck >= 2 * ksb && workspace != nullptr &&
               workspace_bytes >= static_cast<size_t>(ksb * M * N) * sizeof(float);
    };
    if (N <= 8192) {
        const int64_t cus = device_cus();
        const int64_t ntiles = (N + kBlockRows - 1) / kBlockRows;
        int best = 1;
        double best_load = static_cast<double>((ntiles + cus - 1) / cus);
        for (int ksb = 2; ksb <= 4; ++ksb) {
            if (!fits(ksb) || ntiles * ksb > 2 * cus) continue;  // at most two blocks per CU
            const double load = static_cast<double>((ntiles * ksb + cus - 1) / cus) / ksb;
            if (load <= best_load) {
                best = ksb;
                best_load = load;
            }
        }
        return best;
    }
    int ksb = N <= 20480 ? 2 : 1;
    while (ksb > 1 && !fits(ksb)) ksb /= 2;
    return ksb;
}

int mfma_entry(MfmaArgs& a, int epilogue, void* workspace, size_t workspace_bytes, hipStream_t s) {
    {
        const int rc = check_gemm_extents(a.y, a.ldy, a.x, a.ldx, a.wq != nullptr ? static_cast<const void*>(a.wq)
                                                                                   : static_cast<const void*>(a.w),
                                          a.wq != nullptr ? 1 : 2, a.M, a.N, a.K, epilogue, a.res, a.ldres);
        if (rc != HAI_OK) return rc;
        if (workspace != nullptr && workspace_bytes > 0) {
            const int r2 = check_extent(workspace, workspace_bytes, "gemm_mfma workspace");
            if (r2 != HAI_OK) return r2;
        }
    }
    if (a.M == 0 || a.N == 0) return HAI_OK;
    a.keep = (epilogue & HAI_MFMA_KEEP_PARTIALS) != 0;
    epilogue &= ~HAI_MFMA_KEEP_PARTIALS;
    if (a.keep && epilogue != HAI_EPI_RESIDUAL) return invalid("gemm_mfma: keeping partials needs the residual epilogue");
    a.part = static_cast<float*>(workspace);
    a.ws_bytes = workspace != nullptr ? workspace_bytes : 0;
    a.KSB = choose_splits(a.M, a.N, a.K, workspace, workspace_bytes);
    switch (epilogue) {
        case HAI_EPI_STORE:
            if (a.ldy < a.N) return invalid("gemm_mfma: ldy < N");
            return dispatch_mfma<HAI_EPI_STORE>(a, s);
        case HAI_EPI_RESIDUAL:
            if (a.res == nullptr || a.ldy < a.N || a.ldres < a.N) return invalid("gemm_mfma: residual operands");
            return dispatch_mfma<HAI_EPI_RESIDUAL>(a, s);
        case HAI_EPI_SILU_MUL:
            if (a.N % 2 != 0 || a.ldy < a.N / 2) return invalid("gemm_mfma: silu_mul needs even N and ldy >= N/2");
            a.paired = a.wq != nullptr ? 1 : 0;
            return dispatch_mfma<HAI_EPI_SILU_MUL>(a, s);
        default:
            return invalid("gemm_mfma: unknown epilogue");
    }
}

int check_mfma(const void* y, const void* x, const void* w, int64_t M, int64_t N, int64_t K, int64_t ldx,
               int elem_bytes) {
    if (y == nullptr || x == nullptr || w == nullptr) return invalid("gemm_mfma: null pointer");
    if (M < 0 || M > kMaxMfmaRows || N < 0 || K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldx < K)
        return invalid("gemm_mfma: shape (need 0<=M<=128, K%8==0, ldx%8==0, ldx>=K)");
    if (N > INT32_MAX || K > INT32_MAX) return invalid("gemm_mfma: dimension too large");
    if ((N + kBlockRows) * K * elem_bytes >= (int64_t{1} << 32) || (kMaxMfmaRows + M) * ldx * 2 >= (int64_t{1} << 32))
        return invalid("gemm_mfma: W or X exceeds the 4 GiB buffer-offset range");
    if (!aligned16(x) || !aligned16(w)) return invalid("gemm_mfma: x and w must be 16-byte aligned");
    return HAI_OK;
}

}  // namespace

extern "C" int hai_gemm_mfma_splits(int64_t M, int64_t N, int64_t K, const void* workspace,
                                    size_t workspace_bytes) {
    if (M <= 0 || N <= 0 || K <= 0) return 1;
    return choose_splits(M, N, K, workspace, workspace_bytes);
}

extern "C" int hai_mfma_residual_rmsnorm_bf16(void* h, int64_t ldh, const void* workspace, size_t workspace_bytes,
                                              int64_t M, int64_t N, int64_t splits, const void* norm_w, float eps,
                                              int unit_offset, void* xn, int64_t ld_xn, void* stream) {
    if (h == nullptr || workspace == nullptr) return invalid("mfma_residual_rmsnorm: null pointer");
    if (M < 0 || M > kMaxMfmaRows || N <= 0 || N % 8 != 0 || N > kMaxResidualNormCols || ldh < N || ldh % 8 != 0 ||
        splits < 2 || splits > 4)
        return invalid("mfma_residual_rmsnorm: shape (need N % 8 == 0, N <= 8192, 2 <= splits <= 4; a GEMM that "
                       "takes one split finishes its rows itself and leaves no partials)");
    if (static_cast<size_t>(splits) * static_cast<size_t>(M) * static_cast<size_t>(N) * sizeof(float) >
        workspace_bytes)
        return invalid("mfma_residual_rmsnorm: workspace_bytes below splits * M * N * 4");
    {
        int rc = check_extent(workspace, static_cast<size_t>(splits * M * N) * sizeof(float), "residual_rmsnorm ws");
        if (rc == HAI_OK) rc = check_extent(h, rows_extent(M, N, ldh, 2), "residual_rmsnorm h");
        if (rc == HAI_OK && norm_w != nullptr) rc = check_extent(norm_w, static_cast<size_t>(N) * 2, "norm_w");
        if (rc == HAI_OK && norm_w != nullptr) rc = check_extent(xn, rows_extent(M, N, ld_xn, 2), "residual xn");
        if (rc != HAI_OK) return rc;
    }
    if (norm_w != nullptr && (xn == nullptr || ld_xn < N || ld_xn % 8 != 0 || !aligned16(norm_w) || !aligned16(xn)))
        return invalid("mfma_residual_rmsnorm: normalised output needs xn, ld_xn >= N, 16-byte alignment");
    if (!aligned16(h) || !aligned16(workspace)) return invalid("mfma_residual_rmsnorm: 16-byte alignment");
    if (M == 0) return HAI_OK;
    const dim3 grid(static_cast<unsigned>(M));
    auto* hh = static_cast<uint16_t*>(h);
    const auto* part = static_cast<const float*>(workspace);
    const auto* w = static_cast<const uint16_t*>(norm_w);
    auto* x = static_cast<uint16_t*>(xn);
    const float off = unit_offset ? 1.0f : 0.0f;
    const auto s = as_stream(stream);
    const int n = int(N), m = int(M), k = int(splits);
    if (N <= 2048)
        mfma_residual_rmsnorm_kernel<1><<<grid, dim3(256), 0, s>>>(hh, ldh, part, k, m, n, w, eps, off, x, ld_xn);
    else if (N <= 6144)
        mfma_residual_rmsnorm_kernel<3><<<grid, dim3(256), 0, s>>>(hh, ldh, part, k, m, n, w, eps, off, x, ld_xn);
    else
        mfma_residual_rmsnorm_kernel<4><<<grid, dim3(256), 0, s>>>(hh, ldh, part, k, m, n, w, eps, off, x, ld_xn);
    return launched("mfma_residual_rmsnorm_kernel");
}

extern "C" int hai_gemm_bf16_mfma(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t M,
                                  int64_t N, int64_t K, int epilogue, const void* res, int64_t ld_res,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    const int rc = check_mfma(y, x, w, M, N, K, ldx, 2);
    if (rc != HAI_OK) return rc;
    MfmaArgs a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx,
               static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(res), ld_res,
               int(M), int(N), int(K), nullptr, 1};
    return mfma_entry(a, epilogue, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int hai_gemm_fp8_mfma(void* y, int64_t ldy, const void* x, int64_t ldx, const void* wq,
                                 const float* scales, const int32_t* scale_rows, int64_t M, int64_t N, int64_t K,
                                 int epilogue, const void* res, int64_t ld_res, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    if (scales == nullptr) return invalid("gemm_fp8_mfma: null scales");
    const int rc = check_mfma(y, x, wq, M, N, K, ldx, 1);
    if (rc != HAI_OK) return rc;
    if (K % 16 != 0) return invalid("gemm_fp8_mfma: K % 16 != 0");
    MfmaArgs a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx, nullptr,
               static_cast<const uint16_t*>(res), ld_res, int(M), int(N), int(K), nullptr, 1};
    a.wq = static_cast<const uint8_t*>(wq);
    a.scales = scales;
    a.scale_rows = scale_rows;
    a.check = (epilogue & HAI_FP8_NO_SPECIAL_CODES) == 0;
    return mfma_entry(a, epilogue & ~HAI_FP8_NO_SPECIAL_CODES, workspace, workspace_bytes, as_stream(stream));
}

// ---------------------------------------------------------------------------
// Prefill-sized linear layers: Y[M, N] = X[M, K] . W[N, K]^T for M of
// hundreds to thousands of rows (prompt chunks of one or several sequences).
// The weight-streaming kernel above re-reads every weight once per 128 rows;
// here both operands are tiled and the layer is compute bound.
//   * block = 4 waves, output tile 128 rows of X x BN rows of W (BN = 128, or
//     64 when 128-wide tiles would leave CUs without one); wave (wm, wn) owns
//     64 x BN/2 outputs as 32 x 32 tiles of v_mfma_f32_32x32x16_bf16 (on
//     MI355X this form issues at twice the rate of the 16 x 16 x 32 one)
//     with fp32 accumulators;
//   * K in steps of 64: both operand tiles staged in LDS (two buffers, rows
//     padded by 16 bytes), a step's global loads requested two steps ahead
//     into registers, and the next step's pieces written to the other buffer
//     between the current step's k-slices of MFMAs; one barrier per step;
//   * FP8 weights: codes decoded exactly to bf16 as they are staged, each
//     128-k scale block summed on its own and scaled in fp32 (the arithmetic
//     of hai_gemm_fp8_mfma);
//   * workgroups are dispatched to the 8 XCDs in turn, so block b is given
//     tile base(b % 8) + b / 8: every XCD takes a contiguous range of the tile
//     order, which runs in groups of 4 row tiles with the weight panels
//     sweeping inside a group, so the blocks resident on one XCD share a few
//     row tiles and weight panels in its L2;
//   * the epilogues of the other GEMMs (store, residual add, SwiGLU over
//     interleaved gate / up rows).
// Tolerance mode, as the other matrix-core GEMMs.
// ---------------------------------------------------------------------------
namespace {

constexpr int kTileM = 128;
constexpr int kTileK = 64;
constexpr int kTileRow = kTileK + 8;  // padded LDS row, bf16 elements
constexpr int kXcds = 8;

struct TiledArgs {
    uint16_t* y;
    int64_t ldy;
    const uint16_t* x;
    int64_t ldx;
    const void* w;               // bf16 [N][K], or E4M3 codes [N][K]
    const float* scales;         // FP8: [rows][ceil(K/128)]
    const int32_t* scale_rows;   // FP8: per-row scale row, or null
    int paired;                  // FP8 SiLU-mul without a map: interleaved gate / up grids
    const uint16_t* res;
    int64_t ldres;
    int M, N, K;
    int mtiles, ntiles;
    int group_m;  // tile order: groups of group_m row tiles (0: panel by panel)
};

// WM / WN: 16-row MFMA tiles per wave along X rows / weight rows; block =
// 2 x 2 waves, output tile (32 WM) x (32 WN).
template <int WM, int WN, int NWV = 4>
__host__ __device__ constexpr size_t tiled_lds_bytes() {
    return static_cast<size_t>(2) * (16 * WM * (NWV / 2) + 32 * WN) * kTileRow * 2;
}

template <int WM, int WN, int EPI, bool FP8, bool CHECK, bool M32, int PIPE, int NWV>
__global__ __launch_bounds__(64 * NWV) void gemm_tiled_kernel(TiledArgs a) {
    constexpr int NT = 64 * NWV;
    constexpr int BM = 16 * WM * (NWV / 2);
    constexpr int BN = 32 * WN;
    constexpr int XP = BM * kTileK / 8 / NT;                 // 16-byte X pieces per thread
    constexpr int WP = FP8 ? BN * kTileK / 16 / NT : BN * kTileK / 8 / NT;  // W pieces per thread
    static_assert(XP >= 1 && WP >= 1, "tile must split over the block");
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* xs = lds;                      // [2][BM][kTileRow]
    uint16_t* ws = lds + 2 * BM * kTileRow;  // [2][BN][kTileRow]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_index();
    const int li = lane & 15;
    const int kg = lane >> 4;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    // XCD-aware tile of this block: each XCD takes a contiguous range of the
    // tile order; GM > 0 orders the tiles in groups of GM row tiles, the
    // weight panels sweeping inside a group (row tiles fastest), so the
    // blocks resident on an XCD cover about GM row tiles x (blocks / GM)
    // panels; GM = 0: all row tiles of a panel, then the next panel.
    const int nb = static_cast<int>(gridDim.x);
    const int bid = static_cast<int>(blockIdx.x);
    const int xcd = bid % kXcds;
    const int tile = xcd * (nb / kXcds) + min(xcd, nb % kXcds) + bid / kXcds;
    int tm, tn;
    if (a.group_m > 0) {
        const int per_group = a.group_m * a.ntiles;
        const int g = tile / per_group;
        const int first = g * a.group_m;
        const int gsize = min(a.mtiles - first, a.group_m);
        const int r = tile - g * per_group;
        tm = first + r % gsize;
        tn = r / gsize;
    } else {
        tm = tile % a.mtiles;
        tn = tile / a.mtiles;
    }
    const int64_t m0 = static_cast<int64_t>(tm) * BM;
    const int64_t n0 = static_cast<int64_t>(tn) * BN;
    const int M = a.M, N = a.N, K = a.K;

    // Operand buffers start at the tile; rows past M / N read as zeros.  The
    // host bounds M * ldx * 2 and N * K * elem below 4 GiB.
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(a.x + m0 * a.ldx, static_cast<uint32_t>((M - m0) * a.ldx * 2));
    const __amdgpu_buffer_rsrc_t rw =
        FP8 ? make_rsrc(static_cast<const uint8_t*>(a.w) + n0 * K, static_cast<uint32_t>((N - n0) * K))
            : make_rsrc(static_cast<const uint16_t*>(a.w) + n0 * K, static_cast<uint32_t>((N - n0) * K * 2));
    uint32_t xoff[XP], woff[WP];
    int xdst[XP], wdst[WP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int e = tid + NT * i;
        const int r = e >> 3, c = (e & 7) * 8;
        xoff[i] = static_cast<uint32_t>((r * a.ldx + c) * 2);
        xdst[i] = r * kTileRow + c;
    }
#pragma unroll
    for (int i = 0; i < WP; ++i) {
        const int e = tid + NT * i;
        if constexpr (FP8) {
            const int r = e >> 2, c = (e & 3) * 16;
            woff[i] = static_cast<uint32_t>(r * K + c);
            wdst[i] = r * kTileRow + c;
        } else {
            const int r = e >> 3, c = (e & 7) * 8;
            woff[i] = static_cast<uint32_t>((r * K + c) * 2);
            wdst[i] = r * kTileRow + c;
        }
    }
    // operand registers of one step, two sets: a step's loads are issued two
    // steps before they are multiplied (one before they are staged)
    auto load = [&](u32x4 (&xv)[XP], u32x4 (&wv)[WP], int step) {
        const uint32_t k0 = static_cast<uint32_t>(step) * kTileK;
#pragma unroll
        for (int i = 0; i < XP; ++i) xv[i] = bload(rx, xoff[i], k0 * 2);
#pragma unroll
        for (int i = 0; i < WP; ++i) wv[i] = bload(rw, woff[i], FP8 ? k0 : k0 * 2);
    };
    // one staged piece: X pieces 0 .. XP-1, then W pieces
    auto stage_piece = [&](const u32x4 (&xv)[XP], const u32x4 (&wv)[WP], int buf, int p) {
        uint16_t* xb = xs + buf * BM * kTileRow;
        uint16_t* wb = ws + buf * BN * kTileRow;
        if (p < XP) {
            *reinterpret_cast<u32x4*>(xb + xdst[p]) = xv[p];
            return;
        }
        const int i = p - XP;
        if constexpr (FP8) {
            uint32_t d[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) e4m3x4_to_bf16<CHECK>(wv[i][q], d[2 * q], d[2 * q + 1]);
            *reinterpret_cast<u32x4*>(wb + wdst[i]) = u32x4{d[0], d[1], d[2], d[3]};
            *reinterpret_cast<u32x4*>(wb + wdst[i] + 8) = u32x4{d[4], d[5], d[6], d[7]};
        } else {
            *reinterpret_cast<u32x4*>(wb + wdst[i]) = wv[i];
        }
    };
    auto stage = [&](const u32x4 (&xv)[XP], const u32x4 (&wv)[WP], int buf) {
        uint16_t* xb = xs + buf * BM * kTileRow;
        uint16_t* wb = ws + buf * BN * kTileRow;
#pragma unroll
        for (int i = 0; i < XP; ++i) *reinterpret_cast<u32x4*>(xb + xdst[i]) = xv[i];
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            if constexpr (FP8) {
                uint32_t d[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) e4m3x4_to_bf16<CHECK>(wv[i][q], d[2 * q], d[2 * q + 1]);
                *reinterpret_cast<u32x4*>(wb + wdst[i]) = u32x4{d[0], d[1], d[2], d[3]};
                *reinterpret_cast<u32x4*>(wb + wdst[i] + 8) = u32x4{d[4], d[5], d[6], d[7]};
            } else {
                *reinterpret_cast<u32x4*>(wb + wdst[i]) = wv[i];
            }
        }
    };

    // MFMA tiles per wave: 16 x 16 (WM x WN of them) or 32 x 32 (M32: half
    // as many each way); lane (li, kg) of a 16-tile, column lc of a 32-tile
    constexpr int TM = M32 ? WM / 2 : WM;
    constexpr int TN = M32 ? WN / 2 : WN;
    constexpr int TS = M32 ? 32 : 16;
    using Acc = typename std::conditional<M32, f32x16, f32x4>::type;
    constexpr int AE = M32 ? 16 : 4;  // accumulator elements per lane and tile
    const int lc = lane & 31;
    const int lh = lane >> 5;
    const int colx = M32 ? lc : li;   // the lane's column within a tile

    // FP8: the scale row of each of the lane's output columns
    const int nkb = (K + 127) / 128;
    const float* srow[TN];
    if constexpr (FP8) {
        const int64_t nsb = ((N >> 1) + 127) / 128;
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) {
            const int64_t n = min(n0 + wn * 16 * WN + ni * TS + colx, static_cast<int64_t>(N) - 1);
            const int64_t sr = a.scale_rows ? a.scale_rows[n] : (a.paired ? (n & 1) * nsb + (n >> 1) / 128 : n / 128);
            srow[ni] = a.scales + sr * nkb;
        }
    }

    Acc acc[TM][TN];   // the current 128-k scale block (FP8) or the whole sum (bf16)
    Acc tot[TM][TN];   // FP8: the scaled sum of the finished blocks
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
#pragma unroll
            for (int e = 0; e < AE; ++e) {
                acc[mi][ni][e] = 0.0f;
                tot[mi][ni][e] = 0.0f;
            }

    const int nsteps = K / kTileK;
    constexpr int NP = XP + WP;  // staged pieces per thread and step
    // PIPE 1: the next step's pieces (xn, wnx) are written to the other
    // buffer (nbuf) between the k-slices' MFMAs, not after all of them
    auto compute = [&](int step, const u32x4 (*xn)[XP], const u32x4 (*wnx)[WP], int nbuf) {
        const int buf = step & 1;
        const uint16_t* xb = xs + buf * BM * kTileRow;
        const uint16_t* wb = ws + buf * BN * kTileRow;
        if constexpr (M32) {
#pragma unroll
            for (int j = 0; j < kTileK / 16; ++j) {
                u32x4 af[TM], bf[TN];
#pragma unroll
                for (int mi = 0; mi < TM; ++mi)
                    af[mi] = *reinterpret_cast<const u32x4*>(xb + (wm * 16 * WM + mi * 32 + lc) * kTileRow + 16 * j +
                                                             8 * lh);
#pragma unroll
                for (int ni = 0; ni < TN; ++ni)
                    bf[ni] = *reinterpret_cast<const u32x4*>(wb + (wn * 16 * WN + ni * 32 + lc) * kTileRow + 16 * j +
                                                             8 * lh);
#pragma unroll
                for (int mi = 0; mi < TM; ++mi)
#pragma unroll
                    for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = mfma32(af[mi], bf[ni], acc[mi][ni]);
                if constexpr (PIPE == 1) {
                    constexpr int NS = kTileK / 16;
#pragma unroll
                    for (int p = j * NP / NS; p < (j + 1) * NP / NS; ++p) stage_piece(*xn, *wnx, nbuf, p);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < kTileK / 32; ++j) {
                u32x4 af[TM], bf[TN];
#pragma unroll
                for (int mi = 0; mi < TM; ++mi)
                    af[mi] = *reinterpret_cast<const u32x4*>(xb + (wm * 16 * WM + mi * 16 + li) * kTileRow + 32 * j +
                                                             8 * kg);
#pragma unroll
                for (int ni = 0; ni < TN; ++ni)
                    bf[ni] = *reinterpret_cast<const u32x4*>(wb + (wn * 16 * WN + ni * 16 + li) * kTileRow + 32 * j +
                                                             8 * kg);
#pragma unroll
                for (int mi = 0; mi < TM; ++mi)
#pragma unroll
                    for (int ni = 0; ni < TN; ++ni) acc[mi][ni] = mfma16(af[mi], bf[ni], acc[mi][ni]);
            }
        }
        if constexpr (FP8) {
            // a 128-k scale block ends every second step (and at the end of K)
            if ((step & 1) == 1 || step + 1 == nsteps) {
                const int kb = step >> 1;
#pragma unroll
                for (int ni = 0; ni < TN; ++ni) {
                    const float sc = srow[ni][kb];
#pragma unroll
                    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
                        for (int i = 0; i < AE; ++i) {
                            tot[mi][ni][i] = fma_(sc, acc[mi][ni][i], tot[mi][ni][i]);
                            acc[mi][ni][i] = 0.0f;
                        }
                }
            }
        }
    };
    // Step s: request step s + 2 into one register set, multiply step s from
    // LDS buffer s % 2, stage step s + 1 (requested a step earlier) into the
    // other buffer, LDS-only barrier (the requests stay in flight).  Loads
    // past the last step are clamped to it and never used, so the code
    // between waits is straight-line and the compiler's wait counts exact.
    auto clamps = [&](int st) { return min(st, nsteps - 1); };
    u32x4 xA[XP], wA[WP], xB[XP], wB[WP];
    load(xA, wA, 0);
    load(xB, wB, clamps(1));
    stage(xA, wA, 0);
    lds_barrier();
    auto step = [&](int st, u32x4 (&xl)[XP], u32x4 (&wl)[WP], const u32x4 (&xn)[XP], const u32x4 (&wn_)[WP]) {
        load(xl, wl, clamps(st + 2));
        pin_memory_order();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PIPE == 1 && M32) {
            compute(st, &xn, &wn_, (st + 1) & 1);
        } else {
            compute(st, nullptr, nullptr, 0);
            pin_memory_order();
            __builtin_amdgcn_sched_barrier(0);
            stage(xn, wn_, (st + 1) & 1);
        }
        lds_barrier();
    };
    int st = 0;
    for (; st + 2 <= nsteps; st += 2) {
        step(st, xA, wA, xB, wB);
        step(st + 1, xB, wB, xA, wA);
    }
    if (st < nsteps) step(st, xA, wA, xB, wB);

    // 16-tiles: lane (li, kg) holds rows 4 kg + i, column li; 32-tiles:
    // rows 8 (i / 4) + 4 lh + i % 4, column lc
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
#pragma unroll
            for (int i = 0; i < AE; ++i) {
                const int r = M32 ? 8 * (i >> 2) + 4 * lh + (i & 3) : 4 * kg + i;
                const int m = static_cast<int>(m0) + wm * 16 * WM + mi * TS + r;
                const int64_t n = n0 + wn * 16 * WN + ni * TS + colx;
                mfma_store<EPI>(a.y, a.ldy, a.res, a.ldres, FP8 ? tot[mi][ni][i] : acc[mi][ni][i], m, n, M, N, colx);
            }
}

// Row tiles per group of the tile order (HAI_TILED_GROUP, read once per
// process, overrides the default of 4 for measurements; 0 = panel by panel).
int tiled_group_m() {
    static const int v = [] {
        const char* e = std::getenv("HAI_TILED_GROUP");
        return e == nullptr ? 4 : std::atoi(e);
    }();
    return v;
}

template <int WM, int WN, int EPI, bool FP8, bool CHECK, bool M32 = false, int PIPE = 0, int NWV = 4>
int launch_tiled(TiledArgs a, hipStream_t s) {
    constexpr size_t shmem = tiled_lds_bytes<WM, WN, NWV>();
    constexpr int BM = 16 * WM * (NWV / 2);
    auto* kern = gemm_tiled_kernel<WM, WN, EPI, FP8, CHECK, M32, PIPE, NWV>;
    static std::atomic<uint8_t> allowed[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return invalid("gemm_tiled: device ordinal");
    if (!allowed[dev].load(std::memory_order_acquire)) {
        bool done = false;
        const int rc = allow_lds(reinterpret_cast<const void*>(kern), shmem, &done);
        if (rc != HAI_OK) return rc;
        allowed[dev].store(1, std::memory_order_release);
    }
    a.mtiles = static_cast<int>((a.M + BM - 1) / BM);
    a.ntiles = static_cast<int>((a.N + 32 * WN - 1) / (32 * WN));
    a.group_m = tiled_group_m();
    const int64_t blocks = static_cast<int64_t>(a.mtiles) * a.ntiles;
    kern<<<dim3(static_cast<unsigned>(blocks)), dim3(64 * NWV), shmem, s>>>(a);
    return launched("gemm_tiled_kernel");
}

// HAI_TILED (read once per process) forces a tile form for measurements:
// 1 = 128 x 64, 2 = 128 x 128 on 16 x 16 MFMAs, staged after the step's
// MFMAs (the earlier kernel); 9 = 128 x 128, 10 = 128 x 64 on 32 x 32 MFMAs,
// staged between them; 30 = 256 x 256 (bf16), 31 = 256 x 128 on 8-wave
// blocks.  0 / unset: the choice below.
int tiled_force() {
    static const int v = [] {
        const char* e = std::getenv("HAI_TILED");
        return e == nullptr ? 0 : std::atoi(e);
    }();
    return v;
}

// 8-wave forms (bf16, TFLOP/s at 1024 | 4096 rows; 128 x 128 in brackets):
// 256 x 256 in_proj 707 | 1028 (810 | 936), q|gate|k|v 1120 | 1116 (794 |
// 987), gate|up 778 | 1032 (816 | 932), out 416 | 769 (606 | 901); 256 x 128
// out 668 | 876, down 791 | 957 (710 | 960); FP8 256 x 128: in_proj 664 |
// 903 (649 | 814), q|gate|k|v 830 | 964 (688 | 847), gate|up 848 | 950
// (793 | 833), out 679 | 842 (565 | 830), down 746 | 911 (615 | 852).
// Measured on MI355X (bf16 / FP8 TFLOP/s, 27B prompt GEMMs at 1024 | 4096
// rows; the earlier 16 x 16 kernel in brackets): in_proj 824 | 951 (672 |
// 786), FP8 664 | 805 (394 | 454); gate|up 830 | 929 (737 | 802), FP8 780 |
// 836 (476 | 478); down 723 | 968 (576 | 784).  The 32 x 32 MFMA issues at
// about twice the rate of the 16 x 16 one, writing the next step's operands
// between the k-slices' MFMAs hides the stores, the FP8 form then fits two
// blocks per CU, and ordering the tiles in groups of 4 row tiles halves the
// bytes fetched beyond L2 (2.7 -> 1.2-1.4 GiB at 4096 x 16480 x 5120).
template <int EPI, bool FP8, bool CHECK>
int dispatch_tiled(TiledArgs a, hipStream_t s) {
    switch (tiled_force()) {
        case 1: return launch_tiled<4, 2, EPI, FP8, CHECK>(a, s);
        case 2: return launch_tiled<4, 4, EPI, FP8, CHECK>(a, s);
        case 10: return launch_tiled<4, 2, EPI, FP8, CHECK, true, 1>(a, s);
        case 30:
            if constexpr (!FP8) return launch_tiled<4, 8, EPI, FP8, CHECK, true, 1, 8>(a, s);
            break;
        case 31: return launch_tiled<4, 4, EPI, FP8, CHECK, true, 1, 8>(a, s);
        default: break;
    }
    // 128-wide weight tiles unless they leave CUs without a tile
    const int64_t mt = (static_cast<int64_t>(a.M) + kTileM - 1) / kTileM;
    const int64_t tiles128 = mt * ((a.N + 127) / 128);
    if constexpr (FP8) {
        // FP8: 256 x 128 on 8-wave blocks wherever 128 x 128 tiles fill the
        // CUs (every 27B shape measured faster, 256 x 256 needs twice the
        // accumulators: the per-scale-block sums are kept apart)
        if (tiled_force() == 0 && tiles128 >= device_cus()) return launch_tiled<4, 4, EPI, FP8, CHECK, true, 1, 8>(a, s);
    } else {
        // bf16: 8-wave blocks (2 waves per SIMD, one block per CU) with
        // 256-row tiles read LDS half as often per product as the 4-wave
        // 128 x 128 form; 256 x 256 where its tiles fill whole rounds of the
        // CUs to 80 % or more, 256 x 128 where they fit one round
        const int64_t cus = device_cus();
        const int64_t mt256 = (static_cast<int64_t>(a.M) + 255) / 256;
        const int64_t t256 = mt256 * ((a.N + 255) / 256);
        const int64_t rounds = (t256 + cus - 1) / cus;
        if (tiled_force() == 0 && tiles128 >= cus) {
            if (5 * t256 >= 4 * rounds * cus) return launch_tiled<4, 8, EPI, FP8, CHECK, true, 1, 8>(a, s);
            if (mt256 * ((a.N + 127) / 128) <= cus) return launch_tiled<4, 4, EPI, FP8, CHECK, true, 1, 8>(a, s);
        }
    }
    if (tiles128 >= 256 || tiled_force() == 9) return launch_tiled<4, 4, EPI, FP8, CHECK, true, 1>(a, s);
    return launch_tiled<4, 2, EPI, FP8, CHECK, true, 1>(a, s);
}

template <bool FP8, bool CHECK>
int tiled_entry(TiledArgs& a, int epilogue, hipStream_t s) {
    switch (epilogue) {
        case HAI_EPI_STORE:
            if (a.ldy < a.N) return invalid("gemm_tiled: ldy < N");
            return dispatch_tiled<HAI_EPI_STORE, FP8, CHECK>(a, s);
        case HAI_EPI_RESIDUAL:
            if (a.res == nullptr || a.ldy < a.N || a.ldres < a.N) return invalid("gemm_tiled: residual operands");
            return dispatch_tiled<HAI_EPI_RESIDUAL, FP8, CHECK>(a, s);
        case HAI_EPI_SILU_MUL:
            if (a.N % 2 != 0 || a.ldy < a.N / 2) return invalid("gemm_tiled: silu_mul needs even N and ldy >= N/2");
            a.paired = FP8 ? 1 : 0;
            return dispatch_tiled<HAI_EPI_SILU_MUL, FP8, CHECK>(a, s);
        default:
            return invalid("gemm_tiled: unknown epilogue");
    }
}

int check_tiled(const void* y, const void* x, const void* w, int64_t M, int64_t N, int64_t K, int64_t ldx,
                int elem_bytes) {
    if (y == nullptr || x == nullptr || w == nullptr) return invalid("gemm_tiled: null pointer");
    if (M < 0 || N < 0 || K <= 0 || K % kTileK != 0 || ldx % 8 != 0 || ldx < K)
        return invalid("gemm_tiled: shape (need K % 64 == 0, ldx % 8 == 0, ldx >= K)");
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return invalid("gemm_tiled: dimension too large");
    if (N * K * elem_bytes >= (int64_t{1} << 32) || M * ldx * 2 >= (int64_t{1} << 32))
        return invalid("gemm_tiled: W or X exceeds the 4 GiB buffer-offset range");
    if ((M + kTileM - 1) / kTileM * ((N + 63) / 64) >= (int64_t{1} << 31)) return invalid("gemm_tiled: grid too large");
    if (!aligned16(x) || !aligned16(w)) return invalid("gemm_tiled: x and w must be 16-byte aligned");
    return HAI_OK;
}

}  // namespace

extern "C" int hai_gemm_bf16_tiled(void* y, int64_t ldy, const void* x, int64_t ldx, const void* w, int64_t M,
                                   int64_t N, int64_t K, int epilogue, const void* res, int64_t ld_res,
                                   void* stream) {
    int rc = check_tiled(y, x, w, M, N, K, ldx, 2);
    if (rc == HAI_OK) rc = check_gemm_extents(y, ldy, x, ldx, w, 2, M, N, K, epilogue, res, ld_res);
    if (rc != HAI_OK) return rc;
    if (M == 0 || N == 0) return HAI_OK;
    TiledArgs a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx, w, nullptr, nullptr, 0,
                static_cast<const uint16_t*>(res), ld_res, int(M), int(N), int(K),
                static_cast<int>((M + kTileM - 1) / kTileM), 0, 0};
    return tiled_entry<false, false>(a, epilogue, as_stream(stream));
}

extern "C" int hai_gemm_fp8_tiled(void* y, int64_t ldy, const void* x, int64_t ldx, const void* wq,
                                  const float* scales, const int32_t* scale_rows, int64_t M, int64_t N, int64_t K,
                                  int epilogue, const void* res, int64_t ld_res, void* stream) {
    if (scales == nullptr) return invalid("gemm_fp8_tiled: null scales");
    int rc = check_tiled(y, x, wq, M, N, K, ldx, 1);
    const int epi = epilogue & ~HAI_FP8_NO_SPECIAL_CODES;
    if (rc == HAI_OK) rc = check_gemm_extents(y, ldy, x, ldx, wq, 1, M, N, K, epi, res, ld_res);
    if (rc != HAI_OK) return rc;
    if (M == 0 || N == 0) return HAI_OK;
    TiledArgs a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx, wq, scales, scale_rows, 0,
                static_cast<const uint16_t*>(res), ld_res, int(M), int(N), int(K),
                static_cast<int>((M + kTileM - 1) / kTileM), 0, 0};
    if ((epilogue & HAI_FP8_NO_SPECIAL_CODES) != 0) return tiled_entry<true, false>(a, epi, as_stream(stream));
    return tiled_entry<true, true>(a, epi, as_stream(stream));
}
