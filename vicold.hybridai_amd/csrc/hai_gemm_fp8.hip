// hai_gemm_fp8.hip -- skinny linear layer over FP8 E4M3 weights with 128x128
// fp32 block scales (QuantizedWeight with ScaleLayout::Block2D,
// qwen3_weights.cc:131-182; dequantization of fp8_dequant.cc:12-146 fused
// into the weight stream).
//
// Arithmetic: w = decode_e4m3(q) * s[n/128][k/128] in fp32 (the reference's
// dequantize_2d), then the same canonical segmented-L64 order as the bf16 GEMM, so
// the result equals the bf16 path run on the dequantized weights.
//   * Lane l of a wave owns weight bytes 512c + 8l .. +7 of every chunk c
//     (8-byte loads, the L64 element-to-lane map) and the matching 8 bf16
//     activations (16-byte loads).
//   * Decode: gfx950's packed E4M3 -> fp32 conversion (2 codes per
//     instruction) agrees with the reference's decode_e4m3 on every code
//     except 0x7F / 0xFF (NaN in OCP E4M3, +-480 in the reference); words
//     holding those codes take an exact bit-level decode.
//   * The scale row (ceil(K/128) floats) of each of a block's 8 weight rows
//     is staged in LDS once: row r reads scale row scale_rows[r] when the
//     caller passes that map (projections of several checkpoint tensors
//     concatenated, each with its own 128x128 grid), else r / 128; with
//     paired scales (fused SwiGLU over gate/up rows interleaved as
//     (gate_f, up_f)) row r reads plane r & 1, block (r >> 1) / 128 of a
//     [2][ceil(F/128)][ceil(K/128)] scale tensor.
#include "hai_gemm_common.h"

namespace {

using namespace hai;

constexpr int kMaxKBlocks = 256;  // K <= 32768

typedef float f2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, HAI_WLOAD_AUX));
}

// decode_e4m3 of fp8_dequant.cc:12-26, exact for every code.
__device__ __forceinline__ float e4m3_exact(uint32_t b) {
    const uint32_t t = b & 0x7fu;
    float v;
    if (t >= 8u) {
        v = __uint_as_float((t << 20) + 0x3c000000u);  // (1 + m/8) * 2^(e-7)
    } else {
        // m * 2^-9 = (1 + m/8) * 2^-6 - 2^-6, exact
        v = __uint_as_float((t << 20) + 0x3c800000u) - 0x1p-6f;
    }
    return (b & 0x80u) ? -v : v;
}

// Eight consecutive codes (two little-endian words) -> floats.  Without
// CHECK the caller guarantees that no code is 0x7F / 0xFF.
template <bool CHECK>
__device__ __forceinline__ void decode8(u32x2 w, float (&f)[8]) {
    const f2v a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[0]), false);
    const f2v b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[0]), true);
    const f2v c = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[1]), false);
    const f2v d = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[1]), true);
    f[0] = a.x; f[1] = a.y; f[2] = b.x; f[3] = b.y;
    f[4] = c.x; f[5] = c.y; f[6] = d.x; f[7] = d.y;
    if (!CHECK) return;
    // a byte whose low 7 bits are all ones (0x7F / 0xFF) decodes to NaN in
    // hardware; adding 1 to the low 7 bits carries into bit 7 only there
    // (never across bytes)
    const uint32_t z = ((w[0] & 0x7f7f7f7fu) + 0x01010101u) | ((w[1] & 0x7f7f7f7fu) + 0x01010101u);
    if (__builtin_expect((z & 0x80808080u) != 0u, 0)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = e4m3_exact((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
    }
}

// Scale rows of weight rows [rb, rb + nr) into srow[0 .. nr) (all 256 threads).
__device__ __forceinline__ void stage_scales(float (*srow)[kMaxKBlocks], int64_t rb, int nr, const float* scales,
                                             const int32_t* scale_rows, int paired, int N, int nkb) {
    const int64_t nsb = ((N >> 1) + 127) / 128;
    for (int i = threadIdx.x; i < nr * nkb; i += blockDim.x) {
        const int rl = i / nkb;
        const int kb = i - rl * nkb;
        const int64_t r = min(rb + rl, static_cast<int64_t>(N) - 1);
        const int64_t sr = scale_rows ? scale_rows[r] : (paired ? (r & 1) * nsb + (r >> 1) / 128 : r / 128);
        srow[rl][kb] = scales[sr * nkb + kb];
    }
}

// One 512-element chunk of RW rows x MB activations: the wave's lanes hold 8
// codes per row (wv) and 8 bf16 activations per row of x (xv).
template <int MB, int RW, bool CHECK>
__device__ __forceinline__ void fp8_chunk(float (&acc)[RW][MB], const u32x2 (&wv)[RW], const u32x4 (&xv)[MB],
                                          const float (&s)[RW]) {
    float xf[MB][8];
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xf[m][2 * q] = lo_bf(xv[m][q]);
            xf[m][2 * q + 1] = hi_bf(xv[m][q]);
        }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        float wf[8];
        decode8<CHECK>(wv[r], wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float we = wf[j] * s[r];
#pragma unroll
            for (int m = 0; m < MB; ++m) acc[r][m] = fma_(xf[m][j], we, acc[r][m]);
        }
    }
}

// Final bf16 stores of one row group (tot already reduced over the wave).
template <int MB, int RW, int EPI>
__device__ __forceinline__ void fp8_store(uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldres,
                                          const float (&tot)[RW][MB], int lane, int64_t row0, int nrows, int M) {
    if (EPI == HAI_EPI_SILU_MUL) {
#pragma unroll
        for (int p = 0; p < RW / 2; ++p)
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                if (lane == p * MB + m && m < M && 2 * p + 1 < nrows) {
                    const float g = bfr(tot[2 * p][m]);
                    const float u = bfr(tot[2 * p + 1][m]);
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
                    float v = bfr(tot[r][m]);
                    if (EPI == HAI_EPI_RESIDUAL) v = bf2f(res[static_cast<int64_t>(m) * ldres + n]) + v;
                    y[static_cast<int64_t>(m) * ldy + n] = f2bf(v);
                }
            }
    }
}

// One group = RW consecutive weight rows of one wave.  The plain launch runs
// one group per wave.  The NORM launch (RMSNorm prologue, activations read
// from LDS) has a grid sized to the machine so that the prologue is paid once
// per resident block; each wave then walks a contiguous run of groups.  A
// wave keeps its rows' scale rows in its own LDS rows and restages a row
// slot only when the scale row changes (every 128 rows of a tensor), so
// waves never wait for each other after the prologue.
template <int MB, int RW, int U, int EPI, bool CHECK, bool NORM>
__global__ __launch_bounds__(256) void gemm_fp8_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                       const uint16_t* __restrict__ x, int64_t ldx,
                                                       const uint8_t* __restrict__ wq,
                                                       const float* __restrict__ scales,
                                                       const int32_t* __restrict__ scale_rows, int paired,
                                                       const uint16_t* res, int64_t ldres, int M, int N, int K,
                                                       NormArgs na) {
    __shared__ float srow[4 * RW][kMaxKBlocks];
    extern __shared__ u32x4 xs[];  // NORM: [M][K/8] normalised rows, then the norm weight
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int nkb = (K + 127) / 128;
    const int npr = K >> 3;
    if constexpr (NORM) rmsnorm_rows_to_lds(xs, x, ldx, M, K, na);
    float (*wsrow)[kMaxKBlocks] = srow + wave * RW;
    const int64_t nsb = ((N >> 1) + 127) / 128;
    auto scale_row = [&](int64_t r) -> int64_t {
        return scale_rows ? scale_rows[r] : (paired ? (r & 1) * nsb + (r >> 1) / 128 : r / 128);
    };

    // Byte offsets fit 32 bits: the caller bounds N*K and M*ldx*2 below 4 GiB.
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq, static_cast<uint32_t>(static_cast<int64_t>(N) * K));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
    const int nck = (K + 511) / 512;
    const int nfull = K / 512;
    const int64_t nwg = (static_cast<int64_t>(N) + RW - 1) / RW;
    int64_t staged[RW];  // scale row held by each of the wave's LDS row slots
#pragma unroll
    for (int r = 0; r < RW; ++r) staged[r] = -1;

    auto group = [&](int64_t g) {
        const int64_t row0 = g * RW;
        const int nrows = static_cast<int>(min(static_cast<int64_t>(RW), static_cast<int64_t>(N) - row0));
        // (re)stage the slots whose scale row changed; LDS accesses of one wave
        // complete in order, so the previous group's reads are done
        bool restage = false;
        int64_t want[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            want[r] = scale_row(min(row0 + r, static_cast<int64_t>(N) - 1));
            restage |= want[r] != staged[r];
        }
        if (restage) {
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                if (want[r] == staged[r]) continue;
                for (int kb = lane; kb < nkb; kb += 64) wsrow[r][kb] = scales[want[r] * nkb + kb];
                staged[r] = want[r];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }

        uint32_t woff[RW], xoff[MB];
#pragma unroll
        for (int r = 0; r < RW; ++r) woff[r] = static_cast<uint32_t>((row0 + r) * static_cast<int64_t>(K) + lane * 8);
#pragma unroll
        for (int m = 0; m < MB; ++m) xoff[m] = static_cast<uint32_t>((static_cast<int64_t>(m) * ldx + lane * 8) * 2);

        // acc: the current 2048-element segment; tot: segments folded in order
        float acc[RW][MB], tot[RW][MB];
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < MB; ++m) acc[r][m] = tot[r][m] = 0.0f;
        auto fold = [&]() {
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    tot[r][m] = tot[r][m] + acc[r][m];
                    acc[r][m] = 0.0f;
                }
        };

        for (int c0 = 0; c0 < nck; c0 += U) {
            u32x2 wv[U][RW];
            u32x4 xv[U][MB];
            if (c0 + U <= nfull) {
                // every lane inside K: chunk offsets go in the scalar operand
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t c = static_cast<uint32_t>(c0 + u);
#pragma unroll
                    for (int r = 0; r < RW; ++r) wv[u][r] = bload8(rw, woff[r], c * 512u);
#pragma unroll
                    for (int m = 0; m < MB; ++m) {
                        if constexpr (NORM)
                            xv[u][m] = m < M ? xs[m * npr + c * 64 + lane] : u32x4{0u, 0u, 0u, 0u};
                        else
                            xv[u][m] = bload(rx, xoff[m], c * 1024u);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int c = c0 + u;
                    const bool ok = c < nfull || (c < nck && c * 512 + lane * 8 < K);
                    const ChunkOffset cw(c < nfull, ok, static_cast<uint32_t>(c) * 512u);
                    const ChunkOffset cx(c < nfull, ok, static_cast<uint32_t>(c) * 1024u);
#pragma unroll
                    for (int r = 0; r < RW; ++r) wv[u][r] = bload8(rw, cw.v(woff[r]), cw.s);
#pragma unroll
                    for (int m = 0; m < MB; ++m) {
                        if constexpr (NORM)
                            xv[u][m] = (ok && m < M) ? xs[m * npr + c * 64 + lane] : u32x4{0u, 0u, 0u, 0u};
                        else
                            xv[u][m] = bload(rx, cx.v(xoff[m]), cx.s);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // scale of k-block 4c + lane/16, clamped to a staged (finite)
                // scale: lanes past K hold zero codes and zero activations,
                // and fma(0, 0 * s, acc) == acc
                const int kb = min(4 * (c0 + u) + (lane >> 4), nkb - 1);
                float sv[RW];
#pragma unroll
                for (int r = 0; r < RW; ++r) sv[r] = wsrow[r][kb];
                fp8_chunk<MB, RW, CHECK>(acc, wv[u], xv[u], sv);
            }
            // a segment is four 512-element chunks (U divides 4)
            if (((c0 + U) & 3) == 0) fold();
        }
        fold();

#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < MB; ++m) tot[r][m] = wave_sum64(tot[r][m]);
        fp8_store<MB, RW, EPI>(y, ldy, res, ldres, tot, lane, row0, nrows, M);
    };

    const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if constexpr (NORM) {
        const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
        const int64_t per = (nwg + waves - 1) / waves;
        const int64_t g1 = min(nwg, (w + 1) * per);
        for (int64_t g = w * per; g < g1; ++g) group(g);
    } else {
        if (w < nwg) group(w);
    }
}

// K-split form: W waves share each row group, wave `sub` taking the
// 2048-element segments sub, sub + W, ...; the segment partials meet in LDS
// and the group's first wave folds them in segment order, which keeps the
// canonical sum (tot = tot + segment, then the 64-lane butterfly).
template <int MB, int RW, int W, int EPI, bool CHECK>
__global__ __launch_bounds__(256) void gemm_fp8_ksplit_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                              const uint16_t* __restrict__ x, int64_t ldx,
                                                              const uint8_t* __restrict__ wq,
                                                              const float* __restrict__ scales,
                                                              const int32_t* __restrict__ scale_rows, int paired,
                                                              const uint16_t* res, int64_t ldres, int M, int N,
                                                              int K) {
    constexpr int G = 4 / W;   // row groups per block
    constexpr int BR = G * RW;  // weight rows per block
    __shared__ float srow[BR][kMaxKBlocks];
    extern __shared__ float part[];  // [G][nseg][RW][MB][64]
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int g = wave / W;
    const int sub = wave % W;
    const int nkb = (K + 127) / 128;
    const int nck = (K + 511) / 512;
    const int nfull = K / 512;
    const int nseg = (nck + 3) / 4;
    stage_scales(srow, static_cast<int64_t>(blockIdx.x) * BR, BR, scales, scale_rows, paired, N, nkb);
    __syncthreads();
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * G + g) * RW;
    const bool active = row0 < N;
    const int nrows = active ? static_cast<int>(min(static_cast<int64_t>(RW), static_cast<int64_t>(N) - row0)) : 0;
    float* gpart = part + static_cast<int64_t>(g) * nseg * RW * MB * 64;

    if (active) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq, static_cast<uint32_t>(static_cast<int64_t>(N) * K));
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(static_cast<int64_t>(M) * ldx * 2));
        uint32_t woff[RW], xoff[MB];
#pragma unroll
        for (int r = 0; r < RW; ++r) woff[r] = static_cast<uint32_t>((row0 + r) * static_cast<int64_t>(K) + lane * 8);
#pragma unroll
        for (int m = 0; m < MB; ++m) xoff[m] = static_cast<uint32_t>((static_cast<int64_t>(m) * ldx + lane * 8) * 2);
        for (int sg = sub; sg < nseg; sg += W) {
            u32x2 wv[4][RW];
            u32x4 xv[4][MB];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = 4 * sg + u;
                const bool ok = c < nfull || (c < nck && c * 512 + lane * 8 < K);
                const ChunkOffset cw(c < nfull, ok, static_cast<uint32_t>(c) * 512u);
                const ChunkOffset cx(c < nfull, ok, static_cast<uint32_t>(c) * 1024u);
#pragma unroll
                for (int r = 0; r < RW; ++r) wv[u][r] = bload8(rw, cw.v(woff[r]), cw.s);
#pragma unroll
                for (int m = 0; m < MB; ++m) xv[u][m] = bload(rx, cx.v(xoff[m]), cx.s);
            }
            float acc[RW][MB];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int m = 0; m < MB; ++m) acc[r][m] = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int kb = min(4 * (4 * sg + u) + (lane >> 4), nkb - 1);
                float sv[RW];
#pragma unroll
                for (int r = 0; r < RW; ++r) sv[r] = srow[g * RW + r][kb];
                fp8_chunk<MB, RW, CHECK>(acc, wv[u], xv[u], sv);
            }
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int m = 0; m < MB; ++m) gpart[((static_cast<int64_t>(sg) * RW + r) * MB + m) * 64 + lane] = acc[r][m];
        }
    }
    __syncthreads();
    if (!active || sub != 0) return;
    float tot[RW][MB];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            float t = 0.0f;
            for (int sg = 0; sg < nseg; ++sg) t = t + gpart[((static_cast<int64_t>(sg) * RW + r) * MB + m) * 64 + lane];
            tot[r][m] = wave_sum64(t);
        }
    fp8_store<MB, RW, EPI>(y, ldy, res, ldres, tot, lane, row0, nrows, M);
}

struct Fp8Args {
    uint16_t* y;
    int64_t ldy;
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* wq;
    const float* scales;
    const int32_t* scale_rows;
    int paired;
    const uint16_t* res;
    int64_t ldres;
    int M, N, K;
    NormArgs na;
};

template <int MB, int RW, int EPI, bool CHECK, bool NORM>
void launch_fp8(const Fp8Args& a, hipStream_t s) {
    // two 512-element chunk groups in flight measured best on MI355X
    constexpr int U = MB <= 2 ? 2 : 1;
    auto* kern = gemm_fp8_kernel<MB, RW, U, EPI, CHECK, NORM>;
    int64_t blocks = (static_cast<int64_t>(a.N) + 4 * RW - 1) / (4 * RW);
    // NORM: LDS holds the M rows and the norm weight staged behind them.
    const size_t shmem = NORM ? static_cast<size_t>(a.M + 1) * a.K * 2 : 0;
    if (NORM) {
        const int64_t resident = resident_blocks(reinterpret_cast<const void*>(kern), shmem);
        if (resident > 0 && resident < blocks) blocks = resident;
    }
    kern<<<dim3(static_cast<unsigned>(blocks)), dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, a.wq, a.scales,
                                                                     a.scale_rows, a.paired, a.res, a.ldres, a.M,
                                                                     a.N, a.K, a.na);
}

constexpr int kKsplitRW = 2, kKsplitW = 4;

template <int MB, int EPI, bool CHECK>
void launch_fp8_ksplit(const Fp8Args& a, hipStream_t s) {
    constexpr int G = 4 / kKsplitW;
    const int64_t blocks = (static_cast<int64_t>(a.N) + G * kKsplitRW - 1) / (G * kKsplitRW);
    const int64_t nseg = ((a.K + 511) / 512 + 3) / 4;
    const size_t shmem = static_cast<size_t>(G * nseg * kKsplitRW * MB * 64) * sizeof(float);
    gemm_fp8_ksplit_kernel<MB, kKsplitRW, kKsplitW, EPI, CHECK>
        <<<dim3(static_cast<unsigned>(blocks)), dim3(256), shmem, s>>>(a.y, a.ldy, a.x, a.ldx, a.wq, a.scales,
                                                                       a.scale_rows, a.paired, a.res, a.ldres, a.M,
                                                                       a.N, a.K);
}

// Short, wide-K layers (M <= 2, N <= 8192) spread each row pair over four
// waves; LDS holds the segment partials (<= 64 KB).
bool use_ksplit_fp8(const Fp8Args& a) {
    if (a.M > 2 || a.N > 8192) return false;
    const int64_t nseg = ((a.K + 511) / 512 + 3) / 4;
    return nseg * kKsplitRW * a.M * 64 * 4 <= 64 * 1024;
}

template <int EPI, bool CHECK, bool NORM>
void dispatch_fp8(const Fp8Args& a, hipStream_t s) {
    if (!NORM && use_ksplit_fp8(a)) {
        if (a.M <= 1) launch_fp8_ksplit<1, EPI, CHECK>(a, s);
        else launch_fp8_ksplit<2, EPI, CHECK>(a, s);
        return;
    }
    // Two rows per wave; at M = 2 on wide layers, four rows per wave share
    // each activation load and conversion (+10-12 % at N >= 16384, fewer
    // waves hurt narrower layers).
    if (a.M <= 1) launch_fp8<1, 2, EPI, CHECK, NORM>(a, s);
    else if (a.M <= 2 && a.N >= 16384) launch_fp8<2, 4, EPI, CHECK, NORM>(a, s);
    else if (a.M <= 2) launch_fp8<2, 2, EPI, CHECK, NORM>(a, s);
    else if (a.M <= 4) launch_fp8<4, 2, EPI, CHECK, NORM>(a, s);
    else if (a.M <= 8) launch_fp8<8, 2, EPI, CHECK, NORM>(a, s);
    else launch_fp8<16, 2, EPI, CHECK, NORM>(a, s);
}

template <int EPI, bool NORM>
void dispatch_fp8_codes(const Fp8Args& a, bool check, hipStream_t s) {
    if (check) dispatch_fp8<EPI, true, NORM>(a, s);
    else dispatch_fp8<EPI, false, NORM>(a, s);
}

// E4M3 code of v, rounded to nearest even, saturated at +-448; NaN -> 0.
__device__ __forceinline__ uint32_t e4m3_encode(float v) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t sign = (b >> 24) & 0x80u;
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return 0u;
    if (a >= 0x43e00000u) return sign | 0x7eu;  // |v| >= 448
    if (a < 0x3c800000u) {
        // below 2^-6: multiples of 2^-9 (a * 512 is exact); 8 is code 0x08 = 2^-6
        return sign | static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 512.0f));
    }
    // normal: biased exponent 1..15, three mantissa bits; a carry out of the
    // mantissa moves to the next binade
    const uint32_t m = a & 0x7fffffu;
    uint32_t code = ((((a >> 23) - 127u + 7u)) << 3) | (m >> 20);
    const uint32_t rem = m & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (code & 1u))) ++code;
    return sign | min(code, 0x7eu);
}

__global__ void fp8_quantize_kernel(uint8_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ w,
                                    int64_t ldw, const float* __restrict__ scales, int64_t rows, int64_t cols) {
    const int64_t nkb = (cols + 127) / 128;
    const int64_t n = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = i / cols;
        const int64_t c = i - r * cols;
        const float s = scales[(r / 128) * nkb + c / 128];
        q[r * ldq + c] = static_cast<uint8_t>(e4m3_encode(bf2f(w[r * ldw + c]) / s));
    }
}

}  // namespace

extern "C" int hai_fp8_quantize_bf16(void* q, int64_t ldq, const void* w, int64_t ldw, const float* scales,
                                     int64_t rows, int64_t cols, void* stream) {
    if (q == nullptr || w == nullptr || scales == nullptr) return invalid("fp8_quantize: null pointer");
    if (rows < 0 || cols < 0 || ldq < cols || ldw < cols) return invalid("fp8_quantize: shape");
    if (rows == 0 || cols == 0) return HAI_OK;
    const int64_t blocks = std::min<int64_t>((rows * cols + 255) / 256, 65536);
    fp8_quantize_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint8_t*>(q), ldq, static_cast<const uint16_t*>(w), ldw, scales, rows, cols);
    return launched("fp8_quantize_kernel");
}

namespace {

int check_fp8(const void* y, const void* x, const void* wq, const float* scales, int64_t M, int64_t N, int64_t K,
              int64_t ldx) {
    if (y == nullptr || x == nullptr || wq == nullptr || scales == nullptr)
        return invalid("gemm_fp8: null pointer");
    if (M < 0 || M > 16 || N < 0 || K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldx < K)
        return invalid("gemm_fp8: shape (need 0<=M<=16, K%8==0, ldx%8==0, ldx>=K)");
    if ((K + 127) / 128 > kMaxKBlocks) return invalid("gemm_fp8: K above 32768");
    if ((N + 16) * K >= (int64_t{1} << 32) || M * ldx * 2 >= (int64_t{1} << 32))
        return invalid("gemm_fp8: W or X exceeds the 4 GiB buffer-offset range");
    if (!aligned16(x) || reinterpret_cast<uintptr_t>(wq) % 8 != 0)
        return invalid("gemm_fp8: x must be 16-byte and wq 8-byte aligned");
    return HAI_OK;
}

template <bool NORM>
int dispatch_fp8_epi(Fp8Args& a, int epilogue, hipStream_t s) {
    const bool check = (epilogue & HAI_FP8_NO_SPECIAL_CODES) == 0;
    switch (epilogue & ~HAI_FP8_NO_SPECIAL_CODES) {
        case HAI_EPI_STORE:
            if (a.ldy < a.N) return invalid("gemm_fp8: ldy < N");
            dispatch_fp8_codes<HAI_EPI_STORE, NORM>(a, check, s);
            break;
        case HAI_EPI_RESIDUAL:
            if (a.res == nullptr || a.ldy < a.N || a.ldres < a.N) return invalid("gemm_fp8: residual operands");
            dispatch_fp8_codes<HAI_EPI_RESIDUAL, NORM>(a, check, s);
            break;
        case HAI_EPI_SILU_MUL:
            if (a.N % 2 != 0 || a.ldy < a.N / 2) return invalid("gemm_fp8: silu_mul needs even N and ldy >= N/2");
            a.paired = 1;
            dispatch_fp8_codes<HAI_EPI_SILU_MUL, NORM>(a, check, s);
            break;
        default:
            return invalid("gemm_fp8: unknown epilogue");
    }
    return launched("gemm_fp8_kernel");
}

}  // namespace

extern "C" int hai_gemm_fp8_bf16(void* y, int64_t ldy, const void* x, int64_t ldx, const void* wq,
                                 const float* scales, const int32_t* scale_rows, int64_t M, int64_t N,
                                 int64_t K, int epilogue, const void* res, int64_t ld_res, void* stream) {
    int rc = check_fp8(y, x, wq, scales, M, N, K, ldx);
    if (rc == HAI_OK) rc = check_gemm_extents(y, ldy, x, ldx, wq, 1, M, N, K, epilogue, res, ld_res);
    if (rc != HAI_OK) return rc;
    if (M == 0 || N == 0) return HAI_OK;
    Fp8Args a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx,
              static_cast<const uint8_t*>(wq), scales, scale_rows, 0, static_cast<const uint16_t*>(res), ld_res,
              int(M), int(N), int(K), NormArgs{}};
    return dispatch_fp8_epi<false>(a, epilogue, as_stream(stream));
}

extern "C" int hai_gemm_rmsnorm_fp8_bf16(void* y, int64_t ldy, const void* x, int64_t ldx, const void* norm_w,
                                         float eps, int unit_offset, void* xn_out, int64_t ld_xn, const void* wq,
                                         const float* scales, const int32_t* scale_rows, int64_t M, int64_t N,
                                         int64_t K, int epilogue, const void* res, int64_t ld_res, void* stream) {
    int rc = check_fp8(y, x, wq, scales, M, N, K, ldx);
    if (rc == HAI_OK) rc = check_gemm_extents(y, ldy, x, ldx, wq, 1, M, N, K, epilogue, res, ld_res);
    if (rc == HAI_OK) rc = check_extent(norm_w, static_cast<size_t>(K) * 2, "gemm_rmsnorm_fp8 norm_w");
    if (rc == HAI_OK && xn_out != nullptr)
        rc = check_extent(xn_out, rows_extent(M, K, ld_xn, 2), "gemm_rmsnorm_fp8 xn");
    if (rc != HAI_OK) return rc;
    if (norm_w == nullptr) return invalid("gemm_rmsnorm_fp8: null norm weight");
    if (xn_out != nullptr && (ld_xn < K || ld_xn % 8 != 0 || !aligned16(xn_out)))
        return invalid("gemm_rmsnorm_fp8: xn_out needs ld_xn >= K, ld_xn % 8 == 0 and 16-byte alignment");
    if (!aligned16(norm_w)) return invalid("gemm_rmsnorm_fp8: norm weight must be 16-byte aligned");
    if (M == 0) return HAI_OK;
    if (M * K > kNormMaxElems) {
        // Rows too large for the LDS prologue: normalise into xn_out, then multiply.
        if (xn_out == nullptr) return invalid("gemm_rmsnorm_fp8: M*K above the fused limit needs xn_out");
        const int r = hai_rmsnorm_bf16(xn_out, ld_xn, x, ldx, norm_w, M, K, eps, unit_offset, stream);
        if (r != HAI_OK) return r;
        return hai_gemm_fp8_bf16(y, ldy, xn_out, ld_xn, wq, scales, scale_rows, M, N, K, epilogue, res, ld_res,
                                 stream);
    }
    if (N == 0)
        return xn_out != nullptr ? hai_rmsnorm_bf16(xn_out, ld_xn, x, ldx, norm_w, M, K, eps, unit_offset, stream)
                                 : HAI_OK;
    NormArgs na;
    na.w = static_cast<const uint16_t*>(norm_w);
    na.eps = eps;
    na.off = unit_offset ? 1.0f : 0.0f;
    na.xn = static_cast<uint16_t*>(xn_out);
    na.ldxn = ld_xn;
    Fp8Args a{static_cast<uint16_t*>(y), ldy, static_cast<const uint16_t*>(x), ldx,
              static_cast<const uint8_t*>(wq), scales, scale_rows, 0, static_cast<const uint16_t*>(res), ld_res,
              int(M), int(N), int(K), na};
    return dispatch_fp8_epi<true>(a, epilogue, as_stream(stream));
}
