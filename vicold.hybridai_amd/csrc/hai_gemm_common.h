// hai_gemm_common.h -- pieces shared by the skinny bf16 and FP8 GEMMs: the
// RMSNorm prologue that stages normalised activation rows in LDS, and the
// resident-block query that sizes persistent grids.
#pragma once

#include "hai_common.h"
#include "hai_device.h"

namespace hai {

// RMSNorm prologue arguments: y_k = bf16((x_k * inv) * (w_k + off)), exactly
// as rmsnorm_kernel.  Needs M * K <= kNormMaxElems (LDS holds the rows and
// the norm weight).
struct NormArgs {
    const uint16_t* w = nullptr;  // norm weight [K]
    float eps = 0.0f;
    float off = 0.0f;             // 1 for the (w + 1) model norms
    uint16_t* xn = nullptr;       // optional copy of the normalised rows (block 0 writes it)
    int64_t ldxn = 0;
};

constexpr int kNormMaxElems = HAI_GEMM_RMSNORM_FUSED_MAX;  // M * K: 32 KB of LDS

// A compiler-only memory fence (no instruction): loads are neither hoisted
// above nor sunk below it.  It brackets the weight requests that a wait for
// the global -> LDS copies counts (s_waitcnt vmcnt(n) with n those requests):
// without it the compiler may sink a request whose value is used only on a
// conditional path below the wait, and the wait then no longer covers every
// copy (seen on gfx950: 6 of 8 requests left above the wait).  The weight
// pointer of such a kernel must not be __restrict__: loads through a
// restrict-qualified read-only argument count as invariant, and the fence
// does not hold them.
__device__ __forceinline__ void pin_memory_order() { asm volatile("" ::: "memory"); }

// Block barrier for LDS data with global loads left in flight: this wave's
// LDS accesses complete (lgkmcnt(0)) and stay on their side of the barrier
// (compiler fence), vmcnt is not waited for.  __syncthreads() carries a
// workgroup release fence, which the compiler lowers to s_waitcnt vmcnt(0)
// once the kernel has issued global -> LDS copies (it cannot tell them from
// the weight requests behind them), so every block would wait for its
// prefetched weight chunks there (measured on MI355X: 3.6 - 7.5 us of a
// fused-norm launch's prologue).  Only for LDS data written by ds
// instructions or by copies already retired.
__device__ __forceinline__ void lds_barrier() {
    pin_memory_order();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt(63) and expcnt(7): no wait
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pin_memory_order();
}

// The normalisation step of the prologue: the M raw rows are staged in xs
// as 16-byte pieces [M][K/8] with the norm weight behind them (visible to
// the whole block), one wave per row reduces the sum of squares in L64
// order, then every element is scaled in place; ends with a block barrier
// (lds_barrier: weight requests issued before stay in flight).
__device__ __forceinline__ void normalize_staged_rows(u32x4* xs, int M, int K, const NormArgs& na) {
    __shared__ float inv_sh[16];
    const int lane = threadIdx.x & 63;
    const int wave = wave_index();
    const int npr = K >> 3;  // 16-byte pieces per row
    const int total = M * npr;
    for (int r = wave; r < M; r += 4) {
        float acc = 0.0f;
        for (int p = lane; p < npr; p += 64) {
            const u32x4 d = xs[r * npr + p];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a = lo_bf(d[q]);
                const float b = hi_bf(d[q]);
                acc = fma_(a, a, acc);
                acc = fma_(b, b, acc);
            }
        }
        const float ss = wave_sum64(acc);
        if (lane == 0) inv_sh[r] = 1.0f / csqrt(ss / static_cast<float>(K) + na.eps);
    }
    lds_barrier();
    for (int e = threadIdx.x; e < total; e += 256) {
        const int r = e / npr;
        const int p = e - r * npr;
        const float inv = inv_sh[r];
        const u32x4 xv0 = xs[e];
        const u32x4 wv0 = xs[total + p];
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = f2bf2((lo_bf(xv0[q]) * inv) * (lo_bf(wv0[q]) + na.off),
                         (hi_bf(xv0[q]) * inv) * (hi_bf(wv0[q]) + na.off));
        xs[e] = o;
        if (na.xn != nullptr && blockIdx.x == 0) *reinterpret_cast<u32x4*>(na.xn + r * na.ldxn + p * 8) = o;
    }
    lds_barrier();
}

// Stages the M activation rows [M, K] (row pitch ldx) in xs as 16-byte
// pieces, normalised: the raw rows and the norm weight are fetched together
// (one latency), then normalize_staged_rows.  xs holds (M + 1) * K / 8
// pieces; a 256-thread block; ends with a block barrier.
__device__ __forceinline__ void rmsnorm_rows_to_lds(u32x4* xs, const uint16_t* __restrict__ x, int64_t ldx,
                                                    int M, int K, const NormArgs& na) {
    const int npr = K >> 3;  // 16-byte pieces per row
    const int total = M * npr;
    for (int e0 = 0; e0 < total; e0 += 1024) {
        u32x4 xr[4], wr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = e0 + threadIdx.x + 256 * i;
            const int r = e / npr;
            const int p = e - r * npr;
            if (e < total) xr[i] = *reinterpret_cast<const u32x4*>(x + r * ldx + p * 8);
            if (e < npr) wr[i] = *reinterpret_cast<const u32x4*>(na.w + p * 8);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = e0 + threadIdx.x + 256 * i;
            if (e < total) xs[e] = xr[i];
            if (e < npr) xs[total + e] = wr[i];  // norm weight staged once, behind the rows
        }
    }
    __syncthreads();
    normalize_staged_rows(xs, M, K, na);
}

// The same staging done by the memory system: every piece of the raw rows
// and of the norm weight is copied global -> LDS by global_load_lds (16 bytes
// per lane, no registers), so that the caller can request its first weight
// chunks behind these copies and wait for the copies alone: loads complete
// in order, so s_waitcnt vmcnt(n), with n the loads issued after the copies,
// leaves those weight chunks in flight while the prologue computes.  Issues
// kStageOps copy instructions per wave (lanes past the data masked off).
// Needs (M + 1) * K / 8 <= 256 * kStageOps pieces, 16-byte aligned rows.
// Without a norm weight (norm_w null: rows already normalised) only the M
// rows are staged.
constexpr int kStageOps = 12;  // (M + 1) * K <= 24576: M * K <= HAI_GEMM_RMSNORM_FUSED_MAX, K <= 8192
__device__ __forceinline__ void stage_rows_lds_dma(u32x4* xs, const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                   int K, const uint16_t* __restrict__ norm_w) {
    const int wave = wave_index();
    const int npr = K >> 3;
    const int total = M * npr;
    const int pieces = total + (norm_w != nullptr ? npr : 0);
#pragma unroll
    for (int i = 0; i < kStageOps; ++i) {
        const int e = static_cast<int>(threadIdx.x) + 256 * i;
        if (e < pieces) {
            const int r = e / npr;
            const uint16_t* src = e < total ? x + r * ldx + (e - r * npr) * 8 : norm_w + (e - total) * 8;
            // (a C-style cast: the generic -> LDS address-space conversion)
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(xs + wave * 64 + 256 * i),
                                             16, 0, 0);
        }
    }
}

// s_waitcnt with vmcnt(n) and the other counters left alone (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Blocks of 256 threads of `kernel` with `shmem` bytes of dynamic LDS that
// the current device holds at once (occupancy x CUs); 0 if unknown.  Cached
// per (device, kernel, shmem).
int64_t resident_blocks(const void* kernel, size_t shmem);

}  // namespace hai
