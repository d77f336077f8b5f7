// hai_device.h -- device-side numerics shared by every gfx950 kernel.
//
// The verify path must produce the same token ids as a CPU restatement, so
// each rounding point is fixed:
//   * bf16 stores round to nearest even; NaN stays a quiet NaN.
//   * exp / log1p are computed by the canonical algorithms below (fma-based,
//     no hardware transcendental instructions, no libdevice).
//   * division and sqrt are IEEE correctly rounded (the build passes
//     -fhip-fp32-correctly-rounded-divide-sqrt; __fsqrt_rn is avoided because
//     it maps to the native approximation on this toolchain).
//   * a row reduction is the "L64 order": element k belongs to lane
//     (k/8)%64, each lane accumulates its elements in increasing k with fma,
//     then the 64 partials are combined by the xor butterfly 32,16,8,4,2,1.
// Everything is built with -ffp-contract=off so that a*b+c written without
// fma stays two roundings.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hai {

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// f32 -> bf16 by gfx950's v_cvt_pk_bf16_f32: round to nearest even, a NaN
// kept with its sign and upper payload and made quiet ((u >> 16) | 0x40),
// denormals kept -- the same bits as the integer form
//   (u & 0x7fffffff) > 0x7f800000 ? (u >> 16) | 0x40 : (u + 0x7fff + ((u >> 16) & 1)) >> 16
// on every input checked on MI355X (all NaN classes, ties, denormals, 2^20
// random patterns), in one instruction for two values instead of six each.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
// two values rounded and packed: lo in bits 0-15, hi in bits 16-31
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ float bfr(float f) { return bf2f(f2bf(f)); }

// Two bf16 packed in a dword: element 0 in the low half.
__device__ __forceinline__ float lo_bf(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float hi_bf(uint32_t d) { return __uint_as_float(d & 0xffff0000u); }

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

__device__ __forceinline__ float pow2i(int e) {  // e in [-126, 127]
    return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}

// Canonical exp: Cody-Waite reduction with ln2 = hi + lo, degree-8 Taylor
// polynomial in Horner form with fma, exact scaling by 2^n (two steps when
// the result is subnormal).
__device__ __forceinline__ float cexp(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __uint_as_float(0x7f800000u);
    if (x < -103.97208404541015625f) return 0.0f;
    const float t = x * 0x1.715476p+0f;
    const float n = __builtin_rintf(t);
    float r = fma_(n, -0x1.62e4p-1f, x);
    r = fma_(n, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-16f;
    p = fma_(p, r, 0x1.a01a02p-13f);
    p = fma_(p, r, 0x1.6c16c2p-10f);
    p = fma_(p, r, 0x1.111112p-7f);
    p = fma_(p, r, 0x1.555556p-5f);
    p = fma_(p, r, 0x1.555556p-3f);
    p = fma_(p, r, 0.5f);
    p = fma_(p, r, 1.0f);
    p = fma_(p, r, 1.0f);
    int e = static_cast<int>(n);
    if (e > 127) { p = p * 2.0f; e -= 1; }
    if (e < -126) { p = p * pow2i(e + 64); return p * 0x1p-64f; }
    return p * pow2i(e);
}

// Canonical log1p for x > -1: y = 1 + x with first-order correction
// (x - (y - 1)) / y, y = m * 2^k with m in [sqrt(1/2), sqrt(2)), and
// log(m) = 2 atanh(f / (2 + f)) by its odd series to z^4.
__device__ __forceinline__ float clog1p(float x) {
    if (x != x) return x;
    if (x == 0.0f) return x;
    if (x == __uint_as_float(0x7f800000u)) return x;
    if (x <= -1.0f) return x == -1.0f ? __uint_as_float(0xff800000u) : __uint_as_float(0x7fc00000u);
    const float y = 1.0f + x;
    const float c = (x - (y - 1.0f)) / y;
    const uint32_t b = __float_as_uint(y);
    int k = static_cast<int>((b >> 23) & 0xffu) - 126;
    float m = __uint_as_float((b & 0x807fffffu) | (126u << 23));
    if (m < 0x1.6a09e6p-1f) { m = m * 2.0f; k -= 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float w = fma_(z, 0x1.c71c72p-3f, 0x1.24924ap-2f);
    w = fma_(w, z, 0x1.99999ap-2f);
    w = fma_(w, z, 0x1.555556p-1f);
    const float logm = fma_(s * z, w, 2.0f * s);
    const float kf = static_cast<float>(k);
    float tt = logm + c;
    tt = fma_(kf, 0x1.7f7d1cp-20f, tt);
    return fma_(kf, 0x1.62e4p-1f, tt);
}

__device__ __forceinline__ float csigmoid(float x) { return 1.0f / (1.0f + cexp(-x)); }
__device__ __forceinline__ float csilu(float x) { return x / (1.0f + cexp(-x)); }
__device__ __forceinline__ float csqrt(float x) { return __builtin_sqrtf(x); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): loads whose byte offset is
// at or past `bytes` return zero, which masks rows past N or M without
// branches (dword3 = 0x00020000 is the gfx9 raw-buffer format word).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                           static_cast<int>(soff), 0));
}
constexpr uint32_t kOutOfRange = 0xfffffff0u;

// Cache-policy operand of the weight-stream loads: 2 = nt (non-temporal).
// Each weight byte is read once per launch; streaming it non-temporally keeps
// it from displacing the activations and other reused data in the caches
// (measured +5-8 % on the 27B-shape skinny GEMMs on MI355X).
#ifndef HAI_WLOAD_AUX
#define HAI_WLOAD_AUX 2
#endif
__device__ __forceinline__ u32x4 bload_w(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                           static_cast<int>(soff), HAI_WLOAD_AUX));
}
// The weight loads of a launch that reads each weight several times (row
// batches): cached, so that the batches after the first find them in L2.
template <bool kStream>
__device__ __forceinline__ u32x4 bload_wp(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                           static_cast<int>(soff),
                                                                           kStream ? HAI_WLOAD_AUX : 0));
}

// Index of the calling wave in its block, as a wave-uniform (scalar) value:
// derived from threadIdx.x, the compiler would otherwise treat it as
// per-lane.
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// Offsets of one chunk load at byte offset `off` from the lane's base offset.
// The scalar operand of a buffer load must be wave-uniform: a lane-dependent
// value there makes the compiler repeat the load once per distinct value (a
// readfirstlane loop around every load).  So a chunk that lies inside the
// range for every lane (`full`, uniform) passes `off` as the scalar offset;
// a ragged chunk folds `off` into the per-lane offset and sends the lanes
// past the end (ok false) out of range, where the load returns zeros.
struct ChunkOffset {
    bool full, ok;
    uint32_t s;    // scalar offset operand
    uint32_t off;
    __device__ __forceinline__ ChunkOffset(bool full_, bool ok_, uint32_t off_)
        : full(full_), ok(ok_), s(full_ ? off_ : 0u), off(off_) {}
    __device__ __forceinline__ uint32_t v(uint32_t base) const {
        return full ? base : (ok ? base + off : kOutOfRange);
    }
};

// The value of lane 16 r + (l + 8) % 16 for lane 16 r + l: a DPP rotate by
// 8 lanes within each row of 16 (row_ror:8).
__device__ __forceinline__ uint32_t row_ror8(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x128, 0xF, 0xF, false));
}

// Matrix-operand loads of 16 rows x 64 contiguous bytes per instruction (row
// li = lane % 16, 16-byte piece kg = lane / 16) stream poorly (16 rows per
// quarter-wave).  Two loads of 8 rows x 128 bytes instead -- i0: row li % 8,
// piece kg + 4 [li >= 8]; i1: row 8 + li % 8, piece kg + 4 [li < 8] -- read
// whole lines, and this turns them into the operand layout: r0 = piece kg of
// row li, r1 = piece kg + 4 of row li.
template <typename V4>
__device__ __forceinline__ void rows8x128_to_operands(const V4& i0, const V4& i1, bool low, V4& r0, V4& r1) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r0[q] = low ? i0[q] : i1[q];
        r1[q] = row_ror8(low ? i1[q] : i0[q]);
    }
}

// xor butterfly over the 64 lanes of a wave; all lanes get the same bits.
// The value of lane (lane ^ 1) / (lane ^ 2): a DPP quad permutation, no LDS
// round trip (same operands as __shfl_xor with those masks).
__device__ __forceinline__ float quad_xor1(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
}
__device__ __forceinline__ float quad_xor2(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
}
__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int s = 32; s >= 4; s >>= 1) v = v + __shfl_xor(v, s, 64);
    v = v + quad_xor2(v);
    return v + quad_xor1(v);
}
__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
    for (int s = 32; s >= 4; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    v = fmaxf(v, quad_xor2(v));
    return fmaxf(v, quad_xor1(v));
}

// L64-order sum of squares of a bf16 vector of length n (n % 8 == 0),
// computed by one wave (lane = threadIdx.x % 64).
__device__ __forceinline__ float l64_sumsq_bf16(const uint16_t* __restrict__ x, int n, int lane) {
    float acc = 0.0f;
    for (int k0 = lane * 8; k0 < n; k0 += 512) {
        const uint4 d = *reinterpret_cast<const uint4*>(x + k0);
        const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float a = lo_bf(w[q]);
            const float b = hi_bf(w[q]);
            acc = fma_(a, a, acc);
            acc = fma_(b, b, acc);
        }
    }
    return wave_sum64(acc);
}

// RMSNorm of one bf16 row by one wave (rmsnorm_kernel, hip_kernels.hip:
// 105-137): y_k = bf16((x_k * inv) * (w_k + off)), inv = 1 / sqrt(ss / H +
// eps), ss the L64-order sum of squares.  Up to NC * 512 elements: every
// load is issued before the first use; offsets past H read zeros.
template <int NC>
__device__ __forceinline__ void rmsnorm_row_wave(uint16_t* __restrict__ yr, const uint16_t* xr,
                                                 const uint16_t* __restrict__ w, int H, float eps, float off,
                                                 int lane) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xr, static_cast<uint32_t>(H) * 2u);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(H) * 2u);
    u32x4 xd[NC], wd[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t o = static_cast<uint32_t>(c * 512 + lane * 8) * 2u;
        xd[c] = bload(rx, o, 0);
        wd[c] = bload(rw, o, 0);
    }
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (c * 512 + lane * 8 >= H) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float a = lo_bf(xd[c][q]);
            const float b = hi_bf(xd[c][q]);
            acc = fma_(a, a, acc);
            acc = fma_(b, b, acc);
        }
    }
    const float ss = wave_sum64(acc);
    const float inv = 1.0f / csqrt(ss / static_cast<float>(H) + eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int k0 = c * 512 + lane * 8;
        if (k0 >= H) continue;
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = f2bf2((lo_bf(xd[c][q]) * inv) * (lo_bf(wd[c][q]) + off),
                         (hi_bf(xd[c][q]) * inv) * (hi_bf(wd[c][q]) + off));
        *reinterpret_cast<uint4*>(yr + k0) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Same order for an fp32 vector held in LDS or global memory.
__device__ __forceinline__ float l64_sumsq_f32(const float* x, int n, int lane) {
    float acc = 0.0f;
    for (int k0 = lane * 8; k0 < n; k0 += 512) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = k0 + j;
            if (k < n) acc = fma_(x[k], x[k], acc);
        }
    }
    return wave_sum64(acc);
}

// ---- head rows of the q / k norm + RoPE paths (one wave per head row) ----
constexpr int kMaxHeadDim = 512;

// A head row of D <= kMaxHeadDim bf16 values, 8 per lane: lane l holds
// elements 8l .. 8l+7 (the L64 order of l64_sumsq_bf16 for one pass).
struct HeadPiece {
    uint32_t w[4];
    __device__ __forceinline__ float at(int e) const { return (e & 1) ? hi_bf(w[e >> 1]) : lo_bf(w[e >> 1]); }
};
__device__ __forceinline__ HeadPiece load_piece(const uint16_t* __restrict__ row, int D, int lane) {
    HeadPiece p{{0u, 0u, 0u, 0u}};
    if (lane * 8 < D) {
        const uint4 d = *reinterpret_cast<const uint4*>(row + lane * 8);
        p.w[0] = d.x; p.w[1] = d.y; p.w[2] = d.z; p.w[3] = d.w;
    }
    return p;
}
// sum of squares of a head row in l64_sumsq_bf16's order (D <= 512: one pass)
__device__ __forceinline__ float piece_sumsq(const HeadPiece& p) {
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fma_(p.at(e), p.at(e), acc);
    return wave_sum64(acc);
}

// The rotation factors of the lane's dims d = lane + 64 i that RoPE touches
// (d < R), requested as soon as the position is known.
constexpr int kRopeSlots = kMaxHeadDim / 64;
__device__ __forceinline__ void load_rope(float (&cv)[kRopeSlots], float (&sv)[kRopeSlots], const float* cs,
                                          const float* sn, int D, int R, int lane) {
    const int half = R / 2;
#pragma unroll
    for (int i = 0; i < kRopeSlots; ++i) {
        const int d = lane + 64 * i;
        const int p = d < half ? d : d - half;
        cv[i] = d < D && d < R ? cs[p] : 0.0f;
        sv[i] = d < D && d < R ? sn[p] : 0.0f;
    }
}
// rope_at with the lane's factors for d = lane + 64 i in registers
__device__ __forceinline__ float rope_reg(const float* row, int d, int R, float c, float sn) {
    if (d >= R) return row[d];
    const int half = R / 2;
    const int p = d < half ? d : d - half;
    const float xv = row[p];
    const float yv = row[p + half];
    if (d < half) return fma_(xv, c, -(yv * sn));
    return fma_(yv, c, xv * sn);
}

}  // namespace hai
