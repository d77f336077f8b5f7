// oracle_numerics.h -- TEST INFRASTRUCTURE ONLY.
//
// CPU restatement of the numerics that the HybridAI MTP verify path uses,
// written for the parity oracle.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load the oracle; the product never does.
//
// The reference (Dustray/Vicold.HybridAI) computes in fp32 with bf16
// storage between ops:
//   * bf16 stores are round-to-nearest-even (hip_bfloat16(float) is RNE;
//     reference tests restate it at tests/hip_kernels_test.cc:15-20);
//   * transcendental functions are the device expf/log1pf/rsqrtf
//     (src/backends/hip/hip_kernels.hip:164-175, 1037-1049).
// Bit-exact token parity between a CPU and a GPU needs every rounding point
// to be identical, so both sides use one *canonical* definition of each
// primitive, chosen here:
//   * exp: Cody-Waite reduction by ln2 split into hi/lo, degree-8 Taylor
//     polynomial evaluated with fma (Horner), exact scaling by 2^n with a
//     two-step scale for subnormal results.  Accuracy is pinned against libm
//     in tests/test_oracle_numerics.py (<= 2 ulp).
//   * log1p: y = 1+x with the first-order correction (x-(y-1))/y, reduction
//     of y to m*2^k with m in [sqrt(1/2), sqrt(2)), atanh series in s=f/(2+f).
//   * sqrt and division are IEEE correctly rounded; fma is the IEEE fused
//     multiply-add.
//   * "L64 order": a length-n reduction is split over 64 lanes, element k
//     going to lane (k/8)%64 and each lane accumulating its elements in
//     increasing k with fma; the 64 lane partials are then combined by the
//     xor butterfly (offsets 32,16,8,4,2,1).  This is exactly the order in
//     which a 64-wide wavefront that loads 8 consecutive bf16 per lane
//     reduces a row.
// This file is compiled with -ffp-contract=off so that every a*b+c written
// without fma is two roundings, as it is on the GPU side.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace orc {

inline float bits_to_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f_to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// bf16 round-to-nearest-even; NaN stays a quiet NaN with its sign.
inline uint16_t bf16_bits(float f) {
    uint32_t u = f_to_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
inline float bf16_val(uint16_t h) { return bits_to_f(static_cast<uint32_t>(h) << 16); }
inline float bf(float f) { return bf16_val(bf16_bits(f)); }

inline float fmaf_(float a, float b, float c) { return std::fma(a, b, c); }

inline float pow2i(int e) {  // 2^e for e in [-126, 127]
    return bits_to_f(static_cast<uint32_t>(e + 127) << 23);
}

// Canonical exp (see header comment).
inline float cexp(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    const float t = x * 0x1.715476p+0f;
    const float n = std::rint(t);
    float r = fmaf_(n, -0x1.62e4p-1f, x);
    r = fmaf_(n, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-16f;
    p = fmaf_(p, r, 0x1.a01a02p-13f);
    p = fmaf_(p, r, 0x1.6c16c2p-10f);
    p = fmaf_(p, r, 0x1.111112p-7f);
    p = fmaf_(p, r, 0x1.555556p-5f);
    p = fmaf_(p, r, 0x1.555556p-3f);
    p = fmaf_(p, r, 0.5f);
    p = fmaf_(p, r, 1.0f);
    p = fmaf_(p, r, 1.0f);
    int e = static_cast<int>(n);
    if (e > 127) { p = p * 2.0f; e -= 1; }
    if (e < -126) { p = p * pow2i(e + 64); return p * 0x1p-64f; }
    return p * pow2i(e);
}

// Canonical log1p for x > -1 (see header comment).
inline float clog1p(float x) {
    if (x != x) return x;
    if (x == 0.0f) return x;
    if (x == INFINITY) return x;
    if (x <= -1.0f) return x == -1.0f ? -INFINITY : NAN;
    const float y = 1.0f + x;
    const float c = (x - (y - 1.0f)) / y;
    const uint32_t b = f_to_bits(y);
    int k = static_cast<int>((b >> 23) & 0xffu) - 126;
    float m = bits_to_f((b & 0x807fffffu) | (126u << 23));  // [0.5, 1)
    if (m < 0x1.6a09e6p-1f) { m = m * 2.0f; k -= 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float w = fmaf_(z, 0x1.c71c72p-3f, 0x1.24924ap-2f);
    w = fmaf_(w, z, 0x1.99999ap-2f);
    w = fmaf_(w, z, 0x1.555556p-1f);
    const float logm = fmaf_(s * z, w, 2.0f * s);
    const float kf = static_cast<float>(k);
    float t = logm + c;
    t = fmaf_(kf, 0x1.7f7d1cp-20f, t);
    return fmaf_(kf, 0x1.62e4p-1f, t);
}

inline float csigmoid(float x) { return 1.0f / (1.0f + cexp(-x)); }
inline float csilu(float x) { return x / (1.0f + cexp(-x)); }

// xor butterfly over 64 lane partials; every lane ends with the same bits.
inline float butterfly64(float* acc) {
    for (int s = 32; s >= 1; s >>= 1) {
        float t[64];
        for (int l = 0; l < 64; ++l) t[l] = acc[l] + acc[l ^ s];
        for (int l = 0; l < 64; ++l) acc[l] = t[l];
    }
    return acc[0];
}

// L64-order dot product of two fp32 vectors (values already decoded).
inline float l64_dot(const float* a, const float* b, int64_t n) {
    float acc[64];
    for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
    for (int64_t k = 0; k < n; ++k) {
        const int l = static_cast<int>((k >> 3) & 63);
        acc[l] = fmaf_(a[k], b[k], acc[l]);
    }
    return butterfly64(acc);
}

// Linear-layer dot product ("segmented L64"): the L64 element-to-lane map,
// but each lane's fma chain restarts every kGemmSeg elements and the segment
// partials are folded in segment order before the butterfly.  Segments let
// several GPU waves share the K range of one output (each wave owns whole
// segments) without changing a bit; for K <= kGemmSeg it is l64_dot.
constexpr int64_t kGemmSeg = 2048;
inline float gemm_dot(const float* a, const float* b, int64_t n) {
    float tot[64];
    for (int l = 0; l < 64; ++l) tot[l] = 0.0f;
    for (int64_t s0 = 0; s0 < n; s0 += kGemmSeg) {
        float part[64];
        for (int l = 0; l < 64; ++l) part[l] = 0.0f;
        const int64_t e = s0 + kGemmSeg < n ? s0 + kGemmSeg : n;
        for (int64_t k = s0; k < e; ++k) {
            const int l = static_cast<int>((k >> 3) & 63);
            part[l] = fmaf_(a[k], b[k], part[l]);
        }
        for (int l = 0; l < 64; ++l) tot[l] = tot[l] + part[l];
    }
    return butterfly64(tot);
}

// Sequential fma dot (attention scores: one lane owns one key).
inline float seq_dot(const float* a, const float* b, int64_t n) {
    float acc = 0.0f;
    for (int64_t k = 0; k < n; ++k) acc = fmaf_(a[k], b[k], acc);
    return acc;
}

}  // namespace orc
