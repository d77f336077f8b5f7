// hai_deltanet.hip -- fused Gated DeltaNet verify kernel: grouped causal conv
// (deltanet_grouped_conv_kernel, hip_kernels.hip:871-912) + gated delta rule
// (deltanet_recurrent_kernel, :985-1095) + gated RMSNorm, over the T tokens
// of a verify step.
//
// One block per (value head, sequence), 4 threads per state column.  Every
// global load of the step (state, conv history, taps and inputs, gates, z) is
// issued before the first use, and the token loop has no block barrier: the
// q/k norms of all T tokens are computed first and the gated RMSNorm of all
// outputs last.
//   * thread (j, g) keeps the dk/4 state entries S[g*dk/4 .. ][j] of column j
//     in registers for all T tokens; the key-dim reductions are fma chains
//     within the group followed by a 4-lane xor butterfly, (g0+g1)+(g2+g3);
//   * the state of a head is stored column-tiled: entry (key i, column j),
//     i = g*dk/4 + 4m + e, sits at float ((m*dv + j)*4 + g)*4 + e, so load or
//     store m of thread (j, g) = tid is float4 number m*4*dv + tid and every
//     instruction of the block covers one contiguous span;
//   * rollback needs no copies: the state after sequence length L is kept in
//     slot L % nslots and the conv inputs in a ring indexed by position, so
//     accepting a prefix only moves the committed length.
// No MFMA: the update is a rank-1 correction per token, bandwidth and latency
// bound.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kMaxT = 16;   // tokens per launch (verify width k + 1 <= 16)
constexpr int kMaxKc = 8;   // conv taps

template <int DK, int DV>
__global__ __launch_bounds__(DV * 4) void deltanet_verify_kernel(
    uint16_t* __restrict__ out, int64_t ld_out, const uint16_t* __restrict__ proj, int64_t ld_proj,
    int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b, const uint16_t* __restrict__ conv_w,
    uint16_t* __restrict__ ring, int ring_n, float* __restrict__ state, int nslots, int write_all,
    const uint16_t* __restrict__ a_log, const uint16_t* __restrict__ dt_bias,
    const uint16_t* __restrict__ norm_w, const int32_t* lens, int pos_add, int B, int T, int nk, int nv,
    int Kc, float eps) {
    constexpr int NT = DV * 4;
    constexpr int NW = NT / 64;
    constexpr int GI = DK / 4;            // key dims per thread
    constexpr int ZP = kMaxT * DV / NT;   // output elements per thread (all tokens)
    extern __shared__ float smem[];
    float* qs = smem;                  // [T][DK] conv output, q channels
    float* ks = qs + T * DK;           // [T][DK] k channels
    float* vs = ks + T * DK;           // [T][DV] v channels
    float* os = vs + T * DV;           // [T][DV] unrounded recurrent output
    __shared__ float s_q[kMaxT], s_k[kMaxT], s_decay[kMaxT], s_beta[kMaxT], s_rms[kMaxT];

    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = tid >> 2;
    const int g = tid & 3;
    const int group = nv / nk;
    const int gq = h / group;
    const int64_t kw = static_cast<int64_t>(nk) * DK;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t C = 2 * kw + vw;
    const int64_t p0 = static_cast<int64_t>(lens ? lens[b] : 0) + pos_add;
    const int hist = Kc - 1;
    const int64_t row0 = static_cast<int64_t>(b) * T;

    // ---- issue every global load of the step up front ----
    // committed state (slot p0 % nslots), column j, key dims [g*GI, g*GI+GI)
    float S[GI];
    {
        const int64_t slot = p0 % nslots;
        const float4* src = reinterpret_cast<const float4*>(state + ((slot * B + b) * nv + h) * static_cast<int64_t>(DV) * DK) + tid;
#pragma unroll
        for (int m = 0; m < GI / 4; ++m) {
            const float4 v4 = src[m * NT];
            S[4 * m] = v4.x; S[4 * m + 1] = v4.y; S[4 * m + 2] = v4.z; S[4 * m + 3] = v4.w;
        }
    }
    // conv channel of this thread: [0, DK) q, [DK, 2DK) k, [2DK, 2DK+DV) v
    const int cl = tid;
    const bool has_ch = cl < 2 * DK + DV;
    int64_t c = 0;
    if (cl < DK) c = static_cast<int64_t>(gq) * DK + cl;
    else if (cl < 2 * DK) c = kw + static_cast<int64_t>(gq) * DK + (cl - DK);
    else c = 2 * kw + static_cast<int64_t>(h) * DV + (cl - 2 * DK);
    // window: vals[i] = input at position p0 - hist + i (history, then the T new tokens)
    uint16_t vals[kMaxT + kMaxKc - 1];
    float wc[kMaxKc];
    if (has_ch) {
#pragma unroll
        for (int i = 0; i < kMaxKc - 1; ++i) {
            const int64_t pos = p0 - hist + i;
            vals[i] = (i < hist && pos >= 0)
                          ? ring[(static_cast<int64_t>(b) * ring_n + (pos % ring_n)) * C + c]
                          : uint16_t{0};
        }
#pragma unroll
        for (int i = 0; i < kMaxKc; ++i) wc[i] = i < Kc ? bf2f(conv_w[c * Kc + i]) : 0.0f;
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) {
            uint16_t x = 0;
            if (t < T) x = proj[(row0 + t) * ld_proj + off_qkv + c];
            // shift the new tokens in right after the hist history entries
#pragma unroll
            for (int hh = 0; hh < kMaxKc; ++hh)
                if (hh == hist) vals[t + hh] = x;
        }
    }
    // per-token gate scalars (last wave, lane = token)
    float a_in = 0.0f, b_in = 0.0f, dtb = 0.0f, alog = 0.0f;
    const bool scal = wave == NW - 1 && lane < T;
    if (scal) {
        a_in = bf2f(proj[(row0 + lane) * ld_proj + off_a + h]);
        b_in = bf2f(proj[(row0 + lane) * ld_proj + off_b + h]);
        dtb = bf2f(dt_bias[h]);
        alog = bf2f(a_log[h]);
    }
    // gate z and norm weight for the output elements (t, jo) = (tid / DV + r * NT / DV, tid % DV)
    const int jo = tid % DV;
    float zr[ZP];
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int t = tid / DV + r * (NT / DV);
        zr[r] = t < T ? bf2f(proj[(row0 + t) * ld_proj + off_z + static_cast<int64_t>(h) * DV + jo]) : 0.0f;
    }
    const float nwj = bf2f(norm_w[jo]);

    // ---- grouped causal conv + SiLU ----
    if (has_ch) {
        float* dst;
        int di, dstride;
        if (cl < DK) { dst = qs; di = cl; dstride = DK; }
        else if (cl < 2 * DK) { dst = ks; di = cl - DK; dstride = DK; }
        else { dst = vs; di = cl - 2 * DK; dstride = DV; }
        const bool writer = cl >= 2 * DK || (h % group) == 0;
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) {
            if (t < T) {
                float acc = bf2f(vals[t]) * wc[0];
#pragma unroll
                for (int i = 1; i < kMaxKc; ++i)
                    if (i < Kc) acc = fma_(bf2f(vals[t + i]), wc[i], acc);
                dst[t * dstride + di] = bfr(csilu(acc));
                if (writer) {
                    uint16_t xv = 0;
#pragma unroll
                    for (int hh = 0; hh < kMaxKc; ++hh)
                        if (hh == hist) xv = vals[t + hh];
                    ring[(static_cast<int64_t>(b) * ring_n + ((p0 + t) % ring_n)) * C + c] = xv;
                }
            }
        }
    }
    if (scal) {
        const float dtv = dtb + a_in;
        const float sp = fmaxf(dtv, 0.0f) + clog1p(cexp(-fabsf(dtv)));
        s_decay[lane] = cexp(-(cexp(alog) * sp));
        s_beta[lane] = csigmoid(b_in);
    }
    __syncthreads();

    // ---- L2 norms of q and k for every token (one wave per vector) ----
    const float rs_dk = 1.0f / csqrt(static_cast<float>(DK));
    for (int task = wave; task < 2 * T; task += NW) {
        const int t = task >> 1;
        if ((task & 1) == 0) {
            const float ssq = l64_sumsq_f32(qs + t * DK, DK, lane);
            if (lane == 0) s_q[t] = (1.0f / csqrt(ssq + 1.0e-6f)) * rs_dk;
        } else {
            const float ssk = l64_sumsq_f32(ks + t * DK, DK, lane);
            if (lane == 0) s_k[t] = 1.0f / csqrt(ssk + 1.0e-6f);
        }
    }
    __syncthreads();

    // ---- gated delta rule, token by token (column-local: no block barrier) ----
    for (int t = 0; t < T; ++t) {
        const float qsc = s_q[t], ksc = s_k[t], decay = s_decay[t], beta = s_beta[t];
        const float* qt = qs + t * DK + g * GI;
        const float* kt = ks + t * DK + g * GI;
        float r = 0.0f;
#pragma unroll
        for (int i = 0; i < GI; ++i) {
            S[i] = S[i] * decay;
            r = fma_(kt[i] * ksc, S[i], r);
        }
        r = r + __shfl_xor(r, 1, 64);
        r = r + __shfl_xor(r, 2, 64);
        const float cj = vs[t * DV + j] - r;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < GI; ++i) {
            S[i] = fma_(beta * (kt[i] * ksc), cj, S[i]);
            o = fma_(qt[i] * qsc, S[i], o);
        }
        o = o + __shfl_xor(o, 1, 64);
        o = o + __shfl_xor(o, 2, 64);
        if (write_all || t == T - 1) {
            const int64_t slot = (p0 + t + 1) % nslots;
            float4* dstp = reinterpret_cast<float4*>(state + ((slot * B + b) * nv + h) * static_cast<int64_t>(DV) * DK) + tid;
#pragma unroll
            for (int m = 0; m < GI / 4; ++m)
                dstp[m * NT] = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
        }
        if (g == 0) os[t * DV + j] = o;
    }
    __syncthreads();

    // ---- gated RMSNorm: rms from the unrounded output, one wave per token ----
    for (int t = wave; t < T; t += NW) {
        const float sso = l64_sumsq_f32(os + t * DV, DV, lane);
        if (lane == 0) s_rms[t] = 1.0f / csqrt(sso / static_cast<float>(DV) + eps);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int t = tid / DV + r * (NT / DV);
        if (t < T) {
            const float ob = bfr(os[t * DV + jo]);
            out[(row0 + t) * ld_out + static_cast<int64_t>(h) * DV + jo] =
                f2bf(((ob * s_rms[t]) * nwj) * csilu(zr[r]));
        }
    }
}

template <int DK, int DV>
int launch(uint16_t* out, int64_t ld_out, const uint16_t* proj, int64_t ld_proj, int64_t off_qkv,
           int64_t off_z, int64_t off_a, int64_t off_b, const uint16_t* conv_w, uint16_t* ring, int ring_n,
           float* state, int nslots, int write_all, const uint16_t* a_log, const uint16_t* dt_bias,
           const uint16_t* norm_w, const int32_t* lens, int pos_add, int B, int T, int nk, int nv, int Kc,
           float eps, hipStream_t s) {
    const size_t shmem = static_cast<size_t>(T) * (2 * DK + 2 * DV) * sizeof(float);
    deltanet_verify_kernel<DK, DV><<<dim3(nv, B), dim3(DV * 4), shmem, s>>>(
        out, ld_out, proj, ld_proj, off_qkv, off_z, off_a, off_b, conv_w, ring, ring_n, state, nslots,
        write_all, a_log, dt_bias, norm_w, lens, pos_add, B, T, nk, nv, Kc, eps);
    return launched("deltanet_verify_kernel");
}

}  // namespace

extern "C" int hai_deltanet_verify_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                        int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b,
                                        const void* conv_w, void* conv_ring, int64_t ring, float* state,
                                        int64_t nslots, int write_all_slots, const void* a_log,
                                        const void* dt_bias, const void* norm_w, const int32_t* lens,
                                        int32_t pos_add, int64_t B, int64_t T, int64_t nk, int64_t nv,
                                        int64_t dk, int64_t dv, int64_t Kc, float eps, void* stream) {
    if (out == nullptr || proj == nullptr || conv_w == nullptr || conv_ring == nullptr || state == nullptr ||
        a_log == nullptr || dt_bias == nullptr || norm_w == nullptr)
        return invalid("deltanet_verify: null pointer");
    if (B < 0 || T < 0 || nk <= 0 || nv <= 0 || nv % nk != 0 || Kc < 1 || Kc > 8 || nslots < 1)
        return invalid("deltanet_verify: shape");
    if (T + Kc - 1 > ring) return invalid("deltanet_verify: conv ring too short for T");
    if (write_all_slots && nslots < T) return invalid("deltanet_verify: fewer state slots than tokens");
    if (lens == nullptr && pos_add < 0) return invalid("deltanet_verify: negative position");
    if (!aligned16(state)) return invalid("deltanet_verify: state alignment");
    if (B == 0 || T == 0) return HAI_OK;
    if (T > kMaxT) return invalid("deltanet_verify: at most 16 tokens per launch");
    const auto s = as_stream(stream);
    auto* o = static_cast<uint16_t*>(out);
    const auto* pr = static_cast<const uint16_t*>(proj);
    const auto* cw = static_cast<const uint16_t*>(conv_w);
    auto* rg = static_cast<uint16_t*>(conv_ring);
    const auto* al = static_cast<const uint16_t*>(a_log);
    const auto* db = static_cast<const uint16_t*>(dt_bias);
    const auto* nw = static_cast<const uint16_t*>(norm_w);
    if (dk == 128 && dv == 128)
        return launch<128, 128>(o, ld_out, pr, ld_proj, off_qkv, off_z, off_a, off_b, cw, rg, int(ring), state,
                                int(nslots), write_all_slots, al, db, nw, lens, pos_add, int(B), int(T), int(nk),
                                int(nv), int(Kc), eps, s);
    if (dk == 64 && dv == 64)
        return launch<64, 64>(o, ld_out, pr, ld_proj, off_qkv, off_z, off_a, off_b, cw, rg, int(ring), state,
                              int(nslots), write_all_slots, al, db, nw, lens, pos_add, int(B), int(T), int(nk),
                              int(nv), int(Kc), eps, s);
    return invalid("deltanet_verify: (dk, dv) must be (128,128) or (64,64)");
}
