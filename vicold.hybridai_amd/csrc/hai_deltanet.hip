// hai_deltanet.hip -- fused Gated DeltaNet verify kernel: grouped causal conv
// (deltanet_grouped_conv_kernel, hip_kernels.hip:871-912) + gated delta rule
// (deltanet_recurrent_kernel, :985-1095) + gated RMSNorm, over the T tokens
// of a verify step.
//
// One block per (value head, sequence), 4 threads per state column:
//   * thread (j, g) keeps the dk/4 state entries S[g*dk/4 .. ][j] of column j
//     in registers for all T tokens; the key-dim reductions are fma chains
//     within the group followed by a 4-lane xor butterfly, (g0+g1)+(g2+g3);
//   * the state is stored value-major [dv][dk] so the 4 threads of a column
//     read and write 512 contiguous bytes;
//   * rollback needs no copies: the state after sequence length L is kept in
//     slot L % nslots and the conv inputs in a ring indexed by position, so
//     accepting a prefix only moves the committed length.
// No MFMA: the update is a rank-1 correction per token, bandwidth and latency
// bound.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

template <int DK, int DV>
__global__ __launch_bounds__(DV * 4) void deltanet_verify_kernel(
    uint16_t* __restrict__ out, int64_t ld_out, const uint16_t* __restrict__ proj, int64_t ld_proj,
    int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b, const uint16_t* __restrict__ conv_w,
    uint16_t* __restrict__ ring, int ring_n, float* __restrict__ state, int nslots, int write_all,
    const uint16_t* __restrict__ a_log, const uint16_t* __restrict__ dt_bias,
    const uint16_t* __restrict__ norm_w, const int32_t* lens, int pos_add, int B, int T, int nk, int nv,
    int Kc, float eps) {
    constexpr int NT = DV * 4;
    constexpr int GI = DK / 4;  // key dims per thread
    extern __shared__ float smem[];
    float* qs = smem;                  // [T][DK]
    float* ks = qs + T * DK;           // [T][DK]
    float* vs = ks + T * DK;           // [T][DV]
    __shared__ float osh[DV];
    __shared__ float sc[4];            // q scale, k scale, decay, beta
    __shared__ float rms_sh;

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

    // ---- grouped causal conv + SiLU for this head's q, k and v channels ----
    for (int cl = tid; cl < 2 * DK + DV; cl += NT) {
        int64_t c;
        float* dst;
        int di;
        int dstride;
        if (cl < DK) { c = static_cast<int64_t>(gq) * DK + cl; dst = qs; di = cl; dstride = DK; }
        else if (cl < 2 * DK) { c = kw + static_cast<int64_t>(gq) * DK + (cl - DK); dst = ks; di = cl - DK; dstride = DK; }
        else { c = 2 * kw + static_cast<int64_t>(h) * DV + (cl - 2 * DK); dst = vs; di = cl - 2 * DK; dstride = DV; }
        float win[8];  // history window (Kc <= 8)
        for (int i = 0; i < hist; ++i) {
            const int64_t pos = p0 - hist + i;
            win[i] = pos < 0 ? 0.0f
                             : bf2f(ring[(static_cast<int64_t>(b) * ring_n + (pos % ring_n)) * C + c]);
        }
        float wc[8];
        for (int i = 0; i < Kc; ++i) wc[i] = bf2f(conv_w[c * Kc + i]);
        const bool writer = cl >= 2 * DK || (h % group) == 0;
        for (int t = 0; t < T; ++t) {
            const uint16_t xb = proj[(static_cast<int64_t>(b) * T + t) * ld_proj + off_qkv + c];
            const float x = bf2f(xb);
            float acc;
            if (hist > 0) {
                acc = win[0] * wc[0];
                for (int i = 1; i < hist; ++i) acc = fma_(win[i], wc[i], acc);
                acc = fma_(x, wc[hist], acc);
            } else {
                acc = x * wc[0];
            }
            dst[t * dstride + di] = bfr(csilu(acc));
            for (int i = 0; i + 1 < hist; ++i) win[i] = win[i + 1];
            if (hist > 0) win[hist - 1] = x;
            if (writer) ring[(static_cast<int64_t>(b) * ring_n + ((p0 + t) % ring_n)) * C + c] = xb;
        }
    }

    // ---- load the committed state (slot p0 % nslots) ----
    float S[GI];
    {
        const int64_t slot = p0 % nslots;
        const float* src = state + (((slot * B + b) * nv + h) * static_cast<int64_t>(DV) + j) * DK + g * GI;
#pragma unroll
        for (int i = 0; i < GI; i += 4) {
            const float4 v4 = *reinterpret_cast<const float4*>(src + i);
            S[i] = v4.x; S[i + 1] = v4.y; S[i + 2] = v4.z; S[i + 3] = v4.w;
        }
    }
    __syncthreads();

    const float rs_dk = 1.0f / csqrt(static_cast<float>(DK));
    for (int t = 0; t < T; ++t) {
        const int64_t row = static_cast<int64_t>(b) * T + t;
        if (wave == 0) {
            const float ssq = l64_sumsq_f32(qs + t * DK, DK, lane);
            if (lane == 0) sc[0] = (1.0f / csqrt(ssq + 1.0e-6f)) * rs_dk;
        } else if (wave == 1) {
            const float ssk = l64_sumsq_f32(ks + t * DK, DK, lane);
            if (lane == 0) sc[1] = 1.0f / csqrt(ssk + 1.0e-6f);
        } else if (wave == 2 && lane == 0) {
            const float av = bf2f(proj[row * ld_proj + off_a + h]);
            const float bv = bf2f(proj[row * ld_proj + off_b + h]);
            const float dtv = bf2f(dt_bias[h]) + av;
            const float sp = fmaxf(dtv, 0.0f) + clog1p(cexp(-fabsf(dtv)));
            sc[2] = cexp(-(cexp(bf2f(a_log[h])) * sp));
            sc[3] = csigmoid(bv);
        }
        __syncthreads();
        const float qsc = sc[0], ksc = sc[1], decay = sc[2], beta = sc[3];
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
            float* dstp = state + (((slot * B + b) * nv + h) * static_cast<int64_t>(DV) + j) * DK + g * GI;
#pragma unroll
            for (int i = 0; i < GI; i += 4)
                *reinterpret_cast<float4*>(dstp + i) = make_float4(S[i], S[i + 1], S[i + 2], S[i + 3]);
        }
        if (g == 0) osh[j] = o;
        __syncthreads();
        if (wave == 0) {
            const float sso = l64_sumsq_f32(osh, DV, lane);
            if (lane == 0) rms_sh = 1.0f / csqrt(sso / static_cast<float>(DV) + eps);
        }
        __syncthreads();
        if (g == 0) {
            const float ob = bfr(o);
            const float z = bf2f(proj[row * ld_proj + off_z + static_cast<int64_t>(h) * DV + j]);
            out[row * ld_out + static_cast<int64_t>(h) * DV + j] =
                f2bf(((ob * rms_sh) * bf2f(norm_w[j])) * csilu(z));
        }
        __syncthreads();
    }
}

template <int DK, int DV>
int launch(uint16_t* out, int64_t ld_out, const uint16_t* proj, int64_t ld_proj, int64_t off_qkv,
           int64_t off_z, int64_t off_a, int64_t off_b, const uint16_t* conv_w, uint16_t* ring, int ring_n,
           float* state, int nslots, int write_all, const uint16_t* a_log, const uint16_t* dt_bias,
           const uint16_t* norm_w, const int32_t* lens, int pos_add, int B, int T, int nk, int nv, int Kc,
           float eps, hipStream_t s) {
    const size_t shmem = static_cast<size_t>(T) * (2 * DK + DV) * sizeof(float);
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
    if (T * (2 * dk + dv) * 4 > 64 * 1024) return invalid("deltanet_verify: T too large for LDS staging");
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
