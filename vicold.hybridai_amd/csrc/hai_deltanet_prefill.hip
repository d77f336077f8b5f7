// hai_deltanet_prefill.hip -- Gated DeltaNet over prompt chunks (the
// prefill's deltanet_grouped_conv_kernel + deltanet_recurrent_kernel,
// hip_kernels.hip:871-912, 985-1095, and the gated RMSNorm), tolerance mode.
//
// The verify kernel keeps a head's state in one block, 4 threads per value
// column, and walks the tokens one after another: each token is a chain of
// two 32-long fma sums, so a prompt costs ~1.5 us per token and layer.  The
// recurrence is independent per value column, so here
//   * a head's columns are split over DV / 32 blocks and every column over
//     16 threads (8 key dims each at dk = 128): the dependent chain of a
//     token is 8 fmas and a 16-lane sum (DPP: row rotates, then quad
//     swaps), and four times as many CUs work on a head;
//   * the tokens run in groups of 16: the group's conv outputs (from the
//     projection rows, the first ones reading the conv ring), gates and q/k
//     norms are computed in parallel, then the group's recurrence; the state
//     stays in registers across groups and is stored once, to slot
//     (L + T) % nslots, with the conv ring's last entries;
//   * the unrounded outputs go to a workspace, and a second kernel applies
//     the gated RMSNorm per (token, head).
// The sums are regrouped (16 lanes instead of 4), so results equal the
// canonical recurrence to fp32 reassociation, not bit for bit.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kGroup = 16;   // tokens per group
constexpr int kTpc = 16;     // threads per value column
constexpr int kCols = 32;    // value columns per block
constexpr int kMaxKc = 8;

struct PrefillArgs {
    float* o_ws;            // [B*T][nv*dv] unrounded outputs
    const uint16_t* proj;   // rows b*T + t: [qkv | z | a | b] at the offsets
    int64_t ld_proj, off_qkv, off_a, off_b;
    const uint16_t* conv_w;
    uint16_t* ring;
    int ring_n, nslots;
    float* state;
    const uint16_t *a_log, *dt_bias;
    const int32_t* lens;
    int pos_add;
    int B, T, nk, nv, Kc;
};

// sum over the 16 lanes of a DPP row, the same value in every lane
__device__ __forceinline__ float row16_sum(float v) {
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
    v = v + quad_xor2(v);
    return v + quad_xor1(v);
}

// grid (nv, DV / kCols, B); block kCols * kTpc threads.  Thread (jl, g)
// holds keys g*GI .. g*GI + GI - 1 of column j0 + jl.
template <int DK, int DV>
__global__ __launch_bounds__(kCols * kTpc) void deltanet_prefill_kernel(PrefillArgs A) {
    constexpr int NT = kCols * kTpc;
    constexpr int NW = NT / 64;
    constexpr int GI = DK / kTpc;          // key dims per thread
    constexpr int QPT = kTpc / 4;          // threads per quarter of the keys
    constexpr int NCH = 2 * DK + kCols;    // conv channels: q, k, this block's v columns
    static_assert(GI % 4 == 0 && NCH <= NT, "layout");
    __shared__ __align__(16) float qs[kGroup][DK];
    __shared__ __align__(16) float ks[kGroup][DK];
    __shared__ __align__(16) float bks[kGroup][DK];
    __shared__ float vs[kGroup][kCols];
    __shared__ float s_q[kGroup], s_k[kGroup], s_decay[kGroup], s_beta[kGroup];

    const int h = blockIdx.x;
    const int j0 = blockIdx.y * kCols;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int jl = tid / kTpc;
    const int g = tid % kTpc;
    const int j = j0 + jl;
    const int nv = A.nv;
    const int group = nv / A.nk;
    const int gq = h / group;
    const int64_t kw = static_cast<int64_t>(A.nk) * DK;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t C = 2 * kw + vw;
    const int hist = A.Kc - 1;
    const int T = A.T;
    const int64_t row0 = static_cast<int64_t>(b) * T;
    const int64_t p0 = static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;

    // conv channel of this thread: [0, DK) q, [DK, 2DK) k, then the block's v columns
    const bool has_ch = tid < NCH;
    int64_t chan = 0;
    if (tid < DK) chan = static_cast<int64_t>(gq) * DK + tid;
    else if (tid < 2 * DK) chan = kw + static_cast<int64_t>(gq) * DK + (tid - DK);
    else chan = 2 * kw + static_cast<int64_t>(h) * DV + j0 + (tid - 2 * DK);
    float wc[kMaxKc];
#pragma unroll
    for (int i = 0; i < kMaxKc; ++i) wc[i] = (has_ch && i < A.Kc) ? bf2f(A.conv_w[chan * A.Kc + i]) : 0.0f;
    const float dtb = bf2f(A.dt_bias[h]);
    const float alog = bf2f(A.a_log[h]);

    // state: keys g*GI + u of column j, from slot p0 % nslots (column-tiled
    // layout: key i = q4*(DK/4) + 4m + e at float ((m*DV + j)*4 + q4)*4 + e)
    const int q4 = g / QPT;
    const int m0 = (g % QPT) * (GI / 4);
    float S[GI];
    {
        const float* src = A.state + ((p0 % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                           static_cast<int64_t>(h) * DV * DK;
#pragma unroll
        for (int mm = 0; mm < GI / 4; ++mm) {
            const float4 v4 = *reinterpret_cast<const float4*>(src + ((static_cast<int64_t>(m0 + mm) * DV + j) * 4 + q4) * 4);
            S[4 * mm] = v4.x; S[4 * mm + 1] = v4.y; S[4 * mm + 2] = v4.z; S[4 * mm + 3] = v4.w;
        }
    }
    const float rs_dk = 1.0f / csqrt(static_cast<float>(DK));

    for (int t0 = 0; t0 < T; t0 += kGroup) {
        const int TS = min(kGroup, T - t0);
        // ---- conv + SiLU of the group's tokens: input at chunk position
        // t0 - hist + i from the projection rows, before the chunk from the
        // conv ring (positions before 0 read as zero) ----
        if (has_ch) {
            uint16_t x[kGroup + kMaxKc - 1];
#pragma unroll
            for (int i = 0; i < kGroup + kMaxKc - 1; ++i) {
                const int r = t0 - hist + i;
                uint16_t v = 0;
                if (i < TS + hist) {
                    if (r >= 0) {
                        v = A.proj[(row0 + r) * A.ld_proj + A.off_qkv + chan];
                    } else if (p0 + r >= 0) {
                        int64_t rp = (p0 + r) % A.ring_n;
                        v = A.ring[(static_cast<int64_t>(b) * A.ring_n + rp) * C + chan];
                    }
                }
                x[i] = v;
            }
#pragma unroll
            for (int tt = 0; tt < kGroup; ++tt) {
                if (tt < TS) {
                    // taps: x[tt + hist - (Kc - 1) + i] * w[i], i.e. the verify kernel's window
                    float acc = bf2f(x[tt]) * wc[0];
#pragma unroll
                    for (int i = 1; i < kMaxKc; ++i)
                        if (i < A.Kc) acc = fma_(bf2f(x[tt + i]), wc[i], acc);
                    const float y = bfr(csilu(acc));
                    if (tid < DK) qs[tt][tid] = y;
                    else if (tid < 2 * DK) ks[tt][tid - DK] = y;
                    else vs[tt][tid - 2 * DK] = y;
                }
            }
        }
        // ---- gates of the group's tokens (last wave, lane = token) ----
        if (wave == NW - 1 && lane < TS) {
            const float a_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_a + h]);
            const float b_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_b + h]);
            const float dtv = dtb + a_in;
            const float sp = fmaxf(dtv, 0.0f) + clog1p(cexp(-fabsf(dtv)));
            s_decay[lane] = cexp(-(cexp(alog) * sp));
            s_beta[lane] = csigmoid(b_in);
        }
        __syncthreads();
        // ---- L2 norms of q and k (one wave per vector) ----
        for (int task = wave; task < 2 * TS; task += NW) {
            const int t = task >> 1;
            if ((task & 1) == 0) {
                const float ssq = l64_sumsq_f32(qs[t], DK, lane);
                if (lane == 0) s_q[t] = (1.0f / csqrt(ssq + 1.0e-6f)) * rs_dk;
            } else {
                const float ssk = l64_sumsq_f32(ks[t], DK, lane);
                if (lane == 0) s_k[t] = 1.0f / csqrt(ssk + 1.0e-6f);
            }
        }
        __syncthreads();
        for (int e = tid; e < TS * DK; e += NT) {
            const int t = e / DK, d = e % DK;
            qs[t][d] = qs[t][d] * s_q[t];
            const float kh = ks[t][d] * s_k[t];
            ks[t][d] = kh;
            bks[t][d] = s_beta[t] * kh;
        }
        __syncthreads();
        // ---- the group's recurrence (column-local: no block barrier) ----
        for (int tt = 0; tt < TS; ++tt) {
            const float decay = s_decay[tt];
            const float4* kt = reinterpret_cast<const float4*>(&ks[tt][g * GI]);
            const float4* bt = reinterpret_cast<const float4*>(&bks[tt][g * GI]);
            const float4* qt = reinterpret_cast<const float4*>(&qs[tt][g * GI]);
            float r = 0.0f;
#pragma unroll
            for (int mm = 0; mm < GI / 4; ++mm) {
                const float4 k4 = kt[mm];
                const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    S[4 * mm + e] = S[4 * mm + e] * decay;
                    r = fma_(kv[e], S[4 * mm + e], r);
                }
            }
            r = row16_sum(r);
            const float cj = vs[tt][jl] - r;
            float o = 0.0f;
#pragma unroll
            for (int mm = 0; mm < GI / 4; ++mm) {
                const float4 b4 = bt[mm], q4v = qt[mm];
                const float bv[4] = {b4.x, b4.y, b4.z, b4.w}, qv[4] = {q4v.x, q4v.y, q4v.z, q4v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    S[4 * mm + e] = fma_(bv[e], cj, S[4 * mm + e]);
                    o = fma_(qv[e], S[4 * mm + e], o);
                }
            }
            o = row16_sum(o);
            if (g == 0) A.o_ws[(row0 + t0 + tt) * vw + static_cast<int64_t>(h) * DV + j] = o;
        }
        __syncthreads();  // the next group rewrites the LDS rows
    }

    // ---- the state after the chunk, and the conv ring's last entries ----
    {
        float* dst = A.state + (((p0 + T) % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                     static_cast<int64_t>(h) * DV * DK;
#pragma unroll
        for (int mm = 0; mm < GI / 4; ++mm)
            *reinterpret_cast<float4*>(dst + ((static_cast<int64_t>(m0 + mm) * DV + j) * 4 + q4) * 4) =
                make_float4(S[4 * mm], S[4 * mm + 1], S[4 * mm + 2], S[4 * mm + 3]);
    }
}

// The conv ring's entries for the chunk's last Kc - 1 positions (the only
// ones a later step reads), after every block has read the entries before
// the chunk: a chunk of T = ring_n tokens maps its last positions onto the
// same entries.  grid (ceil(C / 256), Kc - 1, B).
__global__ __launch_bounds__(256) void deltanet_ring_update_kernel(uint16_t* __restrict__ ring, int ring_n,
                                                                   const uint16_t* __restrict__ proj,
                                                                   int64_t ld_proj, int64_t off_qkv, int64_t C,
                                                                   const int32_t* lens, int pos_add, int T, int hist) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int i = blockIdx.y;
    const int b = blockIdx.z;
    const int r = T - hist + i;
    if (c >= C || r < 0) return;  // a position before the chunk: the ring has it already
    const int64_t p = static_cast<int64_t>(lens ? lens[b] : 0) + pos_add + r;
    ring[(static_cast<int64_t>(b) * ring_n + p % ring_n) * C + c] = proj[(static_cast<int64_t>(b) * T + r) * ld_proj + off_qkv + c];
}

// Gated RMSNorm of the outputs: one wave per (row, head); rms of the
// unrounded output, then bf16(((bf16(o) * rms) * w) * silu(z))
// (the verify kernel's epilogue).
template <int DV>
__global__ __launch_bounds__(256) void deltanet_gated_norm_kernel(uint16_t* __restrict__ out, int64_t ld_out,
                                                                  const float* __restrict__ o_ws,
                                                                  const uint16_t* __restrict__ proj, int64_t ld_proj,
                                                                  int64_t off_z, const uint16_t* __restrict__ norm_w,
                                                                  int64_t rows, int nv, float eps) {
    constexpr int PER = DV / 64;
    const int lane = threadIdx.x & 63;
    const int64_t task = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (task >= rows * nv) return;
    const int64_t row = task / nv;
    const int h = static_cast<int>(task % nv);
    const float* o = o_ws + (row * nv + h) * DV;
    const float ss = l64_sumsq_f32(o, DV, lane);
    const float rms = 1.0f / csqrt(ss / static_cast<float>(DV) + eps);
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int jo = lane + 64 * r;
        const float z = bf2f(proj[row * ld_proj + off_z + static_cast<int64_t>(h) * DV + jo]);
        out[row * ld_out + static_cast<int64_t>(h) * DV + jo] = f2bf(((bfr(o[jo]) * rms) * bf2f(norm_w[jo])) * csilu(z));
    }
}

template <int DK, int DV>
int launch_prefill(const PrefillArgs& a, uint16_t* out, int64_t ld_out, int64_t off_z, const uint16_t* norm_w,
                   float eps, hipStream_t s) {
    deltanet_prefill_kernel<DK, DV><<<dim3(a.nv, DV / kCols, a.B), dim3(kCols * kTpc), 0, s>>>(a);
    int rc = launched("deltanet_prefill_kernel");
    if (rc != HAI_OK) return rc;
    const int hist = a.Kc - 1;
    if (hist > 0) {
        const int64_t C = 2 * static_cast<int64_t>(a.nk) * DK + static_cast<int64_t>(a.nv) * DV;
        deltanet_ring_update_kernel<<<dim3(static_cast<unsigned>((C + 255) / 256), hist, a.B), dim3(256), 0, s>>>(
            a.ring, a.ring_n, a.proj, a.ld_proj, a.off_qkv, C, a.lens, a.pos_add, a.T, hist);
        rc = launched("deltanet_ring_update_kernel");
        if (rc != HAI_OK) return rc;
    }
    const int64_t tasks = static_cast<int64_t>(a.B) * a.T * a.nv;
    deltanet_gated_norm_kernel<DV><<<dim3(static_cast<unsigned>((tasks + 3) / 4)), dim3(256), 0, s>>>(
        out, ld_out, a.o_ws, a.proj, a.ld_proj, off_z, norm_w, static_cast<int64_t>(a.B) * a.T, a.nv, eps);
    return launched("deltanet_gated_norm_kernel");
}

}  // namespace

extern "C" size_t hai_deltanet_prefill_workspace_bytes(int64_t B, int64_t T, int64_t nv, int64_t dv) {
    if (B < 0 || T < 0 || nv < 0 || dv < 0) return 0;
    return static_cast<size_t>(B * T * nv * dv) * sizeof(float);
}

extern "C" int hai_deltanet_prefill_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                         int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b,
                                         const void* conv_w, void* conv_ring, int64_t ring, float* state,
                                         int64_t nslots, const void* a_log, const void* dt_bias,
                                         const void* norm_w, const int32_t* lens, int32_t pos_add, int64_t B,
                                         int64_t T, int64_t nk, int64_t nv, int64_t dk, int64_t dv, int64_t Kc,
                                         float eps, void* workspace, int64_t workspace_bytes, void* stream) {
    if (out == nullptr || proj == nullptr || conv_w == nullptr || conv_ring == nullptr || state == nullptr ||
        a_log == nullptr || dt_bias == nullptr || norm_w == nullptr || workspace == nullptr)
        return invalid("deltanet_prefill: null pointer");
    if (B < 0 || T < 0 || nk <= 0 || nv <= 0 || nv % nk != 0 || Kc < 1 || Kc > kMaxKc || nslots < 1 || ring < Kc ||
        B > 65535 || nv > 65535 || T > INT32_MAX / 2 || static_cast<int64_t>(pos_add) + T > INT32_MAX)
        return invalid("deltanet_prefill: shape");
    if (lens == nullptr && pos_add < 0) return invalid("deltanet_prefill: negative position");
    if (!aligned16(state) || !aligned16(workspace)) return invalid("deltanet_prefill: alignment");
    if (workspace_bytes < 0 ||
        static_cast<size_t>(workspace_bytes) < hai_deltanet_prefill_workspace_bytes(B, T, nv, dv))
        return invalid("deltanet_prefill: workspace smaller than hai_deltanet_prefill_workspace_bytes");
    if (B == 0 || T == 0) return HAI_OK;
    PrefillArgs a{};
    a.o_ws = static_cast<float*>(workspace);
    a.proj = static_cast<const uint16_t*>(proj);
    a.ld_proj = ld_proj;
    a.off_qkv = off_qkv;
    a.off_a = off_a;
    a.off_b = off_b;
    a.conv_w = static_cast<const uint16_t*>(conv_w);
    a.ring = static_cast<uint16_t*>(conv_ring);
    a.ring_n = int(ring);
    a.nslots = int(nslots);
    a.state = state;
    a.a_log = static_cast<const uint16_t*>(a_log);
    a.dt_bias = static_cast<const uint16_t*>(dt_bias);
    a.lens = lens;
    a.pos_add = pos_add;
    a.B = int(B);
    a.T = int(T);
    a.nk = int(nk);
    a.nv = int(nv);
    a.Kc = int(Kc);
    auto* o = static_cast<uint16_t*>(out);
    const auto* nw = static_cast<const uint16_t*>(norm_w);
    const auto s = as_stream(stream);
    if (dk == 128 && dv == 128) return launch_prefill<128, 128>(a, o, ld_out, off_z, nw, eps, s);
    if (dk == 64 && dv == 64) return launch_prefill<64, 64>(a, o, ld_out, off_z, nw, eps, s);
    return invalid("deltanet_prefill: (dk, dv) must be (128,128) or (64,64)");
}
