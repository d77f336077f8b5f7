// hai_deltanet_prefill.hip -- Gated DeltaNet over prompt chunks (the
// prefill's deltanet_grouped_conv_kernel + deltanet_recurrent_kernel,
// hip_kernels.hip:871-912, 985-1095, and the gated RMSNorm), tolerance mode.
//
// The recurrence per token (v-head h; normalised key k_t, scaled query q_t,
// decay a_t, beta_t; S [dk][dv] fp32):
//   S_t = a_t S_{t-1} + beta_t k_t (v_t - a_t S_{t-1}^T k_t)^T,  o_t = S_t^T q_t.
// Walked token by token it is a chain of dependent dot products (~0.8 us
// per token and layer at the 27B shape).  Here the tokens go in chunks of
// kChunk and the recurrence is restated per chunk -- the chunkwise form of
// the gated delta rule (Yang, Kautz and Hatamizadeh, "Gated Delta Networks",
// 2024): with g_t = sum_{u<=t} log a_u inside the chunk, S the state before
// it, L[t][s] = beta_t e^{g_t - g_s} k_t.k_s (s < t) and w_t the value token
// t writes (S_t = a_t S_{t-1} + k_t w_t^T),
//   (I + L) w = diag(beta) V - diag(beta e^g) K S,   so   w = U - W^ S  with
//   U = (I + L)^-1 diag(beta) V,   W^ = (I + L)^-1 diag(beta e^g) K;
//   o_t = e^{g_t} S^T q_t + sum_{s<=t} e^{g_t - g_s} (q_t.k_s) w_s;
//   S'  = e^{g_last} S + sum_s e^{g_last - g_s} k_s w_s^T.
// Everything but the last two lines is independent of S, so the work splits
// into three launches:
//   1. deltanet_chunk_prep_kernel, one block per (chunk, head, sequence), all
//      chunks at once: conv + SiLU of the chunk's inputs, gates, q / k norms,
//      the Gram matrices (matrix cores), the triangular solve for U and W^
//      (one thread per right-hand column, in order of t), and the scaled keys
//      / queries K~ = e^{g_last - g} K, Q~ = e^{g} Q and P[t][s] =
//      e^{g_t - g_s} q_t.k_s into a per-chunk record, W^ / K~ / Q~ / P already
//      split into bf16 pairs in the operand order of the next pass;
//   2. deltanet_chunk_state_kernel, one block per (head, sequence), the chunks
//      in order: W = U - W^ S, O = Q~ S + P W, S = e^{g_last} S + K~^T W --
//      dense products on the matrix cores with the state held in their
//      accumulators, each record copied global -> LDS one chunk ahead;
//   3. deltanet_gated_norm_kernel: the gated RMSNorm per (token, head).
// The state is stored once, to slot (L + T) % nslots, and the conv ring's
// last entries by deltanet_ring_update_kernel.  The sums are reassociated
// (and the gates use the hardware exp), so results equal the canonical
// recurrence to fp32 rounding, not bit for bit.
#include "hai_common.h"
#include "hai_device.h"
#include "hai_gemm_common.h"

#include <atomic>


namespace {

using namespace hai;

constexpr int kChunk = 32;   // tokens per chunk
constexpr int kMaxKc = 8;

struct PrefillArgs {
    float* o_ws;            // [B*T][nv*dv] unrounded outputs
    float* chunks;          // per (sequence, head, chunk): chunk_floats<DK, DV>() floats
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

// Per-chunk record: U [C][DV], W^ [C][DK], K~ [C][DK], Q~ [C][DK], P [C][C],
// then e^{g_last} (padded to 16 floats).
template <int DK, int DV>
__host__ __device__ constexpr int64_t chunk_floats() {
    return static_cast<int64_t>(kChunk) * (DV + 3 * DK + kChunk) + 16;
}

// tolerance mode: the hardware exp and reciprocal
__device__ __forceinline__ float fast_silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// ---- matrix-core operands (v_mfma_f32_32x32x16_bf16) ----
typedef __bf16 dn_bf16x8 __attribute__((ext_vector_type(8)));
typedef float dn_f32x16 __attribute__((ext_vector_type(16)));

// Position in a 16-k step of the operand slot q (0..7) of lane half lh: the
// k index 16s + op_slot(lh, q) of step s sits in k-slot 8 lh + q.  Elements
// 8s .. 8s + 7 of a lane's 32x32 result tile hold rows 16s + op_slot(lh, q),
// so a result tile is the B operand of the next product as it stands.
__host__ __device__ constexpr int op_slot(int lh, int q) { return 4 * lh + (q & 3) + 8 * (q >> 2); }

// Operand tables: per 16-k step (or tile block) blk, the 64 lanes' 8 bf16 of
// the high parts, then of the low parts (x = hi + lo, hi = bf16(x),
// lo = bf16(x - hi)).  Word e = (blk * 64 + lane) * 4 + pair.
__device__ __forceinline__ void put_split(uint32_t* tab, int e, float x0, float x1) {
    const uint32_t hp = f2bf2(x0, x1);
    const int at = e + ((e >> 8) << 8);
    tab[at] = hp;
    tab[at + 256] = f2bf2(x0 - lo_bf(hp), x1 - hi_bf(hp));
}
// eight values, split the same way
__device__ __forceinline__ void dn_split8(const float (&x)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t hp = f2bf2(x[2 * q], x[2 * q + 1]);
        hi[q] = hp;
        lo[q] = f2bf2(x[2 * q] - lo_bf(hp), x[2 * q + 1] - hi_bf(hp));
    }
}
// elements off .. off + 7 of an accumulator tile, split the same way
__device__ __forceinline__ void dn_split8(const dn_f32x16& x, int off, u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t hp = f2bf2(x[off + 2 * q], x[off + 2 * q + 1]);
        hi[q] = hp;
        lo[q] = f2bf2(x[off + 2 * q] - lo_bf(hp), x[off + 2 * q + 1] - hi_bf(hp));
    }
}
// one global -> LDS copy of 16 bytes per lane (to lds + lane; lds wave-uniform)
__device__ __forceinline__ void dn_copy16(const u32x4* src, u32x4* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ dn_f32x16 dn_mfma(u32x4 a, u32x4 b, dn_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(dn_bf16x8, a), __builtin_bit_cast(dn_bf16x8, b),
                                                   c, 0, 0, 0);
}

// ---- pass 1: one block (256 threads) per (chunk c, head h, sequence b);
// KC: the conv taps (0: any count up to kMaxKc, read from the arguments) ----
template <int DK, int DV, int KC>
__global__ __launch_bounds__(256) void deltanet_chunk_prep_kernel(PrefillArgs A) {
    constexpr int KM = KC > 0 ? KC : kMaxKc;  // tap registers
    constexpr int NT = 256;
    constexpr int NW = NT / 64;
    constexpr int DKP = DK + 4;  // padded LDS rows (the Gram's column reads spread over banks)
    constexpr int NCH = 2 * DK + DV;
    constexpr int NRHS = DV + DK;
    static_assert(NRHS <= NT && NRHS >= kChunk, "one thread per right-hand column");
    __shared__ __align__(16) float qs[kChunk][DKP];
    __shared__ __align__(16) float ks[kChunk][DKP];
    __shared__ uint32_t vs2[kChunk][DV / 2];  // v as bf16 pairs (the conv output is bf16-exact)
    __shared__ __align__(16) float Lm[kChunk][kChunk + 4];  // rows read as float4
    __shared__ float Ps[kChunk][kChunk + 1];
    __shared__ float s_lg[kChunk], s_g[kChunk], s_beta[kChunk], s_q[kChunk], s_k[kChunk], s_ek[kChunk], s_eq[kChunk];

    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nv = A.nv;
    const int gq = h / (nv / A.nk);
    const int64_t kw = static_cast<int64_t>(A.nk) * DK;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t C = 2 * kw + vw;
    const int Kc = KC > 0 ? KC : A.Kc;
    const int hist = Kc - 1;
    const int T = A.T;
    const int t0 = c * kChunk;
    const int TS = min(kChunk, T - t0);
    const int64_t row0 = static_cast<int64_t>(b) * T;
    const int64_t p0 = static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;

    // ---- gate inputs (last wave, lane = token), requested first ----
    float a_in = 0.0f, b_in = 0.0f, dt_b = 0.0f, a_lg = 0.0f;
    if (wave == NW - 1 && lane < TS) {
        a_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_a + h]);
        b_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_b + h]);
        dt_b = bf2f(A.dt_bias[h]);
        a_lg = bf2f(A.a_log[h]);
    }
    // ---- conv + SiLU: thread p < NCH / 2 takes the channel pair 2p, 2p + 1
    // (within one of q, k, v: their widths are even); input at prompt-chunk
    // row t0 + tt - hist + i, rows before the prompt chunk from the conv ring
    // (positions before 0: zero).  Every load is issued before the first use.
    constexpr int NP = NCH / 2;
    static_assert(NCH % 2 == 0 && NP <= NT - 64, "channel pairs leave the last wave to the gates");
    if (tid < NP) {
        const int ch = 2 * tid;
        int64_t chan;
        if (ch < DK) chan = static_cast<int64_t>(gq) * DK + ch;
        else if (ch < 2 * DK) chan = kw + static_cast<int64_t>(gq) * DK + (ch - DK);
        else chan = 2 * kw + static_cast<int64_t>(h) * DV + (ch - 2 * DK);
        float wc0[KM], wc1[KM];
#pragma unroll
        for (int i = 0; i < KM; ++i) {
            wc0[i] = i < Kc ? bf2f(A.conv_w[chan * Kc + i]) : 0.0f;
            wc1[i] = i < Kc ? bf2f(A.conv_w[(chan + 1) * Kc + i]) : 0.0f;
        }
        auto pair_at = [&](const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); };
        uint32_t win[KM];  // the last Kc - 1 input pairs, oldest first
#pragma unroll
        for (int i = 0; i < KM; ++i) {
            uint32_t v = 0;
            if (i < hist) {
                const int r = t0 - hist + i;
                if (r >= 0) v = pair_at(A.proj + (row0 + r) * A.ld_proj + A.off_qkv + chan);
                else if (p0 + r >= 0)
                    v = pair_at(A.ring + (static_cast<int64_t>(b) * A.ring_n + (p0 + r) % A.ring_n) * C + chan);
            }
            win[i] = v;
        }
        uint32_t xr[kChunk];
#pragma unroll
        for (int tt = 0; tt < kChunk; ++tt)
            xr[tt] = tt < TS ? pair_at(A.proj + (row0 + t0 + tt) * A.ld_proj + A.off_qkv + chan) : 0u;
        float* col = ch < DK ? &qs[0][ch] : &ks[0][ch - DK];  // (q and k rows)
#pragma unroll
        for (int tt = 0; tt < kChunk; ++tt) {
            if (tt >= TS) continue;
            const uint32_t xin = xr[tt];
            float acc0 = lo_bf(hist > 0 ? win[0] : xin) * wc0[0];
            float acc1 = hi_bf(hist > 0 ? win[0] : xin) * wc1[0];
#pragma unroll
            for (int i = 1; i < KM; ++i) {
                if (i < hist) {
                    acc0 = fma_(lo_bf(win[i]), wc0[i], acc0);
                    acc1 = fma_(hi_bf(win[i]), wc1[i], acc1);
                } else if (i == hist) {
                    acc0 = fma_(lo_bf(xin), wc0[i], acc0);
                    acc1 = fma_(hi_bf(xin), wc1[i], acc1);
                }
            }
#pragma unroll
            for (int i = 0; i + 1 < KM; ++i)
                if (i + 1 < hist) win[i] = win[i + 1];
#pragma unroll
            for (int i = 0; i < KM; ++i)
                if (i == hist - 1) win[i] = xin;
            const float y0 = bfr(fast_silu(acc0)), y1 = bfr(fast_silu(acc1));
            if (ch < 2 * DK) *reinterpret_cast<float2*>(col + tt * DKP) = make_float2(y0, y1);
            else vs2[tt][(ch - 2 * DK) / 2] = f2bf2(y0, y1);
        }
    }
    // ---- gates: log of the decay exp(-exp(A_log) softplus(dt_bias + a)),
    // beta = sigmoid(b) ----
    if (wave == NW - 1 && lane < TS) {
        const float dtv = dt_b + a_in;
        const float sp = fmaxf(dtv, 0.0f) + log1pf(__expf(-fabsf(dtv)));
        s_lg[lane] = -(__expf(a_lg) * sp);
        s_beta[lane] = __builtin_amdgcn_rcpf(1.0f + __expf(-b_in));
    }
    __syncthreads();
    // ---- L2 norms of q and k (four threads per vector); cumulative log decay ----
    {
        static_assert(NT == 8 * kChunk && DK % 16 == 0, "four threads per q / k vector");
        const float rs_dk = 1.0f / csqrt(static_cast<float>(DK));
        const int vec = tid >> 2, part = tid & 3;
        const int t = vec >> 1;
        const float* x = ((vec & 1) ? ks[t] : qs[t]) + part * (DK / 4);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < DK / 4; k += 4) {
            const float4 v4 = *reinterpret_cast<const float4*>(x + k);
            acc = fma_(v4.x, v4.x, acc); acc = fma_(v4.y, v4.y, acc);
            acc = fma_(v4.z, v4.z, acc); acc = fma_(v4.w, v4.w, acc);
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        if (part == 0 && t < TS) {
            if (vec & 1) s_k[t] = 1.0f / csqrt(acc + 1.0e-6f);
            else s_q[t] = (1.0f / csqrt(acc + 1.0e-6f)) * rs_dk;
        }
    }
    if (tid == NT - 1) {
        float gg = 0.0f;
        for (int t = 0; t < TS; ++t) {
            gg += s_lg[t];
            s_g[t] = gg;
        }
    }
    __syncthreads();
    for (int e = tid; e < kChunk * DK; e += NT) {
        const int t = e / DK, d = e % DK;
        if (t < TS) {
            qs[t][d] = qs[t][d] * s_q[t];
            ks[t][d] = ks[t][d] * s_k[t];
        } else {
            qs[t][d] = 0.0f;  // rows past the chunk's tokens take no part
            ks[t][d] = 0.0f;
        }
    }
    for (int e = tid; e < (kChunk - TS) * (DV / 2); e += NT) vs2[TS + e / (DV / 2)][e % (DV / 2)] = 0u;
    const float glast = s_g[TS - 1];
    if (tid < kChunk) {
        const bool live = tid < TS;
        s_ek[tid] = live ? __expf(glast - s_g[tid]) : 0.0f;
        s_eq[tid] = live ? __expf(s_g[tid]) : 0.0f;
    }
    __syncthreads();

    float* rec = A.chunks + ((static_cast<int64_t>(b) * nv + h) * ((T + kChunk - 1) / kChunk) + c) * chunk_floats<DK, DV>();
    float* rU = rec;
    uint32_t* rW = reinterpret_cast<uint32_t*>(rU + kChunk * DV);
    uint32_t* rK = rW + kChunk * DK;
    uint32_t* rQ = rK + kChunk * DK;
    uint32_t* rP = rQ + kChunk * DK;

    // ---- Gram matrices on the matrix cores: wave 0 K K^T, wave 1 Q K^T, each
    // over all of d in 16-wide k steps (k slot q of lane l: d = 16 step +
    // 8 (l / 32) + q; K's row t is the A operand and its column t the B
    // operand in the same registers); result element i of lane l: row
    // t = 8 (i / 4) + 4 (l / 32) + i % 4, key s = l % 32 ----
    if (wave < 2) {
        const int r = lane & 31;
        const float* arow = wave == 0 ? ks[r] : qs[r];
        dn_f32x16 G;
#pragma unroll
        for (int i = 0; i < 16; ++i) G[i] = 0.0f;
#pragma unroll
        for (int kst = 0; kst < DK / 16; ++kst) {
            const int d0 = 16 * kst + 8 * (lane >> 5);
            const float4 k0 = *reinterpret_cast<const float4*>(&ks[r][d0]);
            const float4 k1 = *reinterpret_cast<const float4*>(&ks[r][d0 + 4]);
            const float4 a0 = *reinterpret_cast<const float4*>(arow + d0);
            const float4 a1 = *reinterpret_cast<const float4*>(arow + d0 + 4);
            const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            u32x4 kh, kl, ah, al;
            dn_split8(kv, kh, kl);
            dn_split8(av, ah, al);
            G = dn_mfma(al, kh, G);
            G = dn_mfma(ah, kl, G);
            G = dn_mfma(ah, kh, G);
        }
        const int sc = lane & 31;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            const bool live = t < TS && sc < TS && sc <= t;
            const float ratio = live ? __expf(s_g[t] - s_g[sc]) : 0.0f;
            if (wave == 0) Lm[t][sc] = (live && sc < t) ? s_beta[t] * ratio * G[i] : 0.0f;
            else Ps[t][sc] = ratio * G[i];
        }
    }
    __syncthreads();

    // ---- K~ = e^{g_last - g} K, Q~ = e^{g} Q and P, split, in operand order ----
    for (int e = tid; e < 16 * DK; e += NT) {
        const int qp = e & 3, ln = (e >> 2) & 63, blk = e >> 8;
        const int t = ln & 31, r0 = op_slot(ln >> 5, 2 * qp);
        const int kq = 16 * blk + r0;  // Q~ (A of Q~ S): token t, keys kq, kq + 1
        put_split(rQ, e, s_eq[t] * qs[t][kq], s_eq[t] * qs[t][kq + 1]);
        const int kk = 32 * (blk >> 1) + t;  // K~ (A of K~^T w): key kk, tokens tk, tk + 1
        const int tk = 16 * (blk & 1) + r0;
        put_split(rK, e, s_ek[tk] * ks[tk][kk], s_ek[tk + 1] * ks[tk + 1][kk]);
    }
    for (int e = tid; e < 16 * kChunk; e += NT) {
        const int qp = e & 3, ln = (e >> 2) & 63, blk = e >> 8;
        const int t = ln & 31, sc = 16 * blk + op_slot(ln >> 5, 2 * qp);
        put_split(rP, e, Ps[t][sc], Ps[t][sc + 1]);
    }
    if (tid == 0) rP[kChunk * kChunk] = __float_as_uint(__expf(glast));
    __syncthreads();  // qs is reused for W^

    // ---- (I + L) X = R by forward substitution, one thread per right-hand
    // column: R = beta * V (U, to the record) or beta e^g K (W^, to LDS) ----
    float (*Xw)[DKP] = qs;
    if (tid < NRHS) {
        float x[kChunk];
        const bool isv = tid < DV;
        const int col = isv ? tid : tid - DV;
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            float acc = 0.0f;
            if (t < TS) {
                // four partial sums (s = u mod 4) shorten the dependent chain
                float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s4 = 0; s4 < t; s4 += 4) {
                    const float4 l4 = *reinterpret_cast<const float4*>(&Lm[t][s4]);
                    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (s4 + u < t) part[u] = fma_(-lv[u], x[s4 + u], part[u]);
                }
                const uint32_t vp = vs2[t][col >> 1];
                acc = isv ? s_beta[t] * ((col & 1) ? hi_bf(vp) : lo_bf(vp)) : (s_beta[t] * __expf(s_g[t])) * ks[t][col];
                acc += (part[0] + part[1]) + (part[2] + part[3]);
            }
            x[t] = acc;
        }
        if (isv) {
#pragma unroll
            for (int t = 0; t < kChunk; ++t) rU[t * DV + col] = x[t];
        } else {
#pragma unroll
            for (int t = 0; t < kChunk; ++t) Xw[t][col] = x[t];
        }
    }
    __syncthreads();
    for (int e = tid; e < 16 * DK; e += NT) {  // W^ (A of W^ S): token t, keys kw, kw + 1
        const int qp = e & 3, ln = (e >> 2) & 63, blk = e >> 8;
        const int t = ln & 31, kw2 = 16 * blk + op_slot(ln >> 5, 2 * qp);
        put_split(rW, e, Xw[t][kw2], Xw[t][kw2 + 1]);
    }
}

// ---- pass 2 on the matrix cores: one block per (head h, sequence b), one
// wave per 32 value columns, the chunks in order ----
// The state columns of a wave are DK/32 accumulator tiles of
// v_mfma_f32_32x32x16_bf16: tile m, lane l, element i holds
// S[32m + 8(i/4) + 4(l/32) + i%4][j0 + l%32], so elements 8s .. 8s + 7 of a
// tile are the B operand of the 16-k step over keys 32m + 16s + op_slot(.):
// W^ S and Q~ S take S straight from the accumulators, and w = U - W^ S comes
// out in the layout that makes it, in turn, the B operand of P w and K~^T w.
// The A operands (W^, Q~, K~, P) are written by pass 1 in exactly that order,
// split into bf16 pairs; every fp32 product is hi.hi + hi.lo + lo.hi (the
// small terms first), within ~2^-16 of it.
// Records reach LDS by global -> LDS copies (16 bytes per lane, no
// registers), one chunk ahead into the other of two buffers; each wave issues
// the same number of copies per chunk (pieces past the record repeat its
// last piece into the buffer's tail), so s_waitcnt vmcnt(kCopies) leaves
// exactly the next chunk's copies in flight.
template <int DK, int DV>
__host__ __device__ constexpr int state_copies() {  // copy instructions per wave per chunk
    return static_cast<int>((chunk_floats<DK, DV>() / 4 + 64 * (DV / 32) - 1) / (64 * (DV / 32)));
}
template <int DK, int DV>
__host__ __device__ constexpr size_t state_lds_bytes() {  // two record buffers
    return 2 * static_cast<size_t>(state_copies<DK, DV>()) * 64 * (DV / 32) * 16;
}

template <int DK, int DV>
__global__ __launch_bounds__(64 * (DV / 32)) void deltanet_chunk_state_kernel(PrefillArgs A) {
    constexpr int NW = DV / 32;
    constexpr int NT = 64 * NW;
    constexpr int MT = DK / 32;                             // state tiles per wave
    constexpr int RW = 3 * kChunk * DK + kChunk * kChunk;  // operand words of a record
    constexpr int NPC = static_cast<int>(chunk_floats<DK, DV>() / 4);  // 16-byte pieces of a record
    constexpr int kCopies = state_copies<DK, DV>();
    constexpr int BUF = kCopies * NT;                       // pieces per buffer
    static_assert(DK % 32 == 0 && DV % 32 == 0 && kChunk == 32 && chunk_floats<DK, DV>() % 4 == 0 && kCopies < 48,
                  "state pass tiles");
    extern __shared__ __align__(16) u32x4 recs[];  // [2][BUF]: U [C][DV] f32, operands, e^{g_last}

    const int h = blockIdx.x;
    const int b = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int w = wave_index();
    const int j0 = 32 * w;
    const int lc = lane & 31;
    const int lh = lane >> 5;
    const int nv = A.nv;
    const int T = A.T;
    const int nchunks = (T + kChunk - 1) / kChunk;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t row0 = static_cast<int64_t>(b) * T;
    const int64_t p0 = static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;
    auto row_of = [&](int i) { return 8 * (i >> 2) + 4 * lh + (i & 3); };
    // column-tiled head: key i = q4*(DK/4) + 4m + e of column j at float ((m*DV + j)*4 + q4)*4 + e
    auto tiled = [&](int key, int col) {
        const int q4 = key / (DK / 4), m = (key % (DK / 4)) / 4, ee = key % 4;
        return ((static_cast<int64_t>(m) * DV + col) * 4 + q4) * 4 + ee;
    };
    const u32x4* recs0 = reinterpret_cast<const u32x4*>(A.chunks) +
                         (static_cast<int64_t>(b) * nv + h) * nchunks * static_cast<int64_t>(NPC);
    // pieces (i * NW + w) * 64 + lane: in the record for i < kCopies - 1
    static_assert((kCopies - 1) * NT < NPC, "only the last copy runs past the record");
    const int last_piece = min(((kCopies - 1) * NW + w) * 64 + lane, NPC - 1) - ((kCopies - 1) * NW + w) * 64;
    auto copy_record = [&](int ci, int buf) {
        const u32x4* src = recs0 + static_cast<int64_t>(min(ci, nchunks - 1)) * NPC + w * 64;
        u32x4* dst = recs + buf * BUF + w * 64;
#pragma unroll
        for (int i = 0; i < kCopies - 1; ++i) dn_copy16(src + i * NT + lane, dst + i * NT);
        dn_copy16(src + (kCopies - 1) * NT + last_piece, dst + (kCopies - 1) * NT);
    };

    const float* hs = A.state + ((p0 % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                      static_cast<int64_t>(h) * DV * DK;
    dn_f32x16 S[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) S[m][i] = hs[tiled(32 * m + row_of(i), j0 + lc)];
    pin_memory_order();
    copy_record(0, 0);

    for (int c = 0; c < nchunks; ++c) {
        const int t0 = c * kChunk;
        const int TS = min(kChunk, T - t0);
        const int cur = c & 1;
        pin_memory_order();
        __builtin_amdgcn_sched_barrier(0);
        copy_record(c + 1, cur ^ 1);  // (the last chunk copies itself again into the idle buffer)
        pin_memory_order();
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kCopies>();  // this chunk's copies (and every older request) are done
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();          // ... for every wave
        const float* rf = reinterpret_cast<const float*>(recs + cur * BUF);
        const u32x4* opW = reinterpret_cast<const u32x4*>(rf + kChunk * DV);
        const u32x4* opK = opW + kChunk * DK / 4;
        const u32x4* opQ = opK + kChunk * DK / 4;
        const u32x4* opP = opQ + kChunk * DK / 4;
        // ---- W^ S and Q~ S (row t = lane % 32 of the A operands) ----
        dn_f32x16 Wa, Oa;
#pragma unroll
        for (int i = 0; i < 16; ++i) Wa[i] = Oa[i] = 0.0f;
        // (the next step's operands are read from LDS before this step's products)
        u32x4 nwh = opW[lane], nwl = opW[64 + lane], nqh = opQ[lane], nql = opQ[64 + lane];
#pragma unroll
        for (int ks = 0; ks < 2 * MT; ++ks) {
            const u32x4 wh = nwh, wl = nwl, qh = nqh, ql = nql;
            if (ks + 1 < 2 * MT) {
                nwh = opW[(2 * ks + 2) * 64 + lane];
                nwl = opW[(2 * ks + 3) * 64 + lane];
                nqh = opQ[(2 * ks + 2) * 64 + lane];
                nql = opQ[(2 * ks + 3) * 64 + lane];
            }
            u32x4 bh, bl;
            dn_split8(S[ks >> 1], 8 * (ks & 1), bh, bl);
            Wa = dn_mfma(wl, bh, Wa);
            Oa = dn_mfma(ql, bh, Oa);
            Wa = dn_mfma(wh, bl, Wa);
            Oa = dn_mfma(qh, bl, Oa);
            Wa = dn_mfma(wh, bh, Wa);
            Oa = dn_mfma(qh, bh, Oa);
        }
        // ---- w = U - W^ S, then O = Q~ S + P w ----
#pragma unroll
        for (int i = 0; i < 16; ++i) Wa[i] = rf[row_of(i) * DV + j0 + lc] - Wa[i];
        u32x4 wh[2], wl[2];
        dn_split8(Wa, 0, wh[0], wl[0]);
        dn_split8(Wa, 8, wh[1], wl[1]);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const u32x4 ph = opP[(2 * st) * 64 + lane], pl = opP[(2 * st + 1) * 64 + lane];
            Oa = dn_mfma(pl, wh[st], Oa);
            Oa = dn_mfma(ph, wl[st], Oa);
            Oa = dn_mfma(ph, wh[st], Oa);
        }
        float* orow = A.o_ws + (row0 + t0) * vw + static_cast<int64_t>(h) * DV + j0 + lc;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (row_of(i) < TS) orow[row_of(i) * vw] = Oa[i];
        // ---- S = e^{g_last} S + K~^T w (row = key 32m + lane % 32, k = tokens) ----
        const float gl = rf[kChunk * DV + RW];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int i = 0; i < 16; ++i) S[m][i] *= gl;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const u32x4 kh = opK[(4 * m + 2 * st) * 64 + lane], kl = opK[(4 * m + 2 * st + 1) * 64 + lane];
                S[m] = dn_mfma(kl, wh[st], S[m]);
                S[m] = dn_mfma(kh, wl[st], S[m]);
                S[m] = dn_mfma(kh, wh[st], S[m]);
            }
        }
        lds_barrier();  // every wave's reads of this buffer are done before it is refilled
    }
    wait_vmcnt<0>();
    float* hd = A.state + (((p0 + T) % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                static_cast<int64_t>(h) * DV * DK;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) hd[tiled(32 * m + row_of(i), j0 + lc)] = S[m][i];
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
    const unsigned nchunks = static_cast<unsigned>((a.T + kChunk - 1) / kChunk);
    const dim3 pgrid(nchunks, a.nv, a.B);
    if (a.Kc == 4) deltanet_chunk_prep_kernel<DK, DV, 4><<<pgrid, dim3(256), 0, s>>>(a);
    else if (a.Kc == 3) deltanet_chunk_prep_kernel<DK, DV, 3><<<pgrid, dim3(256), 0, s>>>(a);
    else deltanet_chunk_prep_kernel<DK, DV, 0><<<pgrid, dim3(256), 0, s>>>(a);
    int rc = launched("deltanet_chunk_prep_kernel");
    if (rc != HAI_OK) return rc;
    constexpr size_t shmem = state_lds_bytes<DK, DV>();
    static std::atomic<uint8_t> allowed[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return invalid("deltanet_prefill: device ordinal");
    if (!allowed[dev].load(std::memory_order_acquire)) {
        rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(deltanet_chunk_state_kernel<DK, DV>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(shmem)),
                       "hipFuncSetAttribute");
        if (rc != HAI_OK) return rc;
        allowed[dev].store(1, std::memory_order_release);
    }
    deltanet_chunk_state_kernel<DK, DV><<<dim3(a.nv, 1, a.B), dim3(64 * (DV / 32)), shmem, s>>>(a);
    rc = launched("deltanet_chunk_state_kernel");
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

// The unrounded outputs [B*T][nv*dv], then the per-chunk records (dk = dv).
static size_t chunk_record_bytes(int64_t B, int64_t T, int64_t nv, int64_t dv) {
    const int64_t per = dv == 64 ? chunk_floats<64, 64>() : chunk_floats<128, 128>();
    return static_cast<size_t>(B * nv * ((T + kChunk - 1) / kChunk) * per) * sizeof(float);
}
static size_t output_bytes(int64_t B, int64_t T, int64_t nv, int64_t dv) {
    return (static_cast<size_t>(B * T * nv * dv) * sizeof(float) + 255) / 256 * 256;
}

extern "C" size_t hai_deltanet_prefill_workspace_bytes(int64_t B, int64_t T, int64_t nv, int64_t dv) {
    if (B < 0 || T < 0 || nv < 0 || dv < 0) return 0;
    return output_bytes(B, T, nv, dv) + chunk_record_bytes(B, T, nv, dv);
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
    // the conv reads channel pairs as one dword
    if ((reinterpret_cast<uintptr_t>(proj) & 3u) != 0 || (reinterpret_cast<uintptr_t>(conv_ring) & 3u) != 0 ||
        (ld_proj & 1) != 0 || (off_qkv & 1) != 0)
        return invalid("deltanet_prefill: proj and conv_ring must be 4-byte aligned, ld_proj and off_qkv even");
    if (workspace_bytes < 0 ||
        static_cast<size_t>(workspace_bytes) < hai_deltanet_prefill_workspace_bytes(B, T, nv, dv))
        return invalid("deltanet_prefill: workspace smaller than hai_deltanet_prefill_workspace_bytes");
    if (B == 0 || T == 0) return HAI_OK;
    PrefillArgs a{};
    a.o_ws = static_cast<float*>(workspace);
    a.chunks = reinterpret_cast<float*>(static_cast<char*>(workspace) + output_bytes(B, T, nv, dv));
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
