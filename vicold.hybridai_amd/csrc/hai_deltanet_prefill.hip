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
//      the Gram matrices, the triangular solve for U and W^ (one thread per
//      right-hand column, in order of t), and the scaled keys / queries
//      K~ = e^{g_last - g} K, Q~ = e^{g} Q and P[t][s] = e^{g_t - g_s} q_t.k_s
//      into a workspace;
//   2. deltanet_chunk_state_kernel, one block per (head, 32 value columns,
//      sequence), the chunks in order: W = U - W^ S, O = Q~ S + P W,
//      S = e^{g_last} S + K~^T W -- three dense products per chunk, the state
//      in LDS;
//   3. deltanet_gated_norm_kernel: the gated RMSNorm per (token, head).
// The state is stored once, to slot (L + T) % nslots, and the conv ring's
// last entries by deltanet_ring_update_kernel.  The sums are reassociated
// (and the gates use the hardware exp), so results equal the canonical
// recurrence to fp32 rounding, not bit for bit.
#include "hai_common.h"
#include "hai_device.h"

#include <atomic>

namespace {

using namespace hai;

constexpr int kChunk = 32;   // tokens per chunk
// value columns per block of the state pass (every block loads its chunk's
// whole record: 16 columns per block measured slower than 32 on MI355X,
// 307 against 207 us per 1024-token call at the 27B shape)
template <int DK>
constexpr int state_cols() { return 32; }
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
    __shared__ float vs[kChunk][DV];
    __shared__ __align__(16) float Lm[kChunk][kChunk + 4];  // rows read as float4
    __shared__ float s_lg[kChunk], s_g[kChunk], s_beta[kChunk], s_q[kChunk], s_k[kChunk];

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

    // ---- conv + SiLU: input at prompt-chunk row t0 + tt - hist + i, rows
    // before the prompt chunk from the conv ring (positions before 0: zero) ----
    for (int ch = tid; ch < NCH; ch += NT) {
        int64_t chan;
        if (ch < DK) chan = static_cast<int64_t>(gq) * DK + ch;
        else if (ch < 2 * DK) chan = kw + static_cast<int64_t>(gq) * DK + (ch - DK);
        else chan = 2 * kw + static_cast<int64_t>(h) * DV + (ch - 2 * DK);
        float wc[KM];
#pragma unroll
        for (int i = 0; i < KM; ++i) wc[i] = i < Kc ? bf2f(A.conv_w[chan * Kc + i]) : 0.0f;
        float win[KM];  // the last Kc - 1 inputs, oldest first
#pragma unroll
        for (int i = 0; i < KM; ++i) {
            float v = 0.0f;
            if (i < hist) {
                const int r = t0 - hist + i;
                if (r >= 0) v = bf2f(A.proj[(row0 + r) * A.ld_proj + A.off_qkv + chan]);
                else if (p0 + r >= 0)
                    v = bf2f(A.ring[(static_cast<int64_t>(b) * A.ring_n + (p0 + r) % A.ring_n) * C + chan]);
            }
            win[i] = v;
        }
        uint16_t xr[kChunk];  // every input of the chunk requested before the first use
#pragma unroll
        for (int tt = 0; tt < kChunk; ++tt)
            xr[tt] = tt < TS ? A.proj[(row0 + t0 + tt) * A.ld_proj + A.off_qkv + chan] : uint16_t{0};
#pragma unroll
        for (int tt = 0; tt < kChunk; ++tt) {
            if (tt >= TS) continue;
            const float xin = bf2f(xr[tt]);
            float acc = (hist > 0 ? win[0] : xin) * wc[0];
#pragma unroll
            for (int i = 1; i < KM; ++i) {
                if (i < hist) acc = fma_(win[i], wc[i], acc);
                else if (i == hist) acc = fma_(xin, wc[i], acc);
            }
#pragma unroll
            for (int i = 0; i + 1 < KM; ++i)
                if (i + 1 < hist) win[i] = win[i + 1];
#pragma unroll
            for (int i = 0; i < KM; ++i)
                if (i == hist - 1) win[i] = xin;
            const float y = bfr(fast_silu(acc));
            if (ch < DK) qs[tt][ch] = y;
            else if (ch < 2 * DK) ks[tt][ch - DK] = y;
            else vs[tt][ch - 2 * DK] = y;
        }
    }
    // ---- gates (last wave, lane = token): log of the decay
    // exp(-exp(A_log) softplus(dt_bias + a)), beta = sigmoid(b) ----
    if (wave == NW - 1 && lane < TS) {
        const float a_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_a + h]);
        const float b_in = bf2f(A.proj[(row0 + t0 + lane) * A.ld_proj + A.off_b + h]);
        const float dtv = bf2f(A.dt_bias[h]) + a_in;
        const float sp = fmaxf(dtv, 0.0f) + log1pf(__expf(-fabsf(dtv)));
        s_lg[lane] = -(__expf(bf2f(A.a_log[h])) * sp);
        s_beta[lane] = __builtin_amdgcn_rcpf(1.0f + __expf(-b_in));
    }
    __syncthreads();
    // ---- L2 norms of q and k (one wave per vector); cumulative log decay ----
    const float rs_dk = 1.0f / csqrt(static_cast<float>(DK));
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
    for (int e = tid; e < (kChunk - TS) * DV; e += NT) vs[TS + e / DV][e % DV] = 0.0f;
    __syncthreads();

    float* rec = A.chunks + ((static_cast<int64_t>(b) * nv + h) * ((T + kChunk - 1) / kChunk) + c) * chunk_floats<DK, DV>();
    float* rU = rec;
    float* rW = rU + kChunk * DV;
    float* rK = rW + kChunk * DK;
    float* rQ = rK + kChunk * DK;
    float* rP = rQ + kChunk * DK;
    const float glast = s_g[TS - 1];

    // ---- Gram matrices: thread (t4 = tid / 32, s = tid % 32) takes rows
    // t4, t4 + 8, t4 + 16, t4 + 24 against key s ----
    {
        const int sc = tid % kChunk;
        const int t4 = tid / kChunk;
        float kk[4] = {0.0f, 0.0f, 0.0f, 0.0f}, qk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int d = 0; d < DK; d += 4) {
            const float4 c4 = *reinterpret_cast<const float4*>(&ks[sc][d]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 a4 = *reinterpret_cast<const float4*>(&ks[t4 + 8 * r][d]);
                const float4 b4 = *reinterpret_cast<const float4*>(&qs[t4 + 8 * r][d]);
                kk[r] = fma_(a4.x, c4.x, kk[r]); kk[r] = fma_(a4.y, c4.y, kk[r]);
                kk[r] = fma_(a4.z, c4.z, kk[r]); kk[r] = fma_(a4.w, c4.w, kk[r]);
                qk[r] = fma_(b4.x, c4.x, qk[r]); qk[r] = fma_(b4.y, c4.y, qk[r]);
                qk[r] = fma_(b4.z, c4.z, qk[r]); qk[r] = fma_(b4.w, c4.w, qk[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t4 + 8 * r;
            const bool live = t < TS && sc < TS && sc <= t;
            const float ratio = live ? __expf(s_g[t] - s_g[sc]) : 0.0f;
            Lm[t][sc] = (live && sc < t) ? s_beta[t] * ratio * kk[r] : 0.0f;
            rP[t * kChunk + sc] = ratio * qk[r];
        }
    }
    __syncthreads();

    // ---- (I + L) X = R by forward substitution, one thread per right-hand
    // column: R = beta * V (U) or beta e^g K (W^) ----
    if (tid < NRHS) {
        float x[kChunk];
        const bool isv = tid < DV;
        const int col = isv ? tid : tid - DV;
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            float acc = 0.0f;
            if (t < TS) {
                acc = isv ? s_beta[t] * vs[t][col] : (s_beta[t] * __expf(s_g[t])) * ks[t][col];
#pragma unroll
                for (int s4 = 0; s4 < t; s4 += 4) {
                    const float4 l4 = *reinterpret_cast<const float4*>(&Lm[t][s4]);
                    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (s4 + u < t) acc = fma_(-lv[u], x[s4 + u], acc);
                }
            }
            x[t] = acc;
        }
        float* dst = isv ? rU + col : rW + col;
        const int ld = isv ? DV : DK;
#pragma unroll
        for (int t = 0; t < kChunk; ++t) dst[t * ld] = x[t];
    }
    // ---- K~ = e^{g_last - g} K and Q~ = e^{g} Q ----
    for (int e = tid; e < kChunk * DK; e += NT) {
        const int t = e / DK, d = e % DK;
        const bool live = t < TS;
        rK[e] = live ? __expf(glast - s_g[t]) * ks[t][d] : 0.0f;
        rQ[e] = live ? __expf(s_g[t]) * qs[t][d] : 0.0f;
    }
    if (tid == 0) rP[kChunk * kChunk] = __expf(glast);
}

// ---- pass 2: one block (512 threads) per (head h, 32 value columns, sequence b),
// the chunks in order ----
// LDS of the state pass: the block's state columns, the chunk's w, and the
// chunk's record (W^, K~, Q~, P, e^{g_last}; the block's U columns).
template <int DK>
__host__ __device__ constexpr size_t state_lds_floats() {
    constexpr int kCols = state_cols<DK>();
    return static_cast<size_t>(kCols) * (DK + 4) + kChunk * (kCols + 1) + (3 * kChunk * DK + kChunk * kChunk + 16) +
           kChunk * kCols;
}

template <int DK, int DV>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void deltanet_chunk_state_kernel(PrefillArgs A) {
    constexpr int NT = 512;
    constexpr int DKP = DK + 4;
    constexpr int kCols = state_cols<DK>();
    constexpr int TPC = NT / kCols;             // threads per column
    constexpr int RPT = kChunk / TPC;           // rows of W / O per thread
    constexpr int IB = DK / TPC;                // state keys per thread in the update
    static_assert(RPT * TPC == kChunk && IB % 4 == 0, "state pass layout");
    constexpr int RF = 3 * kChunk * DK + kChunk * kChunk + 16;  // W^ .. e^{g_last} of a record
    extern __shared__ __align__(16) float lds_f[];
    float (*St)[DKP] = reinterpret_cast<float (*)[DKP]>(lds_f);                         // St[j][i] = S[i][j0 + j]
    float (*Wm)[kCols + 1] = reinterpret_cast<float (*)[kCols + 1]>(lds_f + kCols * DKP);
    float* Rs = lds_f + kCols * DKP + kChunk * (kCols + 1);                              // the record from W^ on
    float (*Us)[kCols] = reinterpret_cast<float (*)[kCols]>(Rs + RF);                    // U of the block's columns

    const int h = blockIdx.x;
    const int j0 = blockIdx.y * kCols;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int nv = A.nv;
    const int T = A.T;
    const int nchunks = (T + kChunk - 1) / kChunk;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t row0 = static_cast<int64_t>(b) * T;
    const int64_t p0 = static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;
    const int jc = tid % kCols;   // column of the products
    const int tg = tid / kCols;   // rows tg + TPC r (W, O), key block tg (update)

    // state of the block's columns from slot p0 % nslots (column-tiled head:
    // key i = q4*(DK/4) + 4m + e of column j at float ((m*DV + j)*4 + q4)*4 + e)
    const float* hs = A.state + ((p0 % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                      static_cast<int64_t>(h) * DV * DK;
    for (int e = tid; e < kCols * DK; e += NT) {
        const int jl = e / DK, i = e % DK;
        const int q4 = i / (DK / 4), m = (i % (DK / 4)) / 4, ee = i % 4;
        St[jl][i] = hs[((static_cast<int64_t>(m) * DV + j0 + jl) * 4 + q4) * 4 + ee];
    }
    __syncthreads();

    // A chunk's record goes through registers: the next chunk's loads are
    // issued before the current chunk is computed, and stored to LDS after it.
    constexpr int RP = (RF / 4 + NT - 1) / NT;   // record float4 per thread
    constexpr int UP = (kChunk * kCols / 4 + NT - 1) / NT;
    static_assert(RP <= 8 && UP == 1, "record pieces per thread");
    u32x4 rr[RP], ur;  // native vectors (HIP's float4 struct stays in memory here)
    // (unrolled by hand, up to 8 pieces: indices the compiler sees as constants
    // keep rr / ur in registers)
#define HAI_REC_LOAD1(U)                                                                                         \
    if constexpr (RP > (U)) {                                                                                    \
        const int e = tid + (U) * NT;                                                                            \
        if (e < RF / 4) rr[(U) < RP ? (U) : 0] = src_[e];                                                        \
    }
#define HAI_LOAD_RECORD(CI)                                                                                      \
    do {                                                                                                         \
        const float* rec_ = A.chunks + ((static_cast<int64_t>(b) * nv + h) * nchunks + (CI)) * chunk_floats<DK, DV>(); \
        const u32x4* src_ = reinterpret_cast<const u32x4*>(rec_ + kChunk * DV);                                \
        HAI_REC_LOAD1(0) HAI_REC_LOAD1(1) HAI_REC_LOAD1(2) HAI_REC_LOAD1(3)                                      \
        HAI_REC_LOAD1(4) HAI_REC_LOAD1(5) HAI_REC_LOAD1(6) HAI_REC_LOAD1(7)                                      \
        if (tid < kChunk * kCols / 4) {                                                                          \
            const int t_ = tid / (kCols / 4), q_ = tid % (kCols / 4);                                            \
            ur = *reinterpret_cast<const u32x4*>(rec_ + t_ * DV + j0 + 4 * q_);                                 \
        }                                                                                                        \
    } while (0)
    HAI_LOAD_RECORD(0);
    for (int c = 0; c < nchunks; ++c) {
        const int t0 = c * kChunk;
        const int TS = min(kChunk, T - t0);
#define HAI_REC_STORE1(U)                                                                                        \
    if constexpr (RP > (U)) {                                                                                    \
        const int e = tid + (U) * NT;                                                                            \
        if (e < RF / 4) reinterpret_cast<u32x4*>(Rs)[e] = rr[(U) < RP ? (U) : 0];                                \
    }
        HAI_REC_STORE1(0) HAI_REC_STORE1(1) HAI_REC_STORE1(2) HAI_REC_STORE1(3)
        HAI_REC_STORE1(4) HAI_REC_STORE1(5) HAI_REC_STORE1(6) HAI_REC_STORE1(7)
#undef HAI_REC_STORE1
        if (tid < kChunk * kCols / 4) reinterpret_cast<u32x4*>(&Us[0][0])[tid] = ur;
        __syncthreads();
        if (c + 1 < nchunks) HAI_LOAD_RECORD(c + 1);
        const float* rW = Rs;
        const float* rK = rW + kChunk * DK;
        const float* rQ = rK + kChunk * DK;
        const float* rP = rQ + kChunk * DK;
        // ---- W = U - W^ S and Q~ S for rows tg + TPC r of column jc ----
        float wv[RPT], ov[RPT];
#pragma unroll
        for (int r = 0; r < RPT; ++r) wv[r] = ov[r] = 0.0f;
#pragma unroll 4
        for (int i = 0; i < DK; i += 4) {
            const float4 s4 = *reinterpret_cast<const float4*>(&St[jc][i]);
#pragma unroll
            for (int r = 0; r < RPT; ++r) {
                const float4 x4 = *reinterpret_cast<const float4*>(rW + (tg + TPC * r) * DK + i);
                const float4 y4 = *reinterpret_cast<const float4*>(rQ + (tg + TPC * r) * DK + i);
                wv[r] = fma_(x4.x, s4.x, wv[r]); wv[r] = fma_(x4.y, s4.y, wv[r]);
                wv[r] = fma_(x4.z, s4.z, wv[r]); wv[r] = fma_(x4.w, s4.w, wv[r]);
                ov[r] = fma_(y4.x, s4.x, ov[r]); ov[r] = fma_(y4.y, s4.y, ov[r]);
                ov[r] = fma_(y4.z, s4.z, ov[r]); ov[r] = fma_(y4.w, s4.w, ov[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < RPT; ++r) Wm[tg + TPC * r][jc] = Us[tg + TPC * r][jc] - wv[r];
        __syncthreads();
        // ---- outputs O = Q~ S + P W ----
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int t = tg + TPC * r;
            if (t < TS) {
                float o = ov[r];
                const float* pr = rP + t * kChunk;
                for (int s2 = 0; s2 <= t; ++s2) o = fma_(pr[s2], Wm[s2][jc], o);
                A.o_ws[(row0 + t0 + t) * vw + static_cast<int64_t>(h) * DV + j0 + jc] = o;
            }
        }
        // ---- S = e^{g_last} S + K~^T W: thread (tg, jc) updates keys tg*IB .. + IB - 1 ----
        {
            const float gl = rP[kChunk * kChunk];
            float sv[IB];
#pragma unroll
            for (int u = 0; u < IB; u += 4) {
                const float4 s4 = *reinterpret_cast<const float4*>(&St[jc][tg * IB + u]);
                sv[u] = s4.x * gl; sv[u + 1] = s4.y * gl; sv[u + 2] = s4.z * gl; sv[u + 3] = s4.w * gl;
            }
            for (int t = 0; t < TS; ++t) {
                const float wt = Wm[t][jc];
                const float* kr = rK + t * DK + tg * IB;
#pragma unroll
                for (int u = 0; u < IB; u += 4) {
                    const float4 k4 = *reinterpret_cast<const float4*>(kr + u);
                    sv[u] = fma_(k4.x, wt, sv[u]); sv[u + 1] = fma_(k4.y, wt, sv[u + 1]);
                    sv[u + 2] = fma_(k4.z, wt, sv[u + 2]); sv[u + 3] = fma_(k4.w, wt, sv[u + 3]);
                }
            }
            __syncthreads();  // every thread's reads of S and W for this chunk are done
#pragma unroll
            for (int u = 0; u < IB; u += 4)
                *reinterpret_cast<float4*>(&St[jc][tg * IB + u]) = make_float4(sv[u], sv[u + 1], sv[u + 2], sv[u + 3]);
        }
        __syncthreads();
    }
    // ---- the state after the prompt chunk, to slot (p0 + T) % nslots ----
    float* hd = A.state + (((p0 + T) % A.nslots) * A.B + b) * static_cast<int64_t>(nv) * DV * DK +
                static_cast<int64_t>(h) * DV * DK;
    for (int e = tid; e < kCols * DK; e += NT) {
        const int jl = e / DK, i = e % DK;
        const int q4 = i / (DK / 4), m = (i % (DK / 4)) / 4, ee = i % 4;
        hd[((static_cast<int64_t>(m) * DV + j0 + jl) * 4 + q4) * 4 + ee] = St[jl][i];
    }
}
#undef HAI_LOAD_RECORD
#undef HAI_REC_LOAD1

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
    constexpr size_t shmem = state_lds_floats<DK>() * sizeof(float);
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
    deltanet_chunk_state_kernel<DK, DV><<<dim3(a.nv, DV / state_cols<DK>(), a.B), dim3(512), shmem, s>>>(a);
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
