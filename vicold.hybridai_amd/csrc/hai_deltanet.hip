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
//     accepting a prefix only moves the committed length;
//   * or (records mode) only the final state is stored, and every token
//     leaves a record of its rank-1 update instead -- beta * k^ (dk floats),
//     the correction c_j = v_j - k^T (decay S)_j of every value column (dv)
//     and the decay -- in slot position % nslots of a record buffer.  A later
//     call that starts at a committed length inside that span reads the
//     state the span started from and re-applies the kept records,
//     S = fma(beta k^, c, S * decay): the operations of the token loop, so
//     the state is the same to the bit, for 1 KB per token instead of 64 KB.
// No MFMA: the update is a rank-1 correction per token, bandwidth and latency
// bound.
#include "hai_common.h"
#include "hai_device.h"

namespace {

using namespace hai;

constexpr int kMaxT = 16;   // tokens per launch (verify width k + 1 <= 16)
constexpr int kMaxKc = 8;   // conv taps
constexpr int kMaxReplayT = 4;  // tokens of a call that replays records

struct DnArgs {
    uint16_t* out;
    int64_t ld_out;
    // fused verify: projection rows [qkv | z | a | b], conv ring, state slots
    const uint16_t* proj;
    int64_t ld_proj, off_qkv, off_z, off_a, off_b;
    const uint16_t* conv_w;
    uint16_t* ring;
    int ring_n, nslots, write_all;
    const int32_t* lens;
    int pos_add;
    // reference layout (Backend::deltanet_recurrent): separate conv outputs
    const uint16_t *q, *k, *v, *a, *bv, *z;
    float* state;
    const uint16_t *a_log, *dt_bias, *norm_w;
    int B, T, nk, nv, Kc;
    float eps;
    // a|b from the normalised rows (ld_xn) and the [2 nv, H] a|b weight
    // instead of proj columns off_a / off_b (null: read proj)
    const uint16_t* xn;
    int64_t ld_xn;
    const uint16_t* w_ab;
    int H;
    // rows per sequence in proj / out / xn (0: T).  A call of more than
    // kMaxT tokens runs as launches of kMaxT; each sees its own T but the
    // whole call's row layout.
    int64_t seq_rows;
    // records mode (rec non-null): [nslots][B][nv][dk + dv + 4] update
    // records, written for every token; only the final state is stored.
    // base [B]: replay = 0 stores each sequence's start position there
    // (base_out); replay = 1 starts from the state at base[b] and re-applies
    // the records of positions base[b] .. p0 - 1 first.
    float* rec;
    int32_t* base;
    int replay, base_out;
};

// floats per update record: beta * k^ (DK), the column corrections (DV), decay, pad
__host__ __device__ constexpr int64_t record_floats(int64_t dk, int64_t dv) { return dk + dv + 4; }

constexpr int kSeg = 2048;  // the linear layers' fma segment (elements)

// Gated delta rule over T tokens for one (value head, sequence).
// REF = false: fused verify step -- grouped causal conv + SiLU from the
//   projection rows and the conv ring, state read from slot p0 % nslots of
//   the column-tiled layout and written after every token (write_all) or the
//   last one, to slot (p0 + t + 1) % nslots.
// REF = true: the reference's deltanet_recurrent contract -- q, k, v already
//   convolved, a/b/z in their own [T, ...] buffers, one fp32 state
//   [nv][dk][dv] (hip_kernels.hip:985-1095) updated in place.
// TM bounds T (registers per thread for the inputs and outputs of all tokens).
template <int DK, int DV, bool REF, int TM>
__global__ __launch_bounds__(DV * 4) void deltanet_kernel(DnArgs A) {
    constexpr int NT = DV * 4;
    constexpr int NW = NT / 64;
    constexpr int GI = DK / 4;            // key dims per thread
    constexpr int ZP = (TM * DV + NT - 1) / NT;  // output elements per thread (all tokens)
    const int T = A.T;
    extern __shared__ __align__(16) float smem[];
    float* qs = smem;                  // [T][DK] conv output, q channels (then q * q-norm scale)
    float* ks = qs + T * DK;           // [T][DK] k channels (then k * k-norm scale)
    float* vs = ks + T * DK;           // [T][DV] v channels
    float* os = vs + T * DV;           // [T][DV] unrounded recurrent output
    float* bks = os + T * DV;          // [T][DK] beta * normalised k
    float* abp = bks + T * DK;         // w_ab: [T][2][nseg][64] lane partials of the a / b dot segments
    float* rls = abp + (A.w_ab != nullptr ? 2 * T * ((A.H + kSeg - 1) / kSeg) * 64 : 0);  // replayed records
    __shared__ float s_q[kMaxT], s_k[kMaxT], s_decay[kMaxT], s_beta[kMaxT], s_rms[kMaxT];

    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = tid >> 2;
    const int g = tid & 3;
    const int nv = A.nv;
    const int group = nv / A.nk;
    const int gq = h / group;
    const int64_t kw = static_cast<int64_t>(A.nk) * DK;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t C = 2 * kw + vw;
    const int hist = A.Kc - 1;
    const int64_t row0 = static_cast<int64_t>(b) * (A.seq_rows > 0 ? A.seq_rows : T);

    // ---- issue every global load of the step up front: first those that do
    // not depend on the cache length (its load is still in flight) ----
    // channel of this thread: [0, DK) q, [DK, 2DK) k, [2DK, 2DK+DV) v
    const int cl = tid;
    const bool has_ch = cl < 2 * DK + DV;
    float* dst = qs;
    int di = cl, dstride = DK;
    if (cl >= DK && cl < 2 * DK) { dst = ks; di = cl - DK; }
    else if (cl >= 2 * DK) { dst = vs; di = cl - 2 * DK; dstride = DV; }
    // window: vals[i] = input at position p0 - hist + i (history, then the T new tokens)
    uint16_t vals[TM + kMaxKc - 1];
#pragma unroll
    for (int i = 0; i < TM + kMaxKc - 1; ++i) vals[i] = 0;
    float wc[kMaxKc];
    int64_t c = 0;
    if (cl < DK) c = static_cast<int64_t>(gq) * DK + cl;
    else if (cl < 2 * DK) c = kw + static_cast<int64_t>(gq) * DK + (cl - DK);
    else c = 2 * kw + static_cast<int64_t>(h) * DV + (cl - 2 * DK);
    if (has_ch) {
        if constexpr (REF) {
            // convolved q/k/v rows straight from their buffers
            const uint16_t* srcp;
            int64_t ld, col;
            if (cl < DK) { srcp = A.q; ld = kw; col = static_cast<int64_t>(gq) * DK + cl; }
            else if (cl < 2 * DK) { srcp = A.k; ld = kw; col = static_cast<int64_t>(gq) * DK + cl - DK; }
            else { srcp = A.v; ld = vw; col = static_cast<int64_t>(h) * DV + cl - 2 * DK; }
#pragma unroll
            for (int t = 0; t < TM; ++t) vals[t] = t < T ? srcp[t * ld + col] : uint16_t{0};
        } else {
#pragma unroll
            for (int i = 0; i < kMaxKc; ++i) wc[i] = i < A.Kc ? bf2f(A.conv_w[c * A.Kc + i]) : 0.0f;
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                uint16_t x = 0;
                if (t < T) x = A.proj[(row0 + t) * A.ld_proj + A.off_qkv + c];
                // the new tokens go right after the hist history entries
#pragma unroll
                for (int hh = 0; hh < kMaxKc; ++hh)
                    if (hh == hist) vals[t + hh] = x;
            }
        }
    }
    // per-token gate scalars (last wave, lane = token)
    float a_in = 0.0f, b_in = 0.0f, dtb = 0.0f, alog = 0.0f;
    const bool scal = wave == NW - 1 && lane < T;
    if (scal && (REF || A.w_ab == nullptr)) {
        if constexpr (REF) {
            a_in = bf2f(A.a[static_cast<int64_t>(lane) * nv + h]);
            b_in = bf2f(A.bv[static_cast<int64_t>(lane) * nv + h]);
        } else {
            a_in = bf2f(A.proj[(row0 + lane) * A.ld_proj + A.off_a + h]);
            b_in = bf2f(A.proj[(row0 + lane) * A.ld_proj + A.off_b + h]);
        }
        dtb = bf2f(A.dt_bias[h]);
        alog = bf2f(A.a_log[h]);
    }
    // gate z and norm weight for the output elements (t, jo) = (tid / DV + r * NT / DV, tid % DV)
    const int jo = tid % DV;
    float zr[ZP];
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int t = tid / DV + r * (NT / DV);
        float zv = 0.0f;
        if (t < T) {
            if constexpr (REF) zv = bf2f(A.z[t * vw + static_cast<int64_t>(h) * DV + jo]);
            else zv = bf2f(A.proj[(row0 + t) * A.ld_proj + A.off_z + static_cast<int64_t>(h) * DV + jo]);
        }
        zr[r] = zv;
    }
    const float nwj = bf2f(A.norm_w[jo]);

    // ---- then the length-dependent ones: the state slot and the conv
    // history (one modulo each; later positions advance with a wrap) ----
    const int64_t p0 = REF ? 0 : static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;
    // records mode, replay: the state read is that of position base[b],
    // followed by the nrep records of positions base[b] .. p0 - 1 (a start
    // outside the record span reads slot p0 % nslots as the other modes do)
    int nrep = 0;
    if constexpr (!REF) {
        // (replays are compiled into the short-call instantiations only: the
        // host runs them with T <= kMaxReplayT)
        if (TM <= kMaxReplayT && A.replay) {
            const int64_t pb = A.base[b];
            if (pb <= p0 && p0 - pb < A.nslots && p0 - pb <= kMaxT) nrep = static_cast<int>(p0 - pb);
        } else if (A.base_out && h == 0 && tid == 0) {
            A.base[b] = static_cast<int32_t>(p0);
        }
    }
    constexpr int64_t RS = record_floats(DK, DV);
    constexpr int RQ = static_cast<int>(RS / 4);  // float4 per record
    float4 rq0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int64_t rec_r = 0;  // record slot of position base[b] (replay)
    float S[GI];  // column j, key dims [g*GI, g*GI+GI)
    int64_t slot_w = 0, ring_w = 0;  // state slot after token 0, ring entry of token 0
    if constexpr (REF) {
        const float* src = A.state + static_cast<int64_t>(h) * DK * DV + static_cast<int64_t>(g) * GI * DV + j;
#pragma unroll
        for (int i = 0; i < GI; ++i) S[i] = src[i * DV];
    } else {
        const int64_t slot = p0 % A.nslots;
        slot_w = slot + 1 == A.nslots ? 0 : slot + 1;
        const int64_t slot_r = slot >= nrep ? slot - nrep : slot - nrep + A.nslots;  // (p0 - nrep) % nslots
        const float4* src =
            reinterpret_cast<const float4*>(A.state + ((slot_r * A.B + b) * nv + h) * static_cast<int64_t>(DV) * DK) +
            tid;
#pragma unroll
        for (int m = 0; m < GI / 4; ++m) {
            const float4 v4 = src[m * NT];
            S[4 * m] = v4.x; S[4 * m + 1] = v4.y; S[4 * m + 2] = v4.z; S[4 * m + 3] = v4.w;
        }
        // ring entry of position p0 - hist (negative positions read as zero)
        const int64_t base = p0 - hist;
        int64_t rp = base % A.ring_n;
        if (rp < 0) rp += A.ring_n;
        if (has_ch) {
#pragma unroll
            for (int i = 0; i < kMaxKc - 1; ++i) {
                if (i < hist) {
                    if (base + i >= 0) vals[i] = A.ring[(static_cast<int64_t>(b) * A.ring_n + rp) * C + c];
                    rp = rp + 1 == A.ring_n ? 0 : rp + 1;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kMaxKc - 1; ++i)
                if (i < hist) rp = rp + 1 == A.ring_n ? 0 : rp + 1;
        }
        ring_w = rp;
        // records mode, replay: the kept records of positions p0 - nrep ..
        // p0 - 1 are staged in LDS (rls) for the token loop; each thread's
        // first 16-byte piece is requested here with the state, the pieces
        // past the first NT (more than 7 records) where they are stored
        rec_r = slot_r;
        if (tid < nrep * RQ) {
            const int i = tid / RQ;
            const int64_t rs = rec_r + i < A.nslots ? rec_r + i : rec_r + i - A.nslots;
            rq0 = reinterpret_cast<const float4*>(A.rec + ((rs * A.B + b) * nv + h) * RS)[tid - i * RQ];
        }
    }

    // ---- a|b projection of this head (w_ab mode): the 2T dot products of
    // the normalised rows with weight rows h (a) and nv + h (b), in the
    // linear layers' order (hai_gemm_bf16 bit for bit); one wave per
    // (token, a|b, 2048-element segment), lane partials to LDS ----
    const int nseg = (A.H + kSeg - 1) / kSeg;
    if constexpr (!REF) {
        if (A.w_ab != nullptr) {
            for (int task = wave; task < 2 * T * nseg; task += NW) {
                const int sg = task % nseg;
                const int d = task / nseg;  // = 2 t + (0 a | 1 b)
                const int t = d >> 1;
                const uint16_t* xr = A.xn + (row0 + t) * A.ld_xn;
                const uint16_t* wr = A.w_ab + (static_cast<int64_t>(d & 1) * nv + h) * A.H;
                uint4 xd[4], wd[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int k0 = sg * kSeg + u * 512 + lane * 8;
                    const bool ok = k0 < A.H;
                    xd[u] = ok ? *reinterpret_cast<const uint4*>(xr + k0) : make_uint4(0u, 0u, 0u, 0u);
                    wd[u] = ok ? *reinterpret_cast<const uint4*>(wr + k0) : make_uint4(0u, 0u, 0u, 0u);
                }
                float acc = 0.0f;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t xw[4] = {xd[u].x, xd[u].y, xd[u].z, xd[u].w};
                    const uint32_t ww[4] = {wd[u].x, wd[u].y, wd[u].z, wd[u].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc = fma_(lo_bf(xw[q]), lo_bf(ww[q]), acc);
                        acc = fma_(hi_bf(xw[q]), hi_bf(ww[q]), acc);
                    }
                }
                abp[task * 64 + lane] = acc;
            }
        }
    }

    // ---- grouped causal conv + SiLU (REF: inputs are already convolved) ----
    if (has_ch) {
        if constexpr (REF) {
#pragma unroll
            for (int t = 0; t < TM; ++t)
                if (t < T) dst[t * dstride + di] = bf2f(vals[t]);
        } else {
            const bool writer = cl >= 2 * DK || (h % group) == 0;
            int64_t rw = ring_w;  // ring entry of position p0 + t
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                if (t < T) {
                    float acc = bf2f(vals[t]) * wc[0];
#pragma unroll
                    for (int i = 1; i < kMaxKc; ++i)
                        if (i < A.Kc) acc = fma_(bf2f(vals[t + i]), wc[i], acc);
                    dst[t * dstride + di] = bfr(csilu(acc));
                    if (writer) {
                        uint16_t xv = 0;
#pragma unroll
                        for (int hh = 0; hh < kMaxKc; ++hh)
                            if (hh == hist) xv = vals[t + hh];
                        A.ring[(static_cast<int64_t>(b) * A.ring_n + rw) * C + c] = xv;
                    }
                    rw = rw + 1 == A.ring_n ? 0 : rw + 1;
                }
            }
        }
    }
    const bool ab_dots = !REF && A.w_ab != nullptr;
    if (scal && !ab_dots) {
        const float dtv = dtb + a_in;
        const float sp = fmaxf(dtv, 0.0f) + clog1p(cexp(-fabsf(dtv)));
        s_decay[lane] = cexp(-(cexp(alog) * sp));
        s_beta[lane] = csigmoid(b_in);
    }
    if constexpr (!REF) {
        // replayed records into LDS (read before this barrier, so before any
        // thread of this (sequence, head) rewrites one in the token loop)
        if (tid < nrep * RQ) reinterpret_cast<float4*>(rls)[tid] = rq0;
        for (int e = tid + NT; e < nrep * RQ; e += NT) {
            const int i = e / RQ;
            const int64_t rs = rec_r + i < A.nslots ? rec_r + i : rec_r + i - A.nslots;
            reinterpret_cast<float4*>(rls)[e] =
                reinterpret_cast<const float4*>(A.rec + ((rs * A.B + b) * nv + h) * RS)[e - i * RQ];
        }
    }
    __syncthreads();

    // w_ab mode: fold each dot's segments in order and butterfly (the GEMM's
    // reduction), round to bf16 as the projection output, then the gates
    if (ab_dots) {
        const float dtb_h = bf2f(A.dt_bias[h]);
        const float alog_h = bf2f(A.a_log[h]);
        for (int t = NW - 1 - wave; t < T; t += NW) {
            float ab[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                float tot = 0.0f;
                for (int sg = 0; sg < nseg; ++sg) tot = tot + abp[((2 * t + e) * nseg + sg) * 64 + lane];
                ab[e] = bfr(wave_sum64(tot));
            }
            if (lane == 0) {
                const float dtv = dtb_h + ab[0];
                const float sp = fmaxf(dtv, 0.0f) + clog1p(cexp(-fabsf(dtv)));
                s_decay[t] = cexp(-(cexp(alog_h) * sp));
                s_beta[t] = csigmoid(ab[1]);
            }
        }
    }

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

    // ---- every token's q * q-scale, k * k-scale and beta * (k * k-scale),
    // computed once for all columns (the same products the columns used) ----
    for (int e = tid; e < T * DK; e += NT) {
        const int t = e / DK;
        qs[e] = qs[e] * s_q[t];
        const float kh = ks[e] * s_k[t];
        ks[e] = kh;
        bks[e] = s_beta[t] * kh;
    }
    __syncthreads();

    // ---- gated delta rule, token by token (column-local: no block barrier) ----
    int64_t rec_slot = p0 % A.nslots;  // records mode: record slot of token t
    // replayed records first (t < 0, uniform over the block): the update of
    // the token loop with the kept beta * k^, correction and decay
    for (int t = -nrep; t < T; ++t) {
        if (t < 0) {
            const float* rr = rls + (t + nrep) * RS;
            const float dc = rr[DK + DV];
            const float cr = rr[DK + j];
            const float4* br = reinterpret_cast<const float4*>(rr + g * GI);
#pragma unroll
            for (int m = 0; m < GI / 4; ++m) {
                const float4 b4 = br[m];
                const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    S[4 * m + e] = S[4 * m + e] * dc;
                    S[4 * m + e] = fma_(bv[e], cr, S[4 * m + e]);
                }
            }
            continue;
        }
        const float decay = s_decay[t];
        const float4* qt = reinterpret_cast<const float4*>(qs + t * DK + g * GI);
        const float4* kt = reinterpret_cast<const float4*>(ks + t * DK + g * GI);
        const float4* bt = reinterpret_cast<const float4*>(bks + t * DK + g * GI);
        float r = 0.0f;
#pragma unroll
        for (int m = 0; m < GI / 4; ++m) {
            const float4 k4 = kt[m];
            const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S[4 * m + e] = S[4 * m + e] * decay;
                r = fma_(kv[e], S[4 * m + e], r);
            }
        }
        r = r + quad_xor1(r);
        r = r + quad_xor2(r);
        const float cj = vs[t * DV + j] - r;
        if constexpr (!REF) {
            if (A.rec != nullptr) {
                float* rr = A.rec + ((rec_slot * A.B + b) * nv + h) * RS;
                if (tid < DK / 4)
                    *reinterpret_cast<float4*>(rr + 4 * tid) = *reinterpret_cast<const float4*>(bks + t * DK + 4 * tid);
                if (g == 0) rr[DK + j] = cj;
                if (tid == 0) rr[DK + DV] = decay;
                rec_slot = rec_slot + 1 == A.nslots ? 0 : rec_slot + 1;
            }
        }
        float o = 0.0f;
#pragma unroll
        for (int m = 0; m < GI / 4; ++m) {
            const float4 b4 = bt[m], q4 = qt[m];
            const float bv[4] = {b4.x, b4.y, b4.z, b4.w}, qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S[4 * m + e] = fma_(bv[e], cj, S[4 * m + e]);
                o = fma_(qv[e], S[4 * m + e], o);
            }
        }
        o = o + quad_xor1(o);
        o = o + quad_xor2(o);
        if constexpr (REF) {
            if (t == T - 1) {
                float* dstp = A.state + static_cast<int64_t>(h) * DK * DV + static_cast<int64_t>(g) * GI * DV + j;
#pragma unroll
                for (int i = 0; i < GI; ++i) dstp[i * DV] = S[i];
            }
        } else {
            if (A.write_all || t == T - 1) {
                float4* dstp =
                    reinterpret_cast<float4*>(A.state + ((slot_w * A.B + b) * nv + h) * static_cast<int64_t>(DV) * DK) +
                    tid;
#pragma unroll
                for (int m = 0; m < GI / 4; ++m)
                    dstp[m * NT] = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
            }
            slot_w = slot_w + 1 == A.nslots ? 0 : slot_w + 1;  // state after token t + 1
        }
        if (g == 0) os[t * DV + j] = o;
    }
    __syncthreads();

    // ---- gated RMSNorm: rms from the unrounded output, one wave per token ----
    for (int t = wave; t < T; t += NW) {
        const float sso = l64_sumsq_f32(os + t * DV, DV, lane);
        if (lane == 0) s_rms[t] = 1.0f / csqrt(sso / static_cast<float>(DV) + A.eps);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int t = tid / DV + r * (NT / DV);
        if (t < T) {
            const float ob = bfr(os[t * DV + jo]);
            A.out[(row0 + t) * A.ld_out + static_cast<int64_t>(h) * DV + jo] =
                f2bf(((ob * s_rms[t]) * nwj) * csilu(zr[r]));
        }
    }
}

// Column-split fused verify (no a|b dots): CS blocks per (value head,
// sequence), block cs owning value columns [cs*DV/CS, (cs+1)*DV/CS).  The
// columns of the delta rule are independent (hip_kernels.hip:1055-1075), so
// each block runs the recurrence of its columns exactly as deltanet_kernel
// does (4 threads per column, the same fma chains and xor butterflies); the
// per-head work (conv of the q/k channels, q/k norms, gates) is repeated in
// every block.  Only the gated RMSNorm needs the whole head: every block
// stores its unrounded outputs in the workspace and counts itself in the
// head's counter (a device-scope atomic behind a device-scope fence); the
// block that arrives last reads the head's outputs back and finishes the
// norm in deltanet_kernel's order, so the result is bit-identical.  No block
// waits for another, and the last one resets the counter for the next launch.
// A head's state and conv traffic is then spread over CS CUs (one block per
// head used 48 of 256 CUs at B = 1).
template <int DK, int DV, int CS>
__global__ __launch_bounds__(DV / CS * 4 > 256 ? DV / CS * 4 : 256) void deltanet_cols_kernel(
    DnArgs A, float* __restrict__ o_ws, uint32_t* __restrict__ counters) {
    constexpr int DC = DV / CS;                 // value columns of this block
    constexpr int RT = DC * 4;                  // recurrence threads (4 per column)
    constexpr int NT = RT > 256 ? RT : 256;
    constexpr int NW = NT / 64;
    constexpr int GI = DK / 4;
    constexpr int NCH = 2 * DK + DC;            // conv channels: q, k, the block's v columns
    constexpr int CPT = (NCH + NT - 1) / NT;    // channels per thread
    constexpr int ZP = (kMaxT * DV + NT - 1) / NT;  // finishing block: outputs per thread
    const int T = A.T;
    extern __shared__ __align__(16) float smem[];
    float* qs = smem;              // [T][DK] q (then q * q-norm scale)
    float* ks = qs + T * DK;       // [T][DK] k (then k * k-norm scale)
    float* bks = ks + T * DK;      // [T][DK] beta * normalised k
    float* vs = bks + T * DK;      // [T][DC] v of the block's columns
    float* os = vs + T * DC;       // [T][DV] the head's unrounded outputs (finishing block)
    __shared__ float s_q[kMaxT], s_k[kMaxT], s_decay[kMaxT], s_beta[kMaxT], s_rms[kMaxT];
    __shared__ uint32_t s_last;

    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int j0 = static_cast<int>(blockIdx.z) * DC;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int jl = tid >> 2;  // recurrence: column j0 + jl, key quarter g
    const int g = tid & 3;
    const bool rec = tid < RT;
    const int nv = A.nv;
    const int group = nv / A.nk;
    const int gq = h / group;
    const int64_t kw = static_cast<int64_t>(A.nk) * DK;
    const int64_t vw = static_cast<int64_t>(nv) * DV;
    const int64_t C = 2 * kw + vw;
    const int hist = A.Kc - 1;
    const int64_t row0 = static_cast<int64_t>(b) * (A.seq_rows > 0 ? A.seq_rows : T);
    const int64_t head = static_cast<int64_t>(b) * nv + h;

    // ---- loads that do not depend on the cache length ----
    uint16_t vals[CPT][kMaxT + kMaxKc - 1];  // input at position p0 - hist + i
    float wc[CPT][kMaxKc];
    int64_t chan[CPT];
#pragma unroll
    for (int ci = 0; ci < CPT; ++ci) {
        const int cl = tid + NT * ci;
#pragma unroll
        for (int i = 0; i < kMaxT + kMaxKc - 1; ++i) vals[ci][i] = 0;
        if (cl < DK) chan[ci] = static_cast<int64_t>(gq) * DK + cl;
        else if (cl < 2 * DK) chan[ci] = kw + static_cast<int64_t>(gq) * DK + (cl - DK);
        else chan[ci] = 2 * kw + static_cast<int64_t>(h) * DV + j0 + (cl - 2 * DK);
        if (cl < NCH) {
#pragma unroll
            for (int i = 0; i < kMaxKc; ++i) wc[ci][i] = i < A.Kc ? bf2f(A.conv_w[chan[ci] * A.Kc + i]) : 0.0f;
#pragma unroll
            for (int t = 0; t < kMaxT; ++t) {
                uint16_t x = 0;
                if (t < T) x = A.proj[(row0 + t) * A.ld_proj + A.off_qkv + chan[ci]];
#pragma unroll
                for (int hh = 0; hh < kMaxKc; ++hh)
                    if (hh == hist) vals[ci][t + hh] = x;
            }
        }
    }
    float a_in = 0.0f, b_in = 0.0f, dtb = 0.0f, alog = 0.0f;
    const bool scal = wave == NW - 1 && lane < T;
    if (scal) {
        a_in = bf2f(A.proj[(row0 + lane) * A.ld_proj + A.off_a + h]);
        b_in = bf2f(A.proj[(row0 + lane) * A.ld_proj + A.off_b + h]);
        dtb = bf2f(A.dt_bias[h]);
        alog = bf2f(A.a_log[h]);
    }
    // gate z and norm weight of the outputs this thread writes if its block
    // finishes the head: element e = tid + r * NT of [T][DV]
    float zr[ZP], nwr[ZP];
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int e = tid + r * NT;
        const int t = e / DV;
        const int jo = e - t * DV;
        zr[r] = t < T ? bf2f(A.proj[(row0 + t) * A.ld_proj + A.off_z + static_cast<int64_t>(h) * DV + jo]) : 0.0f;
        nwr[r] = t < T ? bf2f(A.norm_w[jo]) : 0.0f;
    }

    // ---- the length-dependent ones: state slot (this block's columns) and
    // conv history ----
    const int64_t p0 = static_cast<int64_t>(A.lens ? A.lens[b] : 0) + A.pos_add;
    const int64_t slot = p0 % A.nslots;
    int64_t slot_w = slot + 1 == A.nslots ? 0 : slot + 1;
    float S[GI];
    if (rec) {
        // column-tiled head: float4 number m * 4 * DV + 4 * j + g holds keys
        // g * GI + 4m .. + 3 of column j
        const float4* src =
            reinterpret_cast<const float4*>(A.state + ((slot * A.B + b) * nv + h) * static_cast<int64_t>(DV) * DK) +
            4 * j0 + tid;
#pragma unroll
        for (int m = 0; m < GI / 4; ++m) {
            const float4 v4 = src[m * 4 * DV];
            S[4 * m] = v4.x; S[4 * m + 1] = v4.y; S[4 * m + 2] = v4.z; S[4 * m + 3] = v4.w;
        }
    }
    const int64_t base = p0 - hist;
    int64_t rp0 = base % A.ring_n;
    if (rp0 < 0) rp0 += A.ring_n;
    int64_t ring_w = rp0;  // ring entry of position p0
#pragma unroll
    for (int i = 0; i < kMaxKc - 1; ++i)
        if (i < hist) ring_w = ring_w + 1 == A.ring_n ? 0 : ring_w + 1;
#pragma unroll
    for (int ci = 0; ci < CPT; ++ci) {
        if (tid + NT * ci < NCH) {
            int64_t rp = rp0;
#pragma unroll
            for (int i = 0; i < kMaxKc - 1; ++i) {
                if (i < hist) {
                    if (base + i >= 0) vals[ci][i] = A.ring[(static_cast<int64_t>(b) * A.ring_n + rp) * C + chan[ci]];
                    rp = rp + 1 == A.ring_n ? 0 : rp + 1;
                }
            }
        }
    }

    // ---- grouped causal conv + SiLU; new inputs into the ring (q/k channels
    // by the first block of the head group's first head) ----
#pragma unroll
    for (int ci = 0; ci < CPT; ++ci) {
        const int cl = tid + NT * ci;
        if (cl < NCH) {
            float* dst = qs;
            int di = cl, dstride = DK;
            if (cl >= DK && cl < 2 * DK) { dst = ks; di = cl - DK; }
            else if (cl >= 2 * DK) { dst = vs; di = cl - 2 * DK; dstride = DC; }
            const bool writer = cl >= 2 * DK || ((h % group) == 0 && j0 == 0);
            int64_t rw = ring_w;
#pragma unroll
            for (int t = 0; t < kMaxT; ++t) {
                if (t < T) {
                    float acc = bf2f(vals[ci][t]) * wc[ci][0];
#pragma unroll
                    for (int i = 1; i < kMaxKc; ++i)
                        if (i < A.Kc) acc = fma_(bf2f(vals[ci][t + i]), wc[ci][i], acc);
                    dst[t * dstride + di] = bfr(csilu(acc));
                    if (writer) {
                        uint16_t xv = 0;
#pragma unroll
                        for (int hh = 0; hh < kMaxKc; ++hh)
                            if (hh == hist) xv = vals[ci][t + hh];
                        A.ring[(static_cast<int64_t>(b) * A.ring_n + rw) * C + chan[ci]] = xv;
                    }
                    rw = rw + 1 == A.ring_n ? 0 : rw + 1;
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

    // ---- q / k L2 norms, then the scaled q, k and beta * k ----
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
    for (int e = tid; e < T * DK; e += NT) {
        const int t = e / DK;
        qs[e] = qs[e] * s_q[t];
        const float kh = ks[e] * s_k[t];
        ks[e] = kh;
        bks[e] = s_beta[t] * kh;
    }
    __syncthreads();

    // ---- gated delta rule of the block's columns ----
    float* ow = o_ws + head * kMaxT * DV;
    if (rec) {
        for (int t = 0; t < T; ++t) {
            const float decay = s_decay[t];
            const float4* qt = reinterpret_cast<const float4*>(qs + t * DK + g * GI);
            const float4* kt = reinterpret_cast<const float4*>(ks + t * DK + g * GI);
            const float4* bt = reinterpret_cast<const float4*>(bks + t * DK + g * GI);
            float r = 0.0f;
#pragma unroll
            for (int m = 0; m < GI / 4; ++m) {
                const float4 k4 = kt[m];
                const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    S[4 * m + e] = S[4 * m + e] * decay;
                    r = fma_(kv[e], S[4 * m + e], r);
                }
            }
            r = r + quad_xor1(r);
            r = r + quad_xor2(r);
            const float cj = vs[t * DC + jl] - r;
            float o = 0.0f;
#pragma unroll
            for (int m = 0; m < GI / 4; ++m) {
                const float4 b4 = bt[m], q4 = qt[m];
                const float bv[4] = {b4.x, b4.y, b4.z, b4.w}, qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    S[4 * m + e] = fma_(bv[e], cj, S[4 * m + e]);
                    o = fma_(qv[e], S[4 * m + e], o);
                }
            }
            o = o + quad_xor1(o);
            o = o + quad_xor2(o);
            if (A.write_all || t == T - 1) {
                float4* dstp = reinterpret_cast<float4*>(A.state + ((slot_w * A.B + b) * nv + h) *
                                                                       static_cast<int64_t>(DV) * DK) +
                               4 * j0 + tid;
#pragma unroll
                for (int m = 0; m < GI / 4; ++m)
                    dstp[m * 4 * DV] = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
            }
            slot_w = slot_w + 1 == A.nslots ? 0 : slot_w + 1;
            if (g == 0) ow[t * DV + j0 + jl] = o;
        }
    }

    // ---- completion: the last block of the head finishes the gated norm ----
    __threadfence();  // this block's outputs are visible device-wide before it counts itself
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(counters + head, 1u) == static_cast<uint32_t>(CS - 1) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    __threadfence();  // and read only after every block has counted itself
    if (tid == 0) atomicExch(counters + head, 0u);
    for (int e = tid; e < T * DV; e += NT) os[e] = ow[e];
    __syncthreads();
    for (int t = wave; t < T; t += NW) {
        const float sso = l64_sumsq_f32(os + t * DV, DV, lane);
        if (lane == 0) s_rms[t] = 1.0f / csqrt(sso / static_cast<float>(DV) + A.eps);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ZP; ++r) {
        const int e = tid + r * NT;
        const int t = e / DV;
        if (t < T) {
            const int jo = e - t * DV;
            const float ob = bfr(os[e]);
            A.out[(row0 + t) * A.ld_out + static_cast<int64_t>(h) * DV + jo] =
                f2bf(((ob * s_rms[t]) * nwr[r]) * csilu(zr[r]));
        }
    }
}

// deltanet_grouped_conv_kernel (hip_kernels.hip:871-912) over the reference's
// conv state [C][Kc-1] (oldest first): one thread per flat [Q|K|V] channel,
// the canonical conv order of the fused kernel, state shifted in place.
__global__ __launch_bounds__(256) void deltanet_conv_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                            uint16_t* __restrict__ v, uint16_t* __restrict__ cs,
                                                            const uint16_t* __restrict__ qkv,
                                                            const uint16_t* __restrict__ w, int64_t T, int64_t kw,
                                                            int64_t vw, int Kc) {
    const int64_t C = 2 * kw + vw;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const int hist = Kc - 1;
    uint16_t* st = cs + c * hist;
    float wc[kMaxKc], win[kMaxKc];
#pragma unroll
    for (int i = 0; i < kMaxKc; ++i) {
        wc[i] = i < Kc ? bf2f(w[c * Kc + i]) : 0.0f;
        win[i] = i < hist ? bf2f(st[i]) : 0.0f;
    }
    uint16_t* dstp;
    int64_t ld, col;
    if (c < kw) { dstp = q; ld = kw; col = c; }
    else if (c < 2 * kw) { dstp = k; ld = kw; col = c - kw; }
    else { dstp = v; ld = vw; col = c - 2 * kw; }
    for (int64_t t = 0; t < T; ++t) {
        const float x = bf2f(qkv[t * C + c]);
        float acc;
        if (hist > 0) {
            acc = win[0] * wc[0];
#pragma unroll
            for (int i = 1; i < kMaxKc - 1; ++i)
                if (i < hist) acc = fma_(win[i], wc[i], acc);
#pragma unroll
            for (int i = 1; i < kMaxKc; ++i)
                if (i == hist) acc = fma_(x, wc[i], acc);
        } else {
            acc = x * wc[0];
        }
        dstp[t * ld + col] = f2bf(csilu(acc));
#pragma unroll
        for (int i = 0; i + 1 < kMaxKc; ++i)
            if (i + 1 < hist) win[i] = win[i + 1];
#pragma unroll
        for (int i = 0; i < kMaxKc; ++i)
            if (i == hist - 1) win[i] = x;
    }
#pragma unroll
    for (int i = 0; i < kMaxKc; ++i)
        if (i < hist) st[i] = f2bf(win[i]);
}

template <int DK, int DV, bool REF, int TM>
int launch_tm(const DnArgs& a, hipStream_t s) {
    const size_t ab = a.w_ab != nullptr ? static_cast<size_t>(2 * a.T) * ((a.H + kSeg - 1) / kSeg) * 64 : 0;
    // replay: up to kMaxT records of the span staged
    const size_t rq = a.replay && a.T <= kMaxReplayT ? static_cast<size_t>(a.nslots - 1 < kMaxT ? a.nslots - 1 : kMaxT) *
                                     record_floats(DK, DV) : 0;
    const size_t shmem = (static_cast<size_t>(a.T) * (3 * DK + 2 * DV) + ab + rq) * sizeof(float);
    deltanet_kernel<DK, DV, REF, TM><<<dim3(a.nv, REF ? 1 : a.B), dim3(DV * 4), shmem, s>>>(a);
    return launched(REF ? "deltanet_recurrent_kernel" : "deltanet_verify_kernel");
}

// the smallest token bound of the instantiations that covers T
template <int DK, int DV, bool REF>
int launch(const DnArgs& a, hipStream_t s) {
    if constexpr (!REF) {
        if (a.T <= 1) return launch_tm<DK, DV, REF, 1>(a, s);
        if (a.T <= 2) return launch_tm<DK, DV, REF, 2>(a, s);
        if (a.T <= 4) return launch_tm<DK, DV, REF, 4>(a, s);
    }
    return launch_tm<DK, DV, REF, kMaxT>(a, s);
}

// Workspace of the column-split kernel: one counter per (sequence, head),
// then the heads' unrounded outputs [B][nv][16][dv] fp32.
int64_t counters_bytes(int64_t B, int64_t nv) { return (B * nv * 4 + 255) / 256 * 256; }
int64_t cols_workspace_bytes(int64_t B, int64_t nv, int64_t dv) {
    return counters_bytes(B, nv) + B * nv * kMaxT * dv * 4;
}

template <int DK, int DV, int CS>
int launch_cols(const DnArgs& a, void* ws, hipStream_t s) {
    constexpr int DC = DV / CS;
    constexpr int NT = DC * 4 > 256 ? DC * 4 : 256;
    const size_t shmem = static_cast<size_t>(a.T) * (3 * DK + DC + DV) * sizeof(float);
    auto* counters = static_cast<uint32_t*>(ws);
    auto* o_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + counters_bytes(a.B, a.nv));
    deltanet_cols_kernel<DK, DV, CS><<<dim3(a.nv, a.B, CS), dim3(NT), shmem, s>>>(a, o_ws, counters);
    return launched("deltanet_cols_kernel");
}

// Column blocks per head: enough blocks for the machine at small batches
// (B * nv heads, 256 CUs); one block per head once the heads alone fill it.
int column_splits(int64_t heads) { return heads < 128 ? 4 : (heads < 256 ? 2 : 1); }

int dispatch_cols(const DnArgs& a, int64_t dk, int64_t dv, void* ws, hipStream_t s) {
    const int cs = column_splits(static_cast<int64_t>(a.B) * a.nv);
    if (dk == 128 && dv == 128) return cs == 4 ? launch_cols<128, 128, 4>(a, ws, s) : launch_cols<128, 128, 2>(a, ws, s);
    if (dk == 64 && dv == 64) return cs == 4 ? launch_cols<64, 64, 4>(a, ws, s) : launch_cols<64, 64, 2>(a, ws, s);
    return invalid("deltanet: (dk, dv) must be (128,128) or (64,64)");
}

template <bool REF>
int dispatch(const DnArgs& a, int64_t dk, int64_t dv, hipStream_t s) {
    if (dk == 128 && dv == 128) return launch<128, 128, REF>(a, s);
    if (dk == 64 && dv == 64) return launch<64, 64, REF>(a, s);
    return invalid("deltanet: (dk, dv) must be (128,128) or (64,64)");
}

}  // namespace

namespace {

int verify(void* out, int64_t ld_out, const void* proj, int64_t ld_proj, int64_t off_qkv, int64_t off_z,
           int64_t off_a, int64_t off_b, const void* conv_w, void* conv_ring, int64_t ring, float* state,
           int64_t nslots, int write_all_slots, const void* a_log, const void* dt_bias, const void* norm_w,
           const int32_t* lens, int32_t pos_add, int64_t B, int64_t T, int64_t nk, int64_t nv, int64_t dk, int64_t dv,
           int64_t Kc, float eps, const void* xn, int64_t ld_xn, const void* w_ab, int64_t H, void* ws,
           int64_t ws_bytes, void* stream, float* rec = nullptr, int32_t* base = nullptr, int replay = 0) {
    if (out == nullptr || proj == nullptr || conv_w == nullptr || conv_ring == nullptr || state == nullptr ||
        a_log == nullptr || dt_bias == nullptr || norm_w == nullptr)
        return invalid("deltanet_verify: null pointer");
    if (B < 0 || T < 0 || nk <= 0 || nv <= 0 || nv % nk != 0 || Kc < 1 || Kc > kMaxKc || nslots < 1)
        return invalid("deltanet_verify: shape");
    if ((T < kMaxT ? T : kMaxT) + Kc - 1 > ring) return invalid("deltanet_verify: conv ring too short for T");
    if (write_all_slots && nslots < T) return invalid("deltanet_verify: fewer state slots than tokens");
    if (lens == nullptr && pos_add < 0) return invalid("deltanet_verify: negative position");
    if (!aligned16(state)) return invalid("deltanet_verify: state alignment");
    if (T > INT32_MAX / 2 || static_cast<int64_t>(pos_add) + T > INT32_MAX)
        return invalid("deltanet_verify: T too large");
    if (w_ab != nullptr) {
        if (xn == nullptr || H <= 0 || H % 8 != 0 || H > 4 * kSeg || ld_xn < H || ld_xn % 8 != 0 || !aligned16(xn) ||
            !aligned16(w_ab))
            return invalid("deltanet_verify_ab: xn / w_ab (need 0 < H <= 8192, H % 8 == 0, ld_xn >= H, "
                           "ld_xn % 8 == 0, 16-byte alignment)");
    }
    if (B == 0 || T == 0) return HAI_OK;
    DnArgs a{};
    a.out = static_cast<uint16_t*>(out);
    a.ld_out = ld_out;
    a.proj = static_cast<const uint16_t*>(proj);
    a.ld_proj = ld_proj;
    a.off_qkv = off_qkv;
    a.off_z = off_z;
    a.off_a = off_a;
    a.off_b = off_b;
    a.conv_w = static_cast<const uint16_t*>(conv_w);
    a.ring = static_cast<uint16_t*>(conv_ring);
    a.ring_n = int(ring);
    a.nslots = int(nslots);
    a.write_all = write_all_slots;
    a.lens = lens;
    a.pos_add = pos_add;
    a.state = state;
    a.a_log = static_cast<const uint16_t*>(a_log);
    a.dt_bias = static_cast<const uint16_t*>(dt_bias);
    a.norm_w = static_cast<const uint16_t*>(norm_w);
    a.B = int(B);
    a.T = int(T);
    a.nk = int(nk);
    a.nv = int(nv);
    a.Kc = int(Kc);
    a.eps = eps;
    a.xn = static_cast<const uint16_t*>(xn);
    a.ld_xn = ld_xn;
    a.w_ab = static_cast<const uint16_t*>(w_ab);
    a.H = w_ab != nullptr ? int(H) : 0;
    a.rec = rec;
    a.base = base;
    if (rec != nullptr) a.write_all = 0;  // the final state only
    if (ws != nullptr && (ws_bytes < cols_workspace_bytes(B, nv, dv) || !aligned16(ws)))
        return invalid("deltanet_verify_ws: workspace smaller than hai_deltanet_workspace_bytes(B, nv, dv) or "
                       "not 16-byte aligned");
    const bool cols = ws != nullptr && w_ab == nullptr && column_splits(B * nv) > 1;
    // launches of at most kMaxT tokens, in order: each starts from the state
    // slot and conv ring entries the previous one left (positions advance by
    // its tokens), so the result equals one pass over all T
    a.seq_rows = T;
    for (int64_t t0 = 0; t0 < T; t0 += kMaxT) {
        DnArgs s = a;
        s.T = static_cast<int>(T - t0 < kMaxT ? T - t0 : kMaxT);
        s.pos_add = pos_add + static_cast<int32_t>(t0);
        s.proj = a.proj + t0 * ld_proj;
        s.out = a.out + t0 * ld_out;
        if (s.xn != nullptr) s.xn = a.xn + t0 * ld_xn;
        // records mode: the first launch replays or records the start
        // positions; the later ones continue from the state it left
        s.replay = rec != nullptr && t0 == 0 ? replay : 0;
        s.base_out = rec != nullptr && t0 == 0 && replay == 0 ? 1 : 0;
        const int rc = cols ? dispatch_cols(s, dk, dv, ws, as_stream(stream)) : dispatch<false>(s, dk, dv, as_stream(stream));
        if (rc != HAI_OK) return rc;
    }
    return HAI_OK;
}

}  // namespace

extern "C" int hai_deltanet_verify_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                        int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b,
                                        const void* conv_w, void* conv_ring, int64_t ring, float* state,
                                        int64_t nslots, int write_all_slots, const void* a_log,
                                        const void* dt_bias, const void* norm_w, const int32_t* lens,
                                        int32_t pos_add, int64_t B, int64_t T, int64_t nk, int64_t nv,
                                        int64_t dk, int64_t dv, int64_t Kc, float eps, void* stream) {
    return verify(out, ld_out, proj, ld_proj, off_qkv, off_z, off_a, off_b, conv_w, conv_ring, ring, state, nslots,
                  write_all_slots, a_log, dt_bias, norm_w, lens, pos_add, B, T, nk, nv, dk, dv, Kc, eps, nullptr, 0,
                  nullptr, 0, nullptr, 0, stream);
}

extern "C" size_t hai_deltanet_workspace_bytes(int64_t B, int64_t nv, int64_t dv) {
    if (B < 0 || nv < 0 || dv < 0) return 0;
    return static_cast<size_t>(cols_workspace_bytes(B, nv, dv));
}

extern "C" int hai_deltanet_verify_ws_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                           int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b,
                                           const void* conv_w, void* conv_ring, int64_t ring, float* state,
                                           int64_t nslots, int write_all_slots, const void* a_log,
                                           const void* dt_bias, const void* norm_w, const int32_t* lens,
                                           int32_t pos_add, int64_t B, int64_t T, int64_t nk, int64_t nv,
                                           int64_t dk, int64_t dv, int64_t Kc, float eps, void* workspace,
                                           int64_t workspace_bytes, void* stream) {
    if (workspace == nullptr) return invalid("deltanet_verify_ws: null workspace");
    if (workspace_bytes < 0) return invalid("deltanet_verify_ws: negative workspace size");
    if (const int rc = check_extent(workspace, static_cast<size_t>(workspace_bytes), "deltanet workspace"); rc != HAI_OK)
        return rc;
    return verify(out, ld_out, proj, ld_proj, off_qkv, off_z, off_a, off_b, conv_w, conv_ring, ring, state, nslots,
                  write_all_slots, a_log, dt_bias, norm_w, lens, pos_add, B, T, nk, nv, dk, dv, Kc, eps, nullptr, 0,
                  nullptr, 0, workspace, workspace_bytes, stream);
}

extern "C" int hai_deltanet_verify_ab_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                           int64_t off_qkv, int64_t off_z, const void* xn, int64_t ld_xn,
                                           const void* w_ab, int64_t H, const void* conv_w, void* conv_ring,
                                           int64_t ring, float* state, int64_t nslots, int write_all_slots,
                                           const void* a_log, const void* dt_bias, const void* norm_w,
                                           const int32_t* lens, int32_t pos_add, int64_t B, int64_t T, int64_t nk,
                                           int64_t nv, int64_t dk, int64_t dv, int64_t Kc, float eps,
                                           void* stream) {
    if (w_ab == nullptr) return invalid("deltanet_verify_ab: null w_ab");
    return verify(out, ld_out, proj, ld_proj, off_qkv, off_z, 0, 0, conv_w, conv_ring, ring, state, nslots,
                  write_all_slots, a_log, dt_bias, norm_w, lens, pos_add, B, T, nk, nv, dk, dv, Kc, eps, xn, ld_xn,
                  w_ab, H, nullptr, 0, stream);
}

extern "C" size_t hai_deltanet_records_bytes(int64_t nslots, int64_t B, int64_t nv, int64_t dk, int64_t dv) {
    if (nslots < 0 || B < 0 || nv < 0 || dk < 0 || dv < 0) return 0;
    const int64_t lim = INT64_MAX / 8;
    int64_t n = record_floats(dk, dv);
    for (const int64_t f : {nslots, B, nv}) {
        if (f != 0 && n > lim / f) return SIZE_MAX;
        n *= f;
    }
    return static_cast<size_t>(n) * sizeof(float);
}

extern "C" int hai_deltanet_verify_rec_bf16(void* out, int64_t ld_out, const void* proj, int64_t ld_proj,
                                            int64_t off_qkv, int64_t off_z, int64_t off_a, int64_t off_b,
                                            const void* xn, int64_t ld_xn, const void* w_ab, int64_t H,
                                            const void* conv_w, void* conv_ring, int64_t ring, float* state,
                                            int64_t nslots, float* records, int32_t* base, int replay,
                                            const void* a_log, const void* dt_bias, const void* norm_w,
                                            const int32_t* lens, int32_t pos_add, int64_t B, int64_t T, int64_t nk,
                                            int64_t nv, int64_t dk, int64_t dv, int64_t Kc, float eps, void* stream) {
    if (records == nullptr) return invalid("deltanet_verify_rec: null records");
    if (base == nullptr) return invalid("deltanet_verify_rec: null base");
    if (!aligned16(records)) return invalid("deltanet_verify_rec: records alignment");
    if (nslots <= T) return invalid("deltanet_verify_rec: need nslots > T");
    if (replay != 0 && replay != 1) return invalid("deltanet_verify_rec: replay must be 0 or 1");
    if (replay == 1 && T > kMaxReplayT) return invalid("deltanet_verify_rec: replay calls take at most 4 tokens");
    if (B > 0 && nslots > 0) {
        const size_t bytes = hai_deltanet_records_bytes(nslots, B, nv, dk, dv);
        if (bytes == SIZE_MAX) return invalid("deltanet_verify_rec: records size overflows");
        if (const int rc = check_extent(records, bytes, "deltanet records"); rc != HAI_OK) return rc;
        if (const int rc = check_extent(base, static_cast<size_t>(B) * 4, "deltanet base"); rc != HAI_OK) return rc;
    }
    return verify(out, ld_out, proj, ld_proj, off_qkv, off_z, off_a, off_b, conv_w, conv_ring, ring, state, nslots, 0,
                  a_log, dt_bias, norm_w, lens, pos_add, B, T, nk, nv, dk, dv, Kc, eps, xn, ld_xn, w_ab, H, nullptr, 0,
                  stream, records, base, replay);
}

extern "C" int hai_deltanet_conv_bf16(void* q, void* k, void* v, void* conv_state, const void* qkv,
                                      const void* conv_w, int64_t T, int64_t nk, int64_t nv, int64_t dk,
                                      int64_t dv, int64_t Kc, void* stream) {
    if (q == nullptr || k == nullptr || v == nullptr || qkv == nullptr || conv_w == nullptr ||
        (Kc > 1 && conv_state == nullptr))
        return invalid("deltanet_conv: null pointer");
    if (T < 0 || nk <= 0 || nv <= 0 || dk <= 0 || dv <= 0 || Kc < 1 || Kc > kMaxKc)
        return invalid("deltanet_conv: shape");
    const int64_t kw = nk * dk, vw = nv * dv, C = 2 * kw + vw;
    if (T == 0) return HAI_OK;
    deltanet_conv_kernel<<<dim3(static_cast<unsigned>((C + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(
        static_cast<uint16_t*>(q), static_cast<uint16_t*>(k), static_cast<uint16_t*>(v),
        static_cast<uint16_t*>(conv_state), static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(conv_w),
        T, kw, vw, int(Kc));
    return launched("deltanet_conv_kernel");
}

extern "C" int hai_deltanet_recurrent_bf16(void* out, float* state, const void* q, const void* k, const void* v,
                                           const void* a, const void* b, const void* a_log, const void* dt_bias,
                                           const void* norm_w, const void* z, int64_t T, int64_t nk, int64_t nv,
                                           int64_t dk, int64_t dv, float eps, void* stream) {
    if (out == nullptr || state == nullptr || q == nullptr || k == nullptr || v == nullptr || a == nullptr ||
        b == nullptr || a_log == nullptr || dt_bias == nullptr || norm_w == nullptr || z == nullptr)
        return invalid("deltanet_recurrent: null pointer");
    if (T < 0 || nk <= 0 || nv <= 0 || nv % nk != 0) return invalid("deltanet_recurrent: shape");
    if (T == 0) return HAI_OK;
    const hipStream_t s = as_stream(stream);
    const int64_t vw = nv * dv, kw = nk * dk;
    // the recurrence is sequential, so chunks of 16 tokens carry the state exactly
    for (int64_t t0 = 0; t0 < T; t0 += kMaxT) {
        const int64_t n = T - t0 < kMaxT ? T - t0 : kMaxT;
        DnArgs d{};
        d.out = static_cast<uint16_t*>(out) + t0 * vw;
        d.ld_out = vw;
        d.q = static_cast<const uint16_t*>(q) + t0 * kw;
        d.k = static_cast<const uint16_t*>(k) + t0 * kw;
        d.v = static_cast<const uint16_t*>(v) + t0 * vw;
        d.a = static_cast<const uint16_t*>(a) + t0 * nv;
        d.bv = static_cast<const uint16_t*>(b) + t0 * nv;
        d.z = static_cast<const uint16_t*>(z) + t0 * vw;
        d.state = state;
        d.a_log = static_cast<const uint16_t*>(a_log);
        d.dt_bias = static_cast<const uint16_t*>(dt_bias);
        d.norm_w = static_cast<const uint16_t*>(norm_w);
        d.B = 1;
        d.T = int(n);
        d.nk = int(nk);
        d.nv = int(nv);
        d.Kc = 1;
        d.eps = eps;
        const int rc = dispatch<true>(d, dk, dv, s);
        if (rc != HAI_OK) return rc;
    }
    return HAI_OK;
}
