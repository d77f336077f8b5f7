// oracle.cpp -- TEST INFRASTRUCTURE ONLY: CPU parity oracle for the MTP
// speculative verify path of Dustray/Vicold.HybridAI.  Loaded only by tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg.
//
// Every function restates reference behaviour and cites the reference line
// it follows.  Reduction orders are the canonical ones documented in
// oracle_numerics.h (the reference leaves them to rocBLAS and to thread
// striding, so an order has to be fixed for bit-exact parity).
#include "oracle.h"
#include "oracle_numerics.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

using namespace orc;

namespace {

inline float store(float v, int round_out) { return round_out ? bf(v) : v; }

}  // namespace

extern "C" {

// OpenMP threads of the oracle's parallel loops (the results do not depend
// on it: every output's reduction runs in one thread in a fixed order);
// returns the count in effect.
int orc_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

void orc_exp_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = cexp(x[i]);
}
void orc_log1p_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = clog1p(x[i]);
}
void orc_bf16_round_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = bf(x[i]);
}

// Linear::forward_into (linear.cc:137-155) -> rocBLAS gemm_ex with fp32
// compute and a bf16 store.  Canonical segmented-L64 order per output.
void orc_gemm(const float* x, const float* w, float* y, int64_t M, int64_t N,
              int64_t K, int round_out) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        const float* wr = w + n * K;
        for (int64_t m = 0; m < M; ++m)
            y[m * N + n] = store(gemm_dot(x + m * K, wr, K), round_out);
    }
}

// rmsnorm_kernel (hip_kernels.hip:105-137) / RMSNorm::forward CPU branch
// (rmsnorm.cc:81-91): inv = 1/sqrt(sum(x^2)/H + eps), y = x*inv*(w+offset).
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows,
                 int64_t H, float eps, int unit_offset, int round_out) {
    const float off = unit_offset ? 1.0f : 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * H;
        const float ss = l64_dot(xr, xr, H);
        const float inv = 1.0f / std::sqrt(ss / static_cast<float>(H) + eps);
        for (int64_t k = 0; k < H; ++k)
            y[r * H + k] = store((xr[k] * inv) * (w[k] + off), round_out);
    }
}

// add_kernel (hip_kernels.hip:43-51).
void orc_add(const float* a, const float* b, float* y, int64_t n, int round_out) {
    for (int64_t i = 0; i < n; ++i) y[i] = store(a[i] + b[i], round_out);
}

// silu_mul_kernel (hip_kernels.hip:164-175): g/(1+exp(-g)) * u.
void orc_silu_mul(const float* g, const float* u, float* y, int64_t n,
                  int round_out) {
    for (int64_t i = 0; i < n; ++i) y[i] = store(csilu(g[i]) * u[i], round_out);
}

// embedding_gather_kernel (hip_kernels.hip:88-103).
void orc_embedding(const float* table, const int64_t* ids, float* y,
                   int64_t n_ids, int64_t V, int64_t H) {
    for (int64_t r = 0; r < n_ids; ++r) {
        const int64_t id = ids[r];
        for (int64_t k = 0; k < H; ++k)
            y[r * H + k] = (id >= 0 && id < V) ? table[id * H + k] : 0.0f;
    }
}

// theta = pos / base^(2p/R) (hip_kernels.hip:209-213); evaluated in double
// and rounded once to fp32 for cos and sin.
void orc_rope_table(float* cos_t, float* sin_t, int64_t pos0, int64_t npos,
                    int64_t R, float base) {
    const int64_t half = R / 2;
    for (int64_t i = 0; i < npos; ++i)
        for (int64_t p = 0; p < half; ++p) {
            const double theta = static_cast<double>(pos0 + i) /
                std::pow(static_cast<double>(base),
                         static_cast<double>(2 * p) / static_cast<double>(R));
            cos_t[i * half + p] = static_cast<float>(std::cos(theta));
            sin_t[i * half + p] = static_cast<float>(std::sin(theta));
        }
}

namespace {

// Rotate-half on fp32 values xs[0..D) at one position (first R dims).
void rope_inplace(float* xs, int64_t D, int64_t R, const float* ct,
                  const float* st) {
    (void)D;
    const int64_t half = R / 2;
    std::vector<float> tmp(static_cast<size_t>(R));
    for (int64_t d = 0; d < R; ++d) {
        const int64_t p = d < half ? d : d - half;
        const float x = xs[p];
        const float y = xs[p + half];
        if (d < half) tmp[d] = fmaf_(x, ct[p], -(y * st[p]));
        else tmp[d] = fmaf_(y, ct[p], x * st[p]);
    }
    for (int64_t d = 0; d < R; ++d) xs[d] = tmp[d];
}

}  // namespace

// q_gate_rmsnorm_rope_kernel (hip_fused_kernels.hip:87-141): normalise the
// query half with (w+1), rotate the first R dims, store once; copy the gate.
void orc_q_gate_rmsnorm_rope(const float* src, const float* w, float* q_out,
                             float* gate_out, int64_t T, int64_t nq, int64_t D,
                             int64_t R, int64_t pos0, float base, float eps,
                             int unit_offset, int round_out) {
    const float off = unit_offset ? 1.0f : 0.0f;
    const int64_t half = R / 2;
    std::vector<float> ct(static_cast<size_t>(T * half + 1)), st(ct.size());
    orc_rope_table(ct.data(), st.data(), pos0, T, R, base);
    std::vector<float> qn(static_cast<size_t>(D));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < nq; ++h) {
            const float* s = src + (t * nq + h) * 2 * D;
            const float ss = l64_dot(s, s, D);
            const float inv = 1.0f / std::sqrt(ss / static_cast<float>(D) + eps);
            for (int64_t d = 0; d < D; ++d) qn[d] = (s[d] * inv) * (w[d] + off);
            rope_inplace(qn.data(), D, R, ct.data() + t * half, st.data() + t * half);
            float* qo = q_out + (t * nq + h) * D;
            float* go = gate_out + (t * nq + h) * D;
            for (int64_t d = 0; d < D; ++d) {
                qo[d] = store(qn[d], round_out);
                go[d] = s[D + d];
            }
        }
}

// attention.cc:459-464: RMSNorm::forward(k, +1) stores the normalised K,
// then RoPE::partial (partial_rope_kernel) rotates it and stores again.
void orc_k_rmsnorm_rope(const float* src, const float* w, float* k_out,
                        int64_t T, int64_t nkv, int64_t D, int64_t R,
                        int64_t pos0, float base, float eps, int round_out) {
    const int64_t half = R / 2;
    std::vector<float> ct(static_cast<size_t>(T * half + 1)), st(ct.size());
    orc_rope_table(ct.data(), st.data(), pos0, T, R, base);
    std::vector<float> kn(static_cast<size_t>(D));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < nkv; ++h) {
            const float* s = src + (t * nkv + h) * D;
            const float ss = l64_dot(s, s, D);
            const float inv = 1.0f / std::sqrt(ss / static_cast<float>(D) + eps);
            for (int64_t d = 0; d < D; ++d)
                kn[d] = store((s[d] * inv) * (w[d] + 1.0f), round_out);
            rope_inplace(kn.data(), D, R, ct.data() + t * half, st.data() + t * half);
            float* ko = k_out + (t * nkv + h) * D;
            for (int64_t d = 0; d < D; ++d) ko[d] = store(kn[d], round_out);
        }
}

// partial_rope_kernel (hip_kernels.hip:192-221) on [T, heads, D].
void orc_partial_rope(const float* src, float* dst, int64_t T, int64_t heads,
                      int64_t D, int64_t R, int64_t pos0, float base,
                      int round_out) {
    const int64_t half = R / 2;
    std::vector<float> ct(static_cast<size_t>(T * half + 1)), st(ct.size());
    orc_rope_table(ct.data(), st.data(), pos0, T, R, base);
    std::vector<float> x(static_cast<size_t>(D));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < heads; ++h) {
            const float* s = src + (t * heads + h) * D;
            for (int64_t d = 0; d < D; ++d) x[d] = s[d];
            rope_inplace(x.data(), D, R, ct.data() + t * half, st.data() + t * half);
            for (int64_t d = 0; d < D; ++d)
                dst[(t * heads + h) * D + d] = store(x[d], round_out);
        }
}

namespace {

// One query over keys [0, L): the canonical chunked softmax.  The reference
// (hip_kernels.hip:759-844) walks keys with an online softmax; here keys are
// grouped into fixed 64-key chunks by absolute index, each chunk is reduced
// on its own max, and chunks are merged against the global max.
void attend_one(const float* q, const float* gate, const float* kc,
                const float* vc, int64_t L, int64_t row_stride, int64_t D,
                float scale, float* out) {
    const int64_t nch = (L + 63) / 64;
    std::vector<float> mc(static_cast<size_t>(nch)), lc(static_cast<size_t>(nch));
    std::vector<float> oc(static_cast<size_t>(nch * D));
    float s[64], p[64];
    for (int64_t c = 0; c < nch; ++c) {
        float m = -INFINITY;
        for (int i = 0; i < 64; ++i) {
            const int64_t j = 64 * c + i;
            if (j < L) {
                s[i] = seq_dot(q, kc + j * row_stride, D) * scale;
                m = std::fmax(m, s[i]);
            }
        }
        for (int i = 0; i < 64; ++i) {
            const int64_t j = 64 * c + i;
            p[i] = j < L ? cexp(s[i] - m) : 0.0f;
        }
        float acc[64];
        for (int i = 0; i < 64; ++i) acc[i] = p[i];
        lc[c] = butterfly64(acc);
        mc[c] = m;
        for (int64_t d = 0; d < D; ++d) {
            float a = 0.0f;
            for (int i = 0; i < 64; ++i) {
                const int64_t j = 64 * c + i;
                if (j < L) a = fmaf_(p[i], vc[j * row_stride + d], a);
            }
            oc[c * D + d] = a;
        }
    }
    float M = -INFINITY;
    for (int64_t c = 0; c < nch; ++c) M = std::fmax(M, mc[c]);
    float Ls = 0.0f;
    std::vector<float> O(static_cast<size_t>(D), 0.0f);
    for (int64_t c = 0; c < nch; ++c) {
        const float wgt = cexp(mc[c] - M);
        Ls = fmaf_(lc[c], wgt, Ls);
        for (int64_t d = 0; d < D; ++d) O[d] = fmaf_(oc[c * D + d], wgt, O[d]);
    }
    for (int64_t d = 0; d < D; ++d) {
        float o = O[d] / Ls;
        if (gate != nullptr) o = o * csigmoid(gate[d]);
        out[d] = o;
    }
}

}  // namespace

// GatedGQAAttention::forward_impl cached branch (attention.cc:535-596):
// queries at positions cache_len-T+t attend to keys 0..position, output
// multiplied by sigmoid(gate), stored bf16.
void orc_attention(const float* q, const float* gate, const float* kc,
                   const float* vc, float* out, int64_t T, int64_t cache_len,
                   int64_t nq, int64_t nkv, int64_t D, int round_out) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    const int64_t group = nq / nkv;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < nq; ++h) {
            const int64_t kvh = h / group;
            const int64_t L = cache_len - T + t + 1;
            std::vector<float> o(static_cast<size_t>(D));
            attend_one(q + (t * nq + h) * D,
                       gate ? gate + (t * nq + h) * D : nullptr,
                       kc + kvh * D, vc + kvh * D, L, nkv * D, D, scale,
                       o.data());
            for (int64_t d = 0; d < D; ++d)
                out[(t * nq + h) * D + d] = store(o[d], round_out);
        }
}

// deltanet_grouped_conv_kernel (hip_kernels.hip:871-912): per flat channel
// of [Q|K|V], depthwise causal conv of size Kc over (state, x), SiLU, then
// the state shifts in the raw input.
void orc_deltanet_conv(const float* qkv, const float* w, float* conv_state,
                       float* q, float* k, float* v, int64_t T, int64_t nk,
                       int64_t nv, int64_t dk, int64_t dv, int64_t Kc,
                       int round_out) {
    const int64_t kw = nk * dk, vw = nv * dv, C = 2 * kw + vw, hist = Kc - 1;
    for (int64_t c = 0; c < C; ++c) {
        float* st = conv_state + c * hist;
        const float* wc = w + c * Kc;
        for (int64_t t = 0; t < T; ++t) {
            const float x = qkv[t * C + c];
            float acc;
            if (hist > 0) {
                acc = st[0] * wc[0];
                for (int64_t i = 1; i < hist; ++i) acc = fmaf_(st[i], wc[i], acc);
                acc = fmaf_(x, wc[hist], acc);
            } else {
                acc = x * wc[0];
            }
            const float y = store(csilu(acc), round_out);
            if (c < kw) q[t * kw + c] = y;
            else if (c < 2 * kw) k[t * kw + c - kw] = y;
            else v[t * vw + c - 2 * kw] = y;
            for (int64_t i = 0; i + 1 < hist; ++i) st[i] = st[i + 1];
            if (hist > 0) st[hist - 1] = x;
        }
    }
}

// deltanet_recurrent_kernel (hip_kernels.hip:985-1095), one v-head at a
// time, tokens in order:
//   q,k L2-normalised (eps 1e-6 inside the sqrt), q also by 1/sqrt(dk);
//   decay = exp(-exp(A_log) * softplus(dt_bias + a)); beta = sigmoid(b);
//   S *= decay; r = k.S; S += beta k (v - r); o = q.S;
//   out = bf(o) * rsqrt(mean(o^2)+eps) * w * silu(z).
// The reductions over the key dimension use four contiguous groups merged
// as (g0+g1)+(g2+g3); state layout [nv, dk, dv] as in the reference.
void orc_deltanet_recurrent(const float* q, const float* k, const float* v,
                            const float* a, const float* b, const float* z,
                            const float* a_log, const float* dt_bias,
                            const float* norm_w, float* state, float* out,
                            int64_t T, int64_t nk, int64_t nv, int64_t dk,
                            int64_t dv, float eps, int round_out) {
    const int64_t group = nv / nk;
    const float rs_dk = 1.0f / std::sqrt(static_cast<float>(dk));
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < nv; ++h) {
        const int64_t g = h / group;
        float* S = state + h * dk * dv;
        std::vector<float> qn(static_cast<size_t>(dk)), kn(static_cast<size_t>(dk)),
            bk(static_cast<size_t>(dk)), o(static_cast<size_t>(dv));
        for (int64_t t = 0; t < T; ++t) {
            const float* qt = q + (t * nk + g) * dk;
            const float* kt = k + (t * nk + g) * dk;
            const float* vt = v + (t * nv + h) * dv;
            const float* zt = z + (t * nv + h) * dv;
            const float ssq = l64_dot(qt, qt, dk);
            const float ssk = l64_dot(kt, kt, dk);
            const float qs = (1.0f / std::sqrt(ssq + 1.0e-6f)) * rs_dk;
            const float ks = 1.0f / std::sqrt(ssk + 1.0e-6f);
            const float dtv = dt_bias[h] + a[t * nv + h];
            const float sp = std::fmax(dtv, 0.0f) + clog1p(cexp(-std::fabs(dtv)));
            const float decay = cexp(-(cexp(a_log[h]) * sp));
            const float beta = csigmoid(b[t * nv + h]);
            for (int64_t i = 0; i < dk; ++i) {
                qn[i] = qt[i] * qs;
                kn[i] = kt[i] * ks;
                bk[i] = beta * kn[i];
            }
            for (int64_t j = 0; j < dv; ++j) {
                float pr[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int64_t i = 0; i < dk; ++i) {
                    float& s = S[i * dv + j];
                    s = s * decay;
                    const int64_t gi = (4 * i) / dk;
                    pr[gi] = fmaf_(kn[i], s, pr[gi]);
                }
                const float r = (pr[0] + pr[1]) + (pr[2] + pr[3]);
                const float cj = vt[j] - r;
                float po[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int64_t i = 0; i < dk; ++i) {
                    float& s = S[i * dv + j];
                    s = fmaf_(bk[i], cj, s);
                    const int64_t gi = (4 * i) / dk;
                    po[gi] = fmaf_(qn[i], s, po[gi]);
                }
                o[j] = (po[0] + po[1]) + (po[2] + po[3]);
            }
            const float sso = l64_dot(o.data(), o.data(), dv);
            const float rms = 1.0f / std::sqrt(sso / static_cast<float>(dv) + eps);
            for (int64_t j = 0; j < dv; ++j) {
                const float ob = store(o[j], round_out);
                out[(t * nv + h) * dv + j] =
                    store(((ob * rms) * norm_w[j]) * csilu(zt[j]), round_out);
            }
        }
    }
}

// argmax_rows_reference CPU branch (generator.cc:343-360): best starts at
// -inf, strictly greater wins, so the first maximum wins, NaN never wins and
// an all-NaN/-inf row returns 0.
void orc_argmax_rows(const float* x, int64_t* out, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        float best = -INFINITY;
        int64_t idx = 0;
        for (int64_t c = 0; c < cols; ++c) {
            const float v = x[r * cols + c];
            if (v > best) { best = v; idx = c; }
        }
        out[r] = idx;
    }
}

// ---- FP8 (A15) ---------------------------------------------------------------
// FP8Dequantizer::decode_e4m3 (fp8_dequant.cc:12-26): exponent 0 is the
// subnormal m * 2^-9, exponents 1..15 the normal (1 + m/8) * 2^(e-7); there
// is no NaN code (0x7F / 0xFF decode as +-480).
float orc_fp8_decode(uint8_t v) {
    const int e = (v >> 3) & 0xf;
    const int m = v & 7;
    const float r = e == 0 ? std::ldexp(static_cast<float>(m), -9)
                           : std::ldexp(1.0f + static_cast<float>(m) / 8.0f, e - 7);
    return (v & 0x80) ? -r : r;
}

void orc_fp8_decode_array(const uint8_t* q, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp8_decode(q[i]);
}

// Round-to-nearest-even E4M3 encoding, saturating at +-448 (code 0x7E) so the
// +-480 codes are never produced; NaN encodes as 0.  (The quantizer of the
// C5 synthetic weights: clamp(round(w / s), +-448).)
void orc_fp8_encode_array(const float* x, uint8_t* q, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        uint8_t sign = std::signbit(v) ? 0x80 : 0;
        const float a = std::fabs(v);
        uint8_t code;
        if (std::isnan(v)) {
            code = 0;
            sign = 0;
        } else if (a >= 448.0f) {
            code = 0x7e;
        } else if (a < std::ldexp(1.0f, -6)) {
            // subnormal grid 2^-9; rounding up to 8 lands on the first normal (code 0x08)
            code = static_cast<uint8_t>(std::nearbyint(a * 512.0f));
        } else {
            int E = 0;
            const float f = std::frexp(a, &E);  // a = f * 2^E, f in [0.5, 1)
            int e = E - 1 + 7;
            int m = static_cast<int>(std::nearbyint((2.0f * f - 1.0f) * 8.0f));
            if (m == 8) {
                m = 0;
                ++e;
            }
            code = (e > 15 || (e == 15 && m == 7)) ? uint8_t{0x7e} : static_cast<uint8_t>((e << 3) | m);
        }
        q[i] = sign | code;
    }
}

// FP8Dequantizer::dequantize_2d (fp8_dequant.cc:89-146): w = decode(q) * s
// with s[r / block_rows][c / block_cols], fp32.
void orc_fp8_dequant_2d(const uint8_t* q, const float* s, float* w, int64_t rows, int64_t cols, int64_t br,
                        int64_t bc) {
    const int64_t sc = (cols + bc - 1) / bc;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            w[r * cols + c] = orc_fp8_decode(q[r * cols + c]) * s[(r / br) * sc + c / bc];
}

// Linear over Block2D(128x128) FP8 weights (qwen3_weights.cc:131-182 loads
// them; Linear::validate, linear.cc:45-50, rejects them on the reference's
// path, so the arithmetic is the dequantized fp32 weight of dequantize_2d fed
// to the canonical GEMM dot): y[m,n] = bf16(sum_k x[m,k] * (decode(q[n,k]) *
// s[n/128][k/128])).
void orc_gemm_fp8(const float* x, const uint8_t* q, const float* s, float* y, int64_t M, int64_t N, int64_t K,
                  int round_out) {
    const int64_t sk = (K + 127) / 128;
#pragma omp parallel
    {
        std::vector<float> w(static_cast<size_t>(K));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t k = 0; k < K; ++k) w[k] = orc_fp8_decode(q[n * K + k]) * s[(n / 128) * sk + k / 128];
            for (int64_t m = 0; m < M; ++m) y[m * N + n] = store(gemm_dot(x + m * K, w.data(), K), round_out);
        }
    }
}

}  // extern "C"
