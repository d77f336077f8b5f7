/* oracle.h -- TEST INFRASTRUCTURE ONLY (parity oracle for the MTP verify path).
 *
 * A CPU restatement of Dustray/Vicold.HybridAI's speculative MTP decode path
 * (src/generator.cc:545-1117) and of the math of the device kernels it runs
 * (src/backends/hip/hip_kernels.hip, hip_fused_kernels.hip).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library; the product path never links or calls it.
 *
 * Conventions: every tensor argument is a float array.  bf16 tensors are
 * passed as their exact fp32 values; when round_out != 0 a result is rounded
 * to bf16 (RNE) at the same point where the reference stores bf16, otherwise
 * it is left in fp32 (the reference's FP32 kernel instantiations, which its
 * known-answer tests use).
 */
#ifndef HYBRIDAI_ORACLE_H
#define HYBRIDAI_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- canonical primitives (pinned against libm in the tests) ---- */
void orc_exp_array(const float* x, float* y, int64_t n);
void orc_log1p_array(const float* x, float* y, int64_t n);
void orc_bf16_round_array(const float* x, float* y, int64_t n);

/* ---- ops ---- */
/* y[m,n] = sum_k x[m,k] w[n,k]; W is [N,K] row-major (linear.cc:137-155). */
void orc_gemm(const float* x, const float* w, float* y, int64_t M, int64_t N,
              int64_t K, int round_out);
/* rmsnorm_kernel (hip_kernels.hip:105-137): y = x*inv*(w + unit_offset). */
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows,
                 int64_t H, float eps, int unit_offset, int round_out);
void orc_add(const float* a, const float* b, float* y, int64_t n, int round_out);
/* silu_mul_kernel (hip_kernels.hip:164-175). */
void orc_silu_mul(const float* g, const float* u, float* y, int64_t n,
                  int round_out);
/* embedding_gather_kernel (hip_kernels.hip:88-103): out-of-range ids -> 0. */
void orc_embedding(const float* table, const int64_t* ids, float* y,
                   int64_t n_ids, int64_t V, int64_t H);
/* cos/sin of theta = pos / base^(2p/R), tables [npos][R/2]. */
void orc_rope_table(float* cos_t, float* sin_t, int64_t pos0, int64_t npos,
                    int64_t R, float base);
/* q_gate_rmsnorm_rope_kernel (hip_fused_kernels.hip:87-141). src is
 * [T, nq, 2D] with per-head [q | gate]; q is single-rounded. */
void orc_q_gate_rmsnorm_rope(const float* src, const float* w, float* q_out,
                             float* gate_out, int64_t T, int64_t nq, int64_t D,
                             int64_t R, int64_t pos0, float base, float eps,
                             int unit_offset, int round_out);
/* K path of GatedGQAAttention (attention.cc:459-464): RMSNorm(+1) stored,
 * then partial rotate-half RoPE (hip_kernels.hip:192-221) stored again. */
void orc_k_rmsnorm_rope(const float* src, const float* w, float* k_out,
                        int64_t T, int64_t nkv, int64_t D, int64_t R,
                        int64_t pos0, float base, float eps, int round_out);
/* partial_rope_kernel alone (used by the reference's SplitAndPartialRope KAT). */
void orc_partial_rope(const float* src, float* dst, int64_t T, int64_t heads,
                      int64_t D, int64_t R, int64_t pos0, float base,
                      int round_out);
/* Multi-query causal GQA over a cache that already holds the T new rows
 * (cached_gqa_head256_wave64_kernel, hip_kernels.hip:759-844).  q/gate are
 * [T, nq, D]; caches are [>=cache_len, nkv, D]; query t sits at position
 * cache_len - T + t.  gate may be NULL. */
void orc_attention(const float* q, const float* gate, const float* kc,
                   const float* vc, float* out, int64_t T, int64_t cache_len,
                   int64_t nq, int64_t nkv, int64_t D, int round_out);
/* deltanet_grouped_conv_kernel (hip_kernels.hip:871-912); conv_state is
 * [C, Kc-1] and is shifted in place. */
void orc_deltanet_conv(const float* qkv, const float* w, float* conv_state,
                       float* q, float* k, float* v, int64_t T, int64_t nk,
                       int64_t nv, int64_t dk, int64_t dv, int64_t Kc,
                       int round_out);
/* deltanet_recurrent_kernel (hip_kernels.hip:985-1095); state is
 * [nv, dk, dv] fp32, updated in place. */
void orc_deltanet_recurrent(const float* q, const float* k, const float* v,
                            const float* a, const float* b, const float* z,
                            const float* a_log, const float* dt_bias,
                            const float* norm_w, float* state, float* out,
                            int64_t T, int64_t nk, int64_t nv, int64_t dk,
                            int64_t dv, float eps, int round_out);
/* argmax_rows (generator.cc:325-360): first maximum, NaN never wins. */
void orc_argmax_rows(const float* x, int64_t* out, int64_t rows, int64_t cols);

/* ---- FP8 E4M3 weights (fp8_dequant.cc:12-146) ---- */
float orc_fp8_decode(uint8_t v);
void orc_fp8_decode_array(const uint8_t* q, float* y, int64_t n);
/* RNE encode saturating at +-448; NaN -> 0. */
void orc_fp8_encode_array(const float* x, uint8_t* q, int64_t n);
void orc_fp8_dequant_2d(const uint8_t* q, const float* s, float* w, int64_t rows,
                        int64_t cols, int64_t block_rows, int64_t block_cols);
/* y = bf16(x . (decode(q) * s[n/128][k/128])^T), L64 order; scales are
 * [ceil(N/128)][ceil(K/128)] fp32. */
void orc_gemm_fp8(const float* x, const uint8_t* q, const float* s, float* y,
                  int64_t M, int64_t N, int64_t K, int round_out);

/* ---- synthetic model ---- */
typedef struct orc_config {
    int32_t hidden;
    int32_t num_layers;
    int32_t full_attention_interval;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t rope_dim;
    int32_t lin_qk_heads;
    int32_t lin_v_heads;
    int32_t lin_k_dim;
    int32_t lin_v_dim;
    int32_t conv_kernel;
    int32_t ffn;
    int32_t vocab;
    int32_t mtp_layers;
    float rms_eps;
    float rope_theta;
} orc_config;

typedef struct orc_spec_stats {
    int64_t rounds;
    int64_t proposed;
    int64_t accepted;
    int64_t rejected;
    int64_t corrections;
    int64_t replay_tokens;
    int64_t mtp_recovery_tokens;
    int64_t max_proposal_width;
    int64_t mtp_cache_clones;
    int64_t target_cache_clones;
} orc_spec_stats;

/* Per-round log record (int32 x 16): [proposal_count, accepted, full,
 * correction(-1 if none), next_target, emitted_before, mtp_len_after,
 * target_len_after, cand0..cand7]. */
#define ORC_ROUND_RECORD 16

uint16_t orc_synthetic_weight_bits(uint64_t seed, uint32_t tensor_id,
                                   uint64_t index, float std_dev);
int orc_set_threads(int n);  /* OpenMP threads (n <= 0: query only) */
void orc_synthetic_prompt(uint64_t seed, int64_t n, int64_t vocab,
                          int32_t* out);

void* orc_model_create(const orc_config* cfg, uint64_t seed, float std_dev);
void orc_model_destroy(void* model);
/* Synthetic FP8 block scales of one tensor: s_i = (0.5 + 1.5 u_i) / 448 in
 * fp32, u_i = (splitmix64(key + i) >> 40) * 2^-24 with key the stream key
 * of id tensor_id + 2^20 (row-major over the [ceil(rows/128)][ceil(cols/128)]
 * block grid). */
void orc_fp8_synthetic_scales(uint64_t seed, uint32_t tensor_id, int64_t n,
                              float* out);
/* Turns every Linear the reference loads as a QuantizedWeight
 * (qwen3_weights.cc:242-283, 347-366: in_proj_qkv, in_proj_z, out_proj,
 * q/k/v/o_proj, gate/up/down_proj) into its FP8 E4M3 Block2D(128x128)
 * form: q = encode(w / s), and the Linear then uses dequantize_2d's
 * decode(q) * s (fp8_dequant.cc:28-146).  in_proj_a/b, conv, norms, fc,
 * embed and lm_head stay bf16, as the reference loads them. */
int orc_model_quantize_fp8(void* model);
/* Copies one synthetic tensor (decoded fp32) into out; returns elements or
 * -1 when the id is unknown. */
int64_t orc_model_tensor(void* model, uint32_t tensor_id, float* out,
                         int64_t capacity);
/* Full target forward from empty caches (prefill): hidden is the
 * post-final-norm hidden [T,H], logits [T,V]. */
int orc_forward(void* model, const int32_t* ids, int64_t T, float* hidden,
                float* logits);
int orc_generate_greedy(void* model, const int32_t* prompt, int64_t P,
                        int64_t max_new, const int32_t* eos, int64_t n_eos,
                        int32_t* out_tokens);
/* generator.cc:545-1117 restated.  draft_override[e] (when e < n_override)
 * replaces the MTP argmax for the candidate at emitted position e. */
int orc_generate_speculative(void* model, const int32_t* prompt, int64_t P,
                             int64_t max_new, int64_t width,
                             const int32_t* eos, int64_t n_eos,
                             const int32_t* draft_override,
                             int64_t n_override, int32_t* out_tokens,
                             orc_spec_stats* stats, int32_t* round_log,
                             int64_t round_log_cap);

/* ---- inspection hooks for the parity tests ---- */
/* Overwrites one tensor (n elements, the tensor's size); 0 or -1. */
int orc_model_set_tensor(void* model, uint32_t tensor_id, const float* data,
                         int64_t n);
/* qwen_mtp_forward_reference (generator.cc:139-183) over `rows` rows on a
 * fresh MTP cache, as the MTP prompt prefill runs it (generator.cc:673-699):
 * row r pairs emb(ids[r]) with hidden[r] at RoPE position r.  out [rows,H];
 * k_cache / v_cache (optional) receive the cache rows [rows, nkv, D]. */
int orc_mtp_forward(void* model, const int32_t* ids, const float* hidden,
                    int64_t rows, float* out, float* k_cache, float* v_cache);
/* The MTP cache the last orc_generate_speculative call left (its length is
 * returned; up to cap_rows rows [len, nkv, D] are copied). */
int64_t orc_last_mtp_cache(void* model, float* k, float* v, int64_t cap_rows);

#ifdef __cplusplus
}
#endif

#endif
