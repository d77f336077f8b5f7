/* hai_engine.h -- C ABI of the MI355X verify engine (C++ host, libhybridai.so).
 *
 * The engine owns a synthetic Qwen3.5-style hybrid model resident in HBM and
 * runs the speculative MTP decode of Generator::generate
 * (src/generator.cc:545-1117 in the reference) on one GPU:
 *   prefill -> MTP prefill -> rounds of {draft x k, verify (k+1 rows),
 *   fused argmax/accept, commit or correction + MTP recovery}.
 * Differences of mechanism, not of result:
 *   - no cache clones: the KV cache and DeltaNet state roll back by committed
 *     length (state slots + a conv-input ring), the MTP cache by length;
 *   - the reject-path replay (generator.cc:935-1003) is replaced by one
 *     forward of the correction token on top of the committed prefix, and the
 *     MTP recovery row only computes what the cache keeps (K and V).
 *   Every emitted token, candidate and accepted count equals the reference
 *   state machine's (tests compare round by round with the CPU oracle).
 */
#ifndef HAI_ENGINE_H
#define HAI_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Qwen3Config fields used by the path (src/models/qwen3_config.h:16-47). */
typedef struct hai_model_config {
    int32_t hidden;
    int32_t num_layers;
    int32_t full_attention_interval; /* layer i is GQA iff (i+1) % interval == 0 */
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
} hai_model_config;

/* Weight formats: every Linear bf16, or the Linears the reference loads as
 * QuantizedWeight (qwen3_weights.cc:242-283, 347-366) stored FP8 E4M3 with
 * 128x128 fp32 block scales (embed, lm_head, MTP fc, in_proj_a/b stay bf16). */
#define HAI_WEIGHTS_BF16 0
#define HAI_WEIGHTS_FP8_BLOCK128 1

typedef struct hai_engine_options {
    int32_t max_context;      /* KV capacity per sequence (prompt + new + slack) */
    int32_t max_verify_tokens;/* largest k+1: up to 17 (width 16) for one
                                 sequence, 16 for batches; prompts prefill
                                 in chunks of min(this, 16) rows */
    int32_t device;           /* HIP device ordinal */
    int32_t use_graphs;       /* replay captured forwards (0 = plain launches) */
    int32_t weight_format;    /* HAI_WEIGHTS_* */
    int32_t max_batch;        /* sequences decoded in lockstep (0 or 1 = one) */
    int32_t mfma;             /* 1: tolerance mode: GEMMs of 4 or more rows
                                 (batches) and the attention on the matrix
                                 cores (bf16 or FP8 weights); 0: every GEMM
                                 and the attention on the bit-exact kernels */
    int32_t prefill_rows;     /* 0 (or at most the verify rows): prompts
                                 prefill through the verify step, 16 rows
                                 per sequence at a time (bit-exact when
                                 mfma = 0).  Above that, up to 8192: prompts
                                 prefill in chunks of this many rows per
                                 sequence on the matrix cores (tiled GEMMs,
                                 matrix-core attention, lm_head on the last
                                 row only): tolerance mode for the prompt,
                                 whatever mfma says for the decode */
} hai_engine_options;

/* Counters of GenerationResult (include/hybrid.h:65-94) that the path fills. */
typedef struct hai_spec_stats {
    int64_t rounds;
    int64_t proposed;
    int64_t accepted;
    int64_t rejected;
    int64_t corrections;
    int64_t replay_tokens;        /* the reference's replay count: next +
                                     accepted + correction per rejected
                                     round (this engine forwards only the
                                     correction row of those) */
    int64_t mtp_recovery_tokens;
    int64_t max_proposal_width;
    int64_t emitted;
    double prefill_seconds;
    double decode_seconds;        /* first round start .. last token */
    double draft_seconds;         /* host wall time, includes queueing */
    double verify_seconds;
    double correction_seconds;
    int64_t host_syncs;           /* waits of the host on the stream during
                                     the rounds: one per round, plus one for
                                     each round that ends in a correction */
} hai_spec_stats;

/* Per-round record, int32 x 16: [proposal_count, accepted, full,
 * correction(-1), next_target, emitted_before, mtp_len_after,
 * target_len_after, cand0..cand7] -- the CPU oracle writes the same. */
#define HAI_ROUND_RECORD 16

void* hai_engine_create(const hai_model_config* cfg, const hai_engine_options* opt);
void hai_engine_destroy(void* engine);
const char* hai_engine_last_error(void* engine);
/* Fill every weight with the synthetic generator (bit-identical to the
 * oracle's orc_model_create with the same seed/std; with FP8 weights, to
 * orc_model_create + orc_model_quantize_fp8: the bf16 weight quantised with
 * synthetic U(0.5,2)/448 block scales). */
int hai_engine_init_synthetic(void* engine, uint64_t seed, float std_dev);
/* Copy one bf16 weight tensor (reference layout) to host memory; -1 for an
 * unknown id or a tensor held as FP8. */
int64_t hai_engine_read_tensor(void* engine, uint32_t tensor_id, uint16_t* out, int64_t capacity);

/* Checkpoints on disk (the reference's Qwen3Config::load_json,
 * models/qwen3_config.cc:12-206, SafeTensorLoader, io/safetensor_loader.cc:
 * 50-406, and Qwen3WeightLoader, models/qwen3_weights.cc:196-380).
 *   hai_model_config_load: <dir>/config.json into cfg (text_config fields
 *     first; head_dim from hidden / heads when absent; rope_theta and the
 *     rotary fraction from rope_parameters; layer_types checked against the
 *     interval), its eos_token_id(s) into eos_ids (n_eos = how many the
 *     config lists) and, when weight_format is not null, the format of the
 *     checkpoint's QuantizedWeight Linears (HAI_WEIGHTS_BF16: BF16;
 *     HAI_WEIGHTS_FP8_BLOCK128: F8_E4M3 + weight_scale_inv); a message on
 *     failure.  Host only: no device is touched.
 *   hai_engine_load_checkpoint: every weight of an engine created from that
 *     config and format, from <dir>/model.safetensors or the shards listed by
 *     <dir>/model.safetensors.index.json, by the reference's tensor names
 *     (model.language_model.layers.{i}.*, mtp.*, lm_head.weight); shapes and
 *     dtypes checked (BF16, F32 holding bf16 numbers, FP8 E4M3 with a BF16 or
 *     F32 128 x 128 scale grid). */
int hai_model_config_load(const char* dir, hai_model_config* cfg, int64_t* eos_ids, int64_t eos_capacity,
                          int64_t* n_eos, int32_t* weight_format, char* message, int64_t message_capacity);
int hai_engine_load_checkpoint(void* engine, const char* dir);
uint64_t hai_engine_weight_bytes(void* engine);

/* generate_* return the number of emitted tokens, or -status on failure. */

/* Prefill-only forward from empty caches: post-final-norm hidden [T,H] and
 * logits [T,V] as bf16 bits (either may be NULL). */
int hai_engine_forward(void* engine, const int32_t* ids, int64_t T, uint16_t* hidden, uint16_t* logits);
int hai_engine_generate_greedy(void* engine, const int32_t* prompt, int64_t P, int64_t max_new,
                               const int32_t* eos, int64_t n_eos, int32_t* out_tokens);
int hai_engine_generate_speculative(void* engine, const int32_t* prompt, int64_t P, int64_t max_new,
                                    int64_t width, const int32_t* eos, int64_t n_eos,
                                    const int32_t* draft_override, int64_t n_override,
                                    int32_t* out_tokens, hai_spec_stats* stats, int32_t* round_log,
                                    int64_t round_log_cap);

/* Batched decode: the engine's B = max_batch sequences, prompts [B][P] of
 * one length, decoded in lockstep rounds (one batched draft per chain
 * position, one verify of B x (k+1) rows, one batched correction forward for
 * the rejected sequences).  Each sequence follows the reference state
 * machine on its own: its tokens, round records and counters equal its
 * single-sequence decode.  out_tokens [B][max_new], n_out [B], stats [B],
 * round_log [B][round_log_cap][HAI_ROUND_RECORD] (NULL allowed),
 * draft_override [B][n_override] (NULL allowed).  Returns 0 or -status. */
int hai_engine_generate_speculative_batch(void* engine, const int32_t* prompts, int64_t P,
                                          int64_t max_new, int64_t width, const int32_t* eos,
                                          int64_t n_eos, const int32_t* draft_override,
                                          int64_t n_override, int32_t* out_tokens, int64_t* n_out,
                                          hai_spec_stats* stats, int32_t* round_log,
                                          int64_t round_log_cap);
/* Prefill-only forward of ids [B][T] for all B sequences: hidden [B][T][H],
 * logits [B][T][V] (either may be NULL). */
int hai_engine_forward_batch(void* engine, const int32_t* ids, int64_t T, uint16_t* hidden,
                             uint16_t* logits);
int64_t hai_engine_batch(void* engine);

/* Benchmark hooks.  hai_engine_prefill + hai_engine_spec_rounds run the same
 * loop as generate_speculative split so the caller can time rounds; the
 * verify-step profile replays n verify forwards of T rows at the current
 * context with events around the whole step and around every GEMM launch. */
typedef struct hai_verify_profile {
    double verify_ms;          /* mean wall of one verify step (forward+accept) */
    double gemm_ms;            /* mean time of the step's GEMM launches replayed
                                  back to back between two events */
    double gemm_bytes;         /* weight bytes streamed by GEMMs per step */
    double gemm_launches;      /* GEMM launches per step */
    double step_bytes;         /* algorithmic bytes per step (weights+KV+state) */
    double draft_ms;           /* mean wall of one draft step (MTP fwd+lm_head+argmax) */
    double draft_bytes;
} hai_verify_profile;

/* prompt is [B][P]; out_tokens [B][out_capacity]; n_out [B]; stats summed
 * over the sequences. */
int hai_engine_prefill(void* engine, const int32_t* prompt, int64_t P, int64_t max_new);
int hai_engine_spec_rounds(void* engine, int64_t rounds, int64_t width, int32_t* out_tokens,
                           int64_t out_capacity, int64_t* n_out, hai_spec_stats* stats);
/* Draft overrides for hai_engine_spec_rounds (benchmark legs with a chosen
 * acceptance pattern): tokens [B][n] replace the MTP proposal for output
 * position pos < n of each sequence, as the override of
 * generate_speculative does, but from a device copy made once here (no host
 * round trip per draft).  tokens == NULL or n == 0 clears them. */
int hai_engine_set_draft_override(void* engine, const int32_t* tokens, int64_t n);
/* Prefill mode of the next prompts: rows <= the verify rows (0 included)
 * prefill through the verify step (bit-exact when mfma = 0), larger values
 * up to the engine's hai_engine_options::prefill_rows run the fast prefill
 * in chunks of that many rows.  Larger values than the engine was created
 * for are rejected (its buffers are sized then). */
int hai_engine_set_prefill_rows(void* engine, int64_t rows);
int hai_engine_profile_verify(void* engine, int64_t T, int64_t iters, hai_verify_profile* out);

#ifdef __cplusplus
}
#endif

#endif /* HAI_ENGINE_H */
