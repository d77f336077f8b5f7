/* hai_kernels.h -- C ABI of the gfx950 kernels for the HybridAI MTP verify path.
 *
 * This is the thin layer through which the C++ host (MI355X Backend and the
 * verify engine) reaches HIP.  It replaces the reference's launcher free
 * functions (src/backends/hip/hip_kernels.h:12-95,
 * src/backends/hip/hip_fused_kernels.h:14-26) and the rocBLAS call inside
 * HipBackend::gemm (src/backends/hip/hip_backend.cc:697-809).
 *
 * Rules shared by every entry point:
 *   - pointers are device pointers owned by the caller; nothing here
 *     allocates except hai_malloc; workspaces are passed in;
 *   - calls are asynchronous on `stream` (NULL = the null stream); the return
 *     value is the argument-check / launch status, device faults surface at
 *     the next synchronisation;
 *   - bf16 tensors are uint16 bit patterns, stores round to nearest even;
 *   - the arithmetic follows one canonical order shared with the CPU oracle
 *     (IEEE fma on the VALU; long sums in "L64" order: element k to lane
 *     (k/8) mod 64, per-lane fma in increasing k, xor-butterfly 32..1), so
 *     results are bit-identical to it and independent of batch and tiling.
 */
#ifndef HAI_KERNELS_H
#define HAI_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the numbers match hybridai::StatusCode (src/core/status.h:9-21). */
enum {
    HAI_OK = 0,
    HAI_ERR_INVALID_ARGUMENT = 1,
    HAI_ERR_OUT_OF_MEMORY = 2,
    HAI_ERR_NOT_IMPLEMENTED = 3,
    HAI_ERR_INVALID_DEVICE = 5,
    HAI_ERR_UNSUPPORTED_DTYPE = 6,
    HAI_ERR_FILE_NOT_FOUND = 7,
    HAI_ERR_INVALID_MODEL = 8,
    HAI_ERR_BACKEND = 9,
};

/* Text of the last error raised on the calling thread. */
const char* hai_last_error(void);

/* ------------------------------------------------------------------ runtime
 * Replaces the HIP runtime calls made by HipBackend (hip_backend.cc:425-695). */
int hai_device_count(int* count);
int hai_set_device(int device);
int hai_get_device(int* device);
int hai_malloc(void** ptr, size_t bytes);
int hai_free(void* ptr);
int hai_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int hai_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int hai_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* height rows of width bytes, host rows src_pitch apart to device rows
 * dst_pitch apart (checkpoint tensors into stacked / interleaved weights). */
int hai_memcpy_h2d_2d(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width, size_t height,
                      void* stream);
/* Copy in whichever direction the two addresses imply (hipMemcpyDefault). */
int hai_memcpy(void* dst, const void* src, size_t bytes, void* stream);
/* Page-locked host memory (MemoryType::HostPinned buffers). */
int hai_host_malloc(void** ptr, size_t bytes);
int hai_host_free(void* ptr);
int hai_memset(void* dst, int value, size_t bytes, void* stream);
int hai_stream_create(void** stream);
int hai_stream_destroy(void* stream);
int hai_stream_synchronize(void* stream);
int hai_device_synchronize(void);
int hai_event_create(void** event);
int hai_event_destroy(void* event);
int hai_event_record(void* event, void* stream);
int hai_event_synchronize(void* event);
/* Work queued on `stream` after this call waits for `event` (Event::wait). */
int hai_stream_wait_event(void* stream, void* event);
int hai_event_elapsed_ms(void* start, void* stop, float* ms);
/* Stream capture into a replayable graph (replaces per-op launches). */
int hai_graph_begin_capture(void* stream);
int hai_graph_end_capture(void* stream, void** graph_exec);
int hai_graph_launch(void* graph_exec, void* stream);
int hai_graph_destroy(void* graph_exec);

/* ------------------------------------------------------------------ linear
 * Y[m, n] = sum_k X[m, k] W[n, k] with W stored [N, K] row-major
 * (Linear::forward_into, linear.cc:117-179; rocblas_gemm_ex at
 * hip_backend.cc:784-789).  Requirements: K % 8 == 0, ldx % 8 == 0,
 * 16-byte aligned X and W.  Any M: a call of more than 16 rows runs them in
 * 16-row batches within one launch, the batches of a weight row group on
 * one XCD one after another, so each weight is read from HBM about once per
 * launch; rows are independent and every row's sum is in the same order, so
 * the batching does not change any bit.
 * Epilogues:
 *   HAI_EPI_STORE     y = bf16(acc)
 *   HAI_EPI_RESIDUAL  y = bf16(res + bf16(acc))   (make_residual fused,
 *                     qwen_reference.cc:121-144; y may alias res)
 *   HAI_EPI_SILU_MUL  weight rows interleave (gate_f, up_f); writes N/2
 *                     columns y = bf16(silu(bf16(g)) * bf16(u))
 *                     (qwen_mlp_reference + silu_mul_kernel,
 *                     qwen_reference.cc:146-175, hip_kernels.hip:164-175). */
enum { HAI_EPI_STORE = 0, HAI_EPI_RESIDUAL = 1, HAI_EPI_SILU_MUL = 2 };
int hai_gemm_bf16(void* y, int64_t ldy, const void* x, int64_t ldx,
                  const void* w, int64_t M, int64_t N, int64_t K, int epilogue,
                  const void* res, int64_t ld_res, void* stream);
/* The model's RMSNorm followed by a linear layer in one launch: the
 * qwen_rmsnorm_reference -> Linear pair of qwen_reference.cc:108-119 and
 * linear.cc:117-179 (the input / post-attention norms before the first
 * projection of every sub-layer, and the final norm before lm_head).
 * y = epilogue(rmsnorm(x; norm_w, eps, unit_offset) . W^T), bit-identical to
 * hai_rmsnorm_bf16 then hai_gemm_bf16.  xn_out, if not null, also receives
 * the normalised rows (ld_xn).  When M > 16 or M * K exceeds
 * HAI_GEMM_RMSNORM_FUSED_MAX the rows do not fit the on-chip prologue: the
 * call then runs the two kernels and needs xn_out as their intermediate. */
#define HAI_GEMM_RMSNORM_FUSED_MAX 16384
int hai_gemm_rmsnorm_bf16(void* y, int64_t ldy, const void* x, int64_t ldx,
                          const void* norm_w, float eps, int unit_offset,
                          void* xn_out, int64_t ld_xn, const void* w,
                          int64_t M, int64_t N, int64_t K, int epilogue,
                          const void* res, int64_t ld_res, void* stream);

/* FP8 E4M3 weights with 128x128 fp32 block scales (QuantizedWeight,
 * ScaleLayout::Block2D, qwen3_weights.cc:131-182), dequantized in the weight
 * stream exactly as FP8Dequantizer::dequantize_2d (fp8_dequant.cc:12-146):
 * w[n,k] = decode_e4m3(wq[n,k]) * scales[sr(n)][k/128] (fp32), then the bf16
 * GEMM's arithmetic and epilogues.  wq is [N, K] bytes; each scale row holds
 * ceil(K/128) floats.  sr(n) = scale_rows[n] when scale_rows is given (rows
 * of several checkpoint tensors concatenated, each with its own 128x128
 * grid), else n / 128; for HAI_EPI_SILU_MUL without a map the rows
 * interleave (gate_f, up_f) and scales are [2][ceil(N/2/128)][...] (gate
 * blocks, then up blocks).  K <= 32768, M <= 16 per call; x 16-byte and wq
 * 8-byte aligned.  epilogue may carry HAI_FP8_NO_SPECIAL_CODES: the caller
 * guarantees that wq holds no 0x7F / 0xFF code (the +-480 codes of the
 * reference's decoder, NaN in OCP E4M3, which a quantiser saturating at 448
 * never writes), and the per-word check for them is skipped. */
enum { HAI_FP8_NO_SPECIAL_CODES = 0x100 };
int hai_gemm_fp8_bf16(void* y, int64_t ldy, const void* x, int64_t ldx,
                      const void* wq, const float* scales,
                      const int32_t* scale_rows, int64_t M, int64_t N,
                      int64_t K, int epilogue, const void* res, int64_t ld_res,
                      void* stream);
/* RMSNorm(+offset) of the rows x [M, K] fused into the FP8 linear layer, as
 * hai_gemm_rmsnorm_bf16 is for bf16 weights: the qwen_rmsnorm_reference ->
 * Linear pair of qwen_reference.cc:108-119 and linear.cc:117-179 over a
 * QuantizedWeight (qwen3_weights.cc:131-182).  The normalised rows are
 * bit-identical to hai_rmsnorm_bf16's;
 * xn_out (optional) receives the normalised rows.  Above
 * HAI_GEMM_RMSNORM_FUSED_MAX elements it runs rmsnorm then the GEMM and needs
 * xn_out. */
int hai_gemm_rmsnorm_fp8_bf16(void* y, int64_t ldy, const void* x,
                              int64_t ldx, const void* norm_w, float eps,
                              int unit_offset, void* xn_out, int64_t ld_xn,
                              const void* wq, const float* scales,
                              const int32_t* scale_rows, int64_t M, int64_t N,
                              int64_t K, int epilogue, const void* res,
                              int64_t ld_res, void* stream);
/* Block-scaled E4M3 quantisation of a bf16 weight [rows, cols] (row pitch
 * ldw elements) into codes with row pitch ldq bytes, given its scales
 * [ceil(rows/128)][ceil(cols/128)] fp32: q = E4M3 of the fp32 quotient w / s,
 * rounded to nearest even and saturated at +-448 (codes 0x7F / 0xFF are
 * never produced).  The quantiser of the synthetic FP8 checkpoints; no
 * reference counterpart (the reference loads FP8 checkpoints as stored,
 * qwen3_weights.cc:131-182). */
int hai_fp8_quantize_bf16(void* q, int64_t ldq, const void* w, int64_t ldw,
                          const float* scales, int64_t rows, int64_t cols,
                          void* stream);
/* Synthetic block scales s_i = (0.5 + 1.5 u_i) / 448 (fp32 arithmetic),
 * u_i = (splitmix64(key + i) >> 40) * 2^-24, key the synthetic-weight stream
 * key of tensor id tensor_id + 2^20: U(0.5, 2)/448 as the FP8 benchmark
 * configuration states, bit-identical to the CPU oracle's. */
int hai_fill_synthetic_scales_f32(float* scales, int64_t n, uint64_t seed,
                                  uint32_t tensor_id, void* stream);

/* ------------------------------------------------------------------ norms
 * rmsnorm_kernel (hip_kernels.hip:105-137): y = x * inv * (w + offset),
 * inv = 1/sqrt(sum x^2 / H + eps).  Strided rows so the MTP concat
 * (generator.cc:24-66) is written in place. */
int hai_rmsnorm_bf16(void* y, int64_t ldy, const void* x, int64_t ldx,
                     const void* w, int64_t rows, int64_t H, float eps,
                     int unit_offset, void* stream);
/* add_kernel (hip_kernels.hip:43-51). */
int hai_add_bf16(void* y, const void* a, const void* b, int64_t n, void* stream);
/* silu_mul_kernel (hip_kernels.hip:164-175). */
int hai_silu_mul_bf16(void* y, const void* g, const void* u, int64_t n,
                      void* stream);
/* embedding_gather_kernel (hip_kernels.hip:88-103); ids are int64, ids out
 * of [0, V) produce a zero row. */
int hai_embedding_gather_bf16(void* y, const void* table, const int64_t* ids,
                              int64_t n_ids, int64_t V, int64_t H, void* stream);

/* RoPE tables: cos/sin[pos][p] of theta = pos / base^(2p/R), p < R/2,
 * computed by the caller on the host in double precision. */

/* q_gate_rmsnorm_rope_kernel (hip_fused_kernels.hip:87-141).  Row m = b*T+t
 * of src holds nq heads of [q(D) | gate(D)] starting at column 0.  Query
 * position = (lens ? lens[b] : 0) + pos_add + t. */
int hai_q_gate_rmsnorm_rope_bf16(void* q_out, void* gate_out, const void* src,
                                 int64_t ld_src, const void* q_norm,
                                 const float* rope_cos, const float* rope_sin,
                                 int64_t rope_positions, int64_t B, int64_t T,
                                 int64_t nq, int64_t D, int64_t R,
                                 const int32_t* lens, int32_t pos_add,
                                 float eps, void* stream);
/* K path of GatedGQAAttention (attention.cc:459-464: RMSNorm(+1) -> bf16
 * -> partial RoPE -> bf16) fused with append_kv_cache_kernel
 * (hip_kernels.hip:295-308).  Caches are [B][cap][nkv][D]; row t of
 * sequence b goes to position (lens ? lens[b] : 0) + pos_add + t.  Values
 * are copied unchanged.  src_k and src_v 16-byte aligned, ld_src a multiple
 * of 8. */
int hai_kv_rmsnorm_rope_append_bf16(void* k_cache, void* v_cache, int64_t cap,
                                    const void* src_k, const void* src_v,
                                    int64_t ld_src, const void* k_norm,
                                    const float* rope_cos,
                                    const float* rope_sin,
                                    int64_t rope_positions, int64_t B,
                                    int64_t T, int64_t nkv, int64_t D,
                                    int64_t R, const int32_t* lens,
                                    int32_t pos_add, float eps, void* stream);
/* Both of the above in one launch for the attention projection rows
 * [q+gate (2 nq D) | k (nkv D) | v (nkv D)] of src (the layout of the fused
 * q|gate|k|v Linear): the same outputs bit for bit, one kernel instead of
 * two. */
int hai_qkv_rmsnorm_rope_append_bf16(void* q_out, void* gate_out,
                                     void* k_cache, void* v_cache, int64_t cap,
                                     const void* src, int64_t ld_src,
                                     const void* q_norm, const void* k_norm,
                                     const float* rope_cos,
                                     const float* rope_sin,
                                     int64_t rope_positions, int64_t B,
                                     int64_t T, int64_t nq, int64_t nkv,
                                     int64_t D, int64_t R,
                                     const int32_t* lens, int32_t pos_add,
                                     float eps, void* stream);
/* partial_rope_kernel (hip_kernels.hip:192-221) as called by
 * Backend::partial_rope: rotate-half on the first R dims of each of the
 * `heads` D-wide heads of T rows, position pos0 + t, dims past R copied;
 * rope_cos / rope_sin are [rope_positions][R/2] tables (theta =
 * pos / base^(2p/R), evaluated in double and rounded to float). */
int hai_partial_rope_bf16(void* dst, const void* src, int64_t T, int64_t heads,
                          int64_t D, int64_t R, const float* rope_cos,
                          const float* rope_sin, int64_t rope_positions,
                          int64_t pos0, void* stream);
/* Plain row append (append_kv_cache_kernel) for callers that already hold
 * the final K/V rows (Backend::append_kv_cache). */
int hai_append_kv_bf16(void* k_cache, void* v_cache, int64_t cap,
                       const void* k, const void* v, int64_t B, int64_t T,
                       int64_t row_width, const int32_t* lens, int32_t pos_add,
                       void* stream);

/* ------------------------------------------------------------------ attention
 * Multi-query causal gated GQA over the cache (cached_gqa_head256_wave64
 * kernel, hip_kernels.hip:759-844, and the T=1 variant :567-675).  The
 * cache of sequence b holds L_b = (lens ? lens[b] : 0) + len_add rows
 * including the T new ones; query t attends keys 0..L_b-T+t.  q/gate/out
 * are [B*T][nq][D]; gate may be NULL.  scratch must hold
 * hai_gqa_scratch_bytes(B, T, nq, D, max_len) bytes (SIZE_MAX when the size
 * overflows or an argument is negative); max_len bounds every L_b and sizes
 * the launch. */
size_t hai_gqa_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t D,
                             int64_t max_len);
int hai_gqa_verify_bf16(void* out, const void* q, const void* gate,
                        const void* k_cache, const void* v_cache, int64_t cap,
                        void* scratch, int64_t B, int64_t T, int64_t nq,
                        int64_t nkv, int64_t D, const int32_t* lens,
                        int32_t len_add, int64_t max_len, void* stream);
/* hai_qkv_rmsnorm_rope_append_bf16 followed by hai_gqa_verify_bf16 in one
 * partial pass (+ the merge pass): the partial blocks normalise and rotate
 * their own query rows from the projection rows proj (ld_proj: [q_h | gate_h]
 * for the nq heads, then the nkv K heads, then the nkv V heads, rows b*T + t
 * at position L_b - T + t, L_b = (lens ? lens[b] : 0) + len_add), build the
 * K / V rows of the T new positions from them for the key chunks that hold
 * those positions and write them to the caches, and copy the gate halves to
 * gate_out ([B*T][nq][D]), which the merge pass reads.  Outputs, cache rows
 * and gate halves are bit-identical to the two calls (the normalised q rows
 * are not stored).  Removes one dependent launch per attention layer.
 * proj 16-byte aligned, ld_proj % 8 == 0; other arguments and the scratch
 * as the two calls. */
int hai_gqa_verify_fused_bf16(void* out, void* gate_out, const void* proj,
                              int64_t ld_proj, const void* q_norm,
                              const void* k_norm, const float* rope_cos,
                              const float* rope_sin, int64_t rope_positions,
                              int64_t R, float eps, void* k_cache,
                              void* v_cache, int64_t cap, void* scratch,
                              int64_t B, int64_t T, int64_t nq, int64_t nkv,
                              int64_t D, const int32_t* lens, int32_t len_add,
                              int64_t max_len, void* stream);
/* hai_gqa_verify_bf16 for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * same kernels and bit-identical results, with the split-KV partials in a
 * fixed 16 MiB device array the library holds on each GPU it runs on until
 * the process ends (HAI_GQA_NOALLOC_SCRATCH_BYTES), so no scratch argument
 * and no allocation.  No counterpart in the reference.  Calls whose
 * hai_gqa_scratch_bytes(B, T, nq, D, max_len) exceeds that size are
 * rejected.  All calls on one GPU share its array: calls that overlap on a
 * GPU (two streams, two threads) race and must be serialised by the caller.
 * The first call on a device resolves the array's address there
 * (hipGetSymbolAddress) with that device current. */
#define HAI_GQA_NOALLOC_SCRATCH_BYTES (16u << 20)
int hai_gqa_verify_noalloc_bf16(void* out, const void* q, const void* gate,
                                const void* k_cache, const void* v_cache,
                                int64_t cap, int64_t B, int64_t T, int64_t nq,
                                int64_t nkv, int64_t D, const int32_t* lens,
                                int32_t len_add, int64_t max_len, void* stream);
/* The same attention in tolerance mode, on the matrix cores (same reference
 * kernels as above; the batched verify / draft steps).  Q.K^T and P.V run
 * as bf16 MFMA with fp32 accumulation (P rounded to bf16), one online
 * softmax per wave over its own keys, merged per block and then across
 * blocks: results agree with hai_gqa_verify_bf16 to bf16 rounding, not bit
 * for bit.  A block serves up to 32 of a KV head's T * nq / nkv queries
 * (more take several blocks); q, the caches and scratch 16-byte aligned;
 * scratch must hold
 * hai_gqa_mfma_scratch_bytes(B, T, nq, D, max_len) bytes. */
size_t hai_gqa_mfma_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t D,
                                  int64_t max_len);
/* The scratch the call with these arguments takes on the current device (its
 * split plan depends on the blocks the device holds): at most
 * hai_gqa_mfma_scratch_bytes, far less for prompt chunks, whose query groups
 * alone fill the device.  Not monotonic in T: fewer rows can take more
 * splits, so a buffer for calls of up to T rows takes the largest value over
 * 1..T. */
size_t hai_gqa_mfma_plan_scratch_bytes(int64_t B, int64_t T, int64_t nq, int64_t nkv,
                                       int64_t D, int64_t max_len);
int hai_gqa_verify_mfma_bf16(void* out, const void* q, const void* gate,
                             const void* k_cache, const void* v_cache,
                             int64_t cap, void* scratch, int64_t B, int64_t T,
                             int64_t nq, int64_t nkv, int64_t D,
                             const int32_t* lens, int32_t len_add,
                             int64_t max_len, void* stream);

/* ------------------------------------------------------------------ DeltaNet
 * Fused grouped causal conv (deltanet_grouped_conv_kernel,
 * hip_kernels.hip:871-912) + gated delta rule (deltanet_recurrent_kernel,
 * :985-1095) + gated RMSNorm, for T tokens of B sequences.
 *   proj rows (ld_proj) hold [qkv(C) | z(nv*dv) | a(nv) | b(nv)] at the given
 *     column offsets, C = 2*nk*dk + nv*dv in flat [Q|K|V] channel order;
 *   conv_ring is [B][ring][C] raw inputs indexed by position % ring;
 *   state is [nslots][B][nv][dk*dv] fp32, each head column-tiled: entry
 *     (key i, value j) of the reference's [dk][dv] matrix, with
 *     i = g*(dk/4) + 4m + e (g, e < 4), is float ((m*dv + j)*4 + g)*4 + e;
 *     the state after sequence length L lives in slot L % nslots;
 *   rows b*T + t of proj / out belong to token t of sequence b, which has
 *     position (lens ? lens[b] : 0) + pos_add + t;
 *   a call of more than 16 tokens (prompt chunks) runs as launches of 16 in
 *   order, each continuing from the state and conv inputs the previous one
 *   left: the result equals one pass over the T tokens.
 * With write_all_slots the state after every token is kept (rollback by
 * length only, no copies); otherwise only the final state is written.
 * Needs min(T, 16) + Kc - 1 <= ring, and nslots >= T when write_all_slots. */
int hai_deltanet_verify_bf16(void* out, int64_t ld_out, const void* proj,
                             int64_t ld_proj, int64_t off_qkv, int64_t off_z,
                             int64_t off_a, int64_t off_b, const void* conv_w,
                             void* conv_ring, int64_t ring, float* state,
                             int64_t nslots, int write_all_slots,
                             const void* a_log, const void* dt_bias,
                             const void* norm_w, const int32_t* lens,
                             int32_t pos_add, int64_t B, int64_t T, int64_t nk,
                             int64_t nv, int64_t dk, int64_t dv, int64_t Kc,
                             float eps, void* stream);
/* hai_deltanet_verify_bf16 (same arguments, same bits) with each head's
 * value columns spread over several blocks (deltanet_recurrent_kernel,
 * hip_kernels.hip:985-1095, updates the columns independently) when B * nv
 * heads alone leave most CUs idle (fewer than 256).  The last block of a
 * head finishes its gated norm behind device-scope fences; measured on
 * MI355X this is slower than one block per head at the verify shapes (48
 * heads, T = 2: 31.6 us against 10.0 us; 11.5 us even without the fences),
 * so the engine does not use it.  The workspace
 * holds one counter per (sequence, head) and the heads' unrounded outputs;
 * it must be zeroed once before the first call (every call leaves the
 * counters zero again) and hold hai_deltanet_workspace_bytes(B, nv, dv)
 * bytes, 16-byte aligned.  Calls that overlap in time must not share a
 * workspace. */
size_t hai_deltanet_workspace_bytes(int64_t B, int64_t nv, int64_t dv);
int hai_deltanet_verify_ws_bf16(void* out, int64_t ld_out, const void* proj,
                                int64_t ld_proj, int64_t off_qkv, int64_t off_z,
                                int64_t off_a, int64_t off_b, const void* conv_w,
                                void* conv_ring, int64_t ring, float* state,
                                int64_t nslots, int write_all_slots,
                                const void* a_log, const void* dt_bias,
                                const void* norm_w, const int32_t* lens,
                                int32_t pos_add, int64_t B, int64_t T, int64_t nk,
                                int64_t nv, int64_t dk, int64_t dv, int64_t Kc,
                                float eps, void* workspace,
                                int64_t workspace_bytes, void* stream);
/* hai_deltanet_verify_bf16 with the a|b projection formed in the kernel
 * instead of read from proj: the in_proj_a / in_proj_b Linears of
 * qwen_reference.cc:205-258 (bf16 weights also when the model's other
 * Linears are FP8, qwen3_weights.cc:242-283), a_t[h] = xn_t . w_ab[h] and
 * b_t[h] = xn_t . w_ab[nv + h] over the normalised input rows xn (ld_xn, row
 * b*T + t), each computed in hai_gemm_bf16's order and rounded to bf16, so
 * the result is bit-identical to running that GEMM into the proj columns
 * first.  w_ab is [2*nv, H] row-major; 0 < H <= 8192, H % 8 == 0. */
int hai_deltanet_verify_ab_bf16(void* out, int64_t ld_out, const void* proj,
                                int64_t ld_proj, int64_t off_qkv, int64_t off_z,
                                const void* xn, int64_t ld_xn, const void* w_ab,
                                int64_t H, const void* conv_w, void* conv_ring,
                                int64_t ring, float* state, int64_t nslots,
                                int write_all_slots, const void* a_log,
                                const void* dt_bias, const void* norm_w,
                                const int32_t* lens, int32_t pos_add, int64_t B,
                                int64_t T, int64_t nk, int64_t nv, int64_t dk,
                                int64_t dv, int64_t Kc, float eps, void* stream);
/* hai_deltanet_verify_bf16 (or, with w_ab non-null, hai_deltanet_verify_ab_bf16:
 * off_a / off_b are then unused) with rollback records in place of the
 * per-token states: the rollback that deltanet_recurrent_kernel's callers
 * get from the reference's state snapshots (generator.cc:909-1021), at 1 KB
 * per token instead of a dk x dv fp32 state.
 *   records is [nslots][B][nv][dk + dv + 4] fp32
 *     (hai_deltanet_records_bytes, 16-byte aligned): every token at position
 *     p leaves in slot p % nslots the update it applied to the state,
 *     beta * k^ (dk floats), c_j = v_j - k^T (decay * S)_j for every value
 *     column j (dv) and decay, so that S' = fma(beta * k^, c, S * decay);
 *   only the final state of the call is stored (slot (L + T) % nslots);
 *   replay = 0: the call starts from the state held in slot L % nslots and
 *     stores its start positions L in base[b];
 *   replay = 1 (T <= 4): the call starts from the state of position base[b]
 *     (slot base[b] % nslots, as a replay = 0 call left it) and re-applies
 *     the records of positions base[b] .. L - 1 (written by that call), bit
 *     for bit the updates it made, before its own tokens; base is not
 *     changed.  A sequence with L - base[b] outside [0, min(nslots - 1, 16)]
 *     starts from slot L % nslots instead.
 * So after a replay = 0 call of T tokens, keeping any prefix of a + 1 of
 * them needs no copy: a replay = 1 call at L = base + a + 1 continues from
 * the state after that prefix.  Needs nslots > T; other arguments and
 * checks as hai_deltanet_verify_bf16 / _ab_bf16. */
size_t hai_deltanet_records_bytes(int64_t nslots, int64_t B, int64_t nv, int64_t dk, int64_t dv);
int hai_deltanet_verify_rec_bf16(void* out, int64_t ld_out, const void* proj,
                                 int64_t ld_proj, int64_t off_qkv, int64_t off_z,
                                 int64_t off_a, int64_t off_b, const void* xn,
                                 int64_t ld_xn, const void* w_ab, int64_t H,
                                 const void* conv_w, void* conv_ring, int64_t ring,
                                 float* state, int64_t nslots, float* records,
                                 int32_t* base, int replay, const void* a_log,
                                 const void* dt_bias, const void* norm_w,
                                 const int32_t* lens, int32_t pos_add, int64_t B,
                                 int64_t T, int64_t nk, int64_t nv, int64_t dk,
                                 int64_t dv, int64_t Kc, float eps, void* stream);
/* The same layer over a prompt chunk (the prefill's conv + recurrence +
 * gated RMSNorm, hip_kernels.hip:871-912, 985-1095), tolerance mode: the
 * chunkwise form of the gated delta rule over 32-token chunks (per chunk, in
 * parallel: conv, gates, norms, Gram matrices and the triangular solve; then
 * the state carried from chunk to chunk through dense products on the
 * matrix cores, split-bf16 operands within ~2^-16 of fp32 products), the
 * gated norm in a third kernel.  Sums regrouped, so equal to the canonical
 * recurrence to fp32 rounding, not bit for bit.  Arguments as
 * hai_deltanet_verify_bf16 (proj columns [qkv | z | a | b] at the offsets,
 * rows b*T + t; proj and conv_ring 4-byte aligned, ld_proj and off_qkv
 * even); only the final state is written (slot (L + T) % nslots), and the
 * conv ring's entries for the chunk's last Kc - 1 positions.  workspace
 * holds the unrounded outputs and the per-chunk records:
 * hai_deltanet_prefill_workspace_bytes(B, T, nv, dv) bytes, 16-byte
 * aligned. */
size_t hai_deltanet_prefill_workspace_bytes(int64_t B, int64_t T, int64_t nv, int64_t dv);
int hai_deltanet_prefill_bf16(void* out, int64_t ld_out, const void* proj,
                              int64_t ld_proj, int64_t off_qkv, int64_t off_z,
                              int64_t off_a, int64_t off_b, const void* conv_w,
                              void* conv_ring, int64_t ring, float* state,
                              int64_t nslots, const void* a_log,
                              const void* dt_bias, const void* norm_w,
                              const int32_t* lens, int32_t pos_add, int64_t B,
                              int64_t T, int64_t nk, int64_t nv, int64_t dk,
                              int64_t dv, int64_t Kc, float eps, void* workspace,
                              int64_t workspace_bytes, void* stream);
/* The reference's two-kernel DeltaNet contract (Backend::deltanet_grouped_conv
 * and Backend::deltanet_recurrent, hip_backend.cc:1357-1470), on the
 * reference's cache layouts:
 *   hai_deltanet_conv_bf16: qkv [T][C] flat [Q|K|V] -> q, k [T][nk*dk] and
 *     v [T][nv*dv] after the causal conv + SiLU; conv_state [C][Kc-1] (oldest
 *     first) is shifted in place (deltanet_grouped_conv_kernel,
 *     hip_kernels.hip:871-912);
 *   hai_deltanet_recurrent_bf16: gated delta rule + gated RMSNorm over T
 *     tokens with the fp32 state [nv][dk][dv] updated in place; a, b are the
 *     raw [T][nv] projections (decay and beta computed inside), z [T][nv*dv]
 *     (deltanet_recurrent_kernel, :985-1095).  Any T (16 tokens per launch,
 *     chained).  (dk, dv) in {(128,128), (64,64)}. */
int hai_deltanet_conv_bf16(void* q, void* k, void* v, void* conv_state,
                           const void* qkv, const void* conv_w, int64_t T,
                           int64_t nk, int64_t nv, int64_t dk, int64_t dv,
                           int64_t Kc, void* stream);
int hai_deltanet_recurrent_bf16(void* out, float* state, const void* q,
                                const void* k, const void* v, const void* a,
                                const void* b, const void* a_log,
                                const void* dt_bias, const void* norm_w,
                                const void* z, int64_t T, int64_t nk,
                                int64_t nv, int64_t dk, int64_t dv, float eps,
                                void* stream);

/* ------------------------------------------------------------------ argmax / accept
 * argmax_rows_kernel (hip_kernels.hip:1243-1274) with the CPU tie-break of
 * argmax_rows_reference (generator.cc:343-360): first maximum, NaN and -inf
 * never win, an all-invalid row gives 0.  scratch must hold
 * hai_argmax_scratch_bytes(rows, V). */
size_t hai_argmax_scratch_bytes(int64_t rows, int64_t V);
int hai_argmax_rows_bf16(int64_t* out, const void* logits, int64_t ld,
                         int64_t rows, int64_t V, void* scratch, void* stream);

/* Greedy acceptance of generator.cc:909-916 computed on the device, fused
 * with the argmax of the T = k+1 verify rows.  For sequence b:
 *   preds[b*T+t] = argmax(logits row b*T+t);
 *   a = longest prefix with preds[t] == ids[b*T+1+t] (t < k_b);
 *   result[b*4+0] = a, [1] = (a == k_b), [2] = ids[b*T] (the round's
 *   next_target), [3] = preds[b*T+a];
 *   target_len[b] += a + 1 (rows 0..a are committed, the rest rolls back);
 *   mtp_len[b] -= k_b - a unless fully accepted (MTP checkpoint[a]);
 *   next[b] = preds[b*T+a] (the target token after the committed rows);
 *   hidden row a is copied to rec_hidden[b] and, on full acceptance, row
 *   T-1 to h_prev[b].
 * n_draft holds k_b per sequence (T - 1 for every b when NULL); B <= 64
 * sequences of T <= 64 rows, one block per sequence. */
int hai_verify_argmax_accept_bf16(const void* logits, int64_t V,
                                  const void* hidden, int64_t H,
                                  const int64_t* ids, const int32_t* n_draft,
                                  int64_t B, int64_t T, int64_t* preds,
                                  int32_t* result, int32_t* target_len,
                                  int32_t* mtp_len, int64_t* next,
                                  void* rec_hidden, void* h_prev,
                                  void* scratch, void* stream);

/* dst[i] += (delta ? delta[i] : 0) + add for i < n: committed-length updates
 * kept on the stream (AttentionKVCache::length / DeltaNetCache::length
 * bookkeeping, attention.h:11-42, delta_net.h:11-55). */
int hai_add_i32(int32_t* dst, const int32_t* delta, int32_t add, int64_t n, void* stream);

/* Draft i (0 <= i < T - 1) of a round's chained MTP proposals, counted on the
 * device (the proposal loop of generator.cc:760-849, its EOS break at
 * :845-847): ndraft[b] becomes i + 1 when i == 0 and cap[b] > 0, or when
 * ndraft[b] == i, i < cap[b] and vids[b*T + i] (the candidate draft i - 1
 * wrote, [B][T] verify layout) is not one of the n_eos ids in eos; otherwise
 * it stays.  After the chain ndraft[b] is the proposal count that
 * hai_verify_argmax_accept_bf16 takes, with no host read per draft. */
int hai_draft_chain_count(int64_t i, const int64_t* vids, int64_t T, const int32_t* cap,
                          const int64_t* eos, int64_t n_eos, int32_t* ndraft, int64_t B,
                          void* stream);

/* dst[i * dst_stride] = src[i * src_stride] for i < n (token ids between the
 * [B][T] verify layout and per-sequence [B] vectors). */
int hai_copy_i64_strided(int64_t* dst, int64_t dst_stride, const int64_t* src,
                         int64_t src_stride, int64_t n, void* stream);
/* After the correction forward of a batch (one row per sequence): for every
 * sequence b whose round ended in a rejection (result[b*4+1] == 0, the
 * layout of hai_verify_argmax_accept_bf16), next[b] = corr_next[b],
 * h_prev[b] = corr_hidden[b] ([B][H] bf16), target_len[b] += 1 and
 * mtp_len[b] += 1 (the correction row and its MTP recovery row are
 * committed, generator.cc:960-1003); fully accepted sequences keep their
 * verify outcome. */
int hai_correction_commit_bf16(const int32_t* result, const int64_t* corr_next,
                               const void* corr_hidden, int64_t H, int64_t B,
                               int64_t* next, void* h_prev,
                               int32_t* target_len, int32_t* mtp_len,
                               void* stream);
/* Batched-verify linear layer on the matrix cores (M up to 128 rows: C4/C5
 * batches and batched prompt chunks), the same contract and epilogues as
 * hai_gemm_bf16 but computed with v_mfma_f32_16x16x32_bf16: equal to the
 * canonical result within fp32 accumulation error (~1e-6 relative before
 * the bf16 output rounding), not bit for bit.  Replaces rocblas_gemm_ex
 * (hip_backend.cc:697-809) for batched rows.  x and w 16-byte aligned,
 * K % 8 == 0, M <= 128.
 * workspace (may be NULL) lets narrow layers split K across blocks; with
 * hai_gemm_mfma_workspace_bytes(M, N) bytes every split is available, with
 * less the call uses fewer splits.  The result does not depend on it. */
size_t hai_gemm_mfma_workspace_bytes(int64_t M, int64_t N);
/* The FP8 block-scaled Linear (arguments as hai_gemm_fp8_bf16, K % 16 == 0)
 * on the matrix cores for M up to 128: codes decoded exactly to bf16, each
 * 128-k scale block summed on its own and scaled in fp32.  Tolerance mode as
 * hai_gemm_bf16_mfma; workspace as there. */
int hai_gemm_fp8_mfma(void* y, int64_t ldy, const void* x, int64_t ldx,
                      const void* wq, const float* scales,
                      const int32_t* scale_rows, int64_t M, int64_t N,
                      int64_t K, int epilogue, const void* res, int64_t ld_res,
                      void* workspace, size_t workspace_bytes, void* stream);
int hai_gemm_bf16_mfma(void* y, int64_t ldy, const void* x, int64_t ldx,
                       const void* w, int64_t M, int64_t N, int64_t K,
                       int epilogue, const void* res, int64_t ld_res,
                       void* workspace, size_t workspace_bytes, void* stream);
/* Prompt-sized linear layers (prefill chunks: hundreds to thousands of rows)
 * on the matrix cores, compute bound: 128 x 128 (or 128 x 64) output tiles
 * with both operands staged in LDS.  Same contract, epilogues and tolerance
 * as hai_gemm_bf16_mfma / hai_gemm_fp8_mfma (FP8: codes decoded exactly,
 * each 128-k scale block scaled in fp32), any M; K % 64 == 0, ldx % 8 == 0,
 * x and w 16-byte aligned, M * ldx * 2 and N * K * elem below 4 GiB.  The
 * reference runs prefill GEMMs through rocblas_gemm_ex
 * (hip_backend.cc:697-809). */
int hai_gemm_bf16_tiled(void* y, int64_t ldy, const void* x, int64_t ldx,
                        const void* w, int64_t M, int64_t N, int64_t K,
                        int epilogue, const void* res, int64_t ld_res,
                        void* stream);
int hai_gemm_fp8_tiled(void* y, int64_t ldy, const void* x, int64_t ldx,
                       const void* wq, const float* scales,
                       const int32_t* scale_rows, int64_t M, int64_t N,
                       int64_t K, int epilogue, const void* res, int64_t ld_res,
                       void* stream);
/* Epilogue flag for the MFMA GEMMs with HAI_EPI_RESIDUAL: when the call
 * splits K (hai_gemm_mfma_splits > 1) it leaves the fp32 partials
 * [splits][M][N] at the start of the workspace instead of finishing y; the
 * caller completes y = res (in place) with hai_mfma_residual_rmsnorm_bf16.
 * With one split the call finishes y itself. */
enum { HAI_MFMA_KEEP_PARTIALS = 0x200 };
/* The number of K splits the MFMA GEMM takes for this shape and workspace. */
int hai_gemm_mfma_splits(int64_t M, int64_t N, int64_t K, const void* workspace,
                         size_t workspace_bytes);
/* Completes a residual MFMA GEMM called with HAI_MFMA_KEEP_PARTIALS, fused
 * with the RMSNorm(+1 when unit_offset) that follows it in the decoder
 * (qwen_reference.cc:108-144): h[M, N] (the residual, ld h) becomes
 * bf16(h + bf16(sum of the partials in split order)), bit-identical to the
 * unfused call, and xn = hai_rmsnorm_bf16(h) bit for bit; norm_w null skips
 * the norm.  N % 8 == 0, N <= 8192, M <= 128; splits is the count the GEMM
 * took (hai_gemm_mfma_splits), 2 <= splits <= 4 (with one split the GEMM
 * finished h itself and left no partials), and the workspace must hold
 * splits * M * N floats (workspace_bytes). */
int hai_mfma_residual_rmsnorm_bf16(void* h, int64_t ldh, const void* workspace,
                                   size_t workspace_bytes, int64_t M, int64_t N,
                                   int64_t splits, const void* norm_w, float eps,
                                   int unit_offset, void* xn, int64_t ld_xn,
                                   void* stream);

/* ------------------------------------------------------------------ synthetic data / checks
 * Synthetic weights: element (r, c) of a [rows, cols] tensor (row stride
 * ld) gets bf16(std * IrwinHall4(splitmix64(key(seed, tensor_id) + r*cols+c))),
 * the generator the CPU oracle uses. */
int hai_fill_synthetic_bf16(void* dst, int64_t rows, int64_t cols, int64_t ld,
                            uint64_t seed, uint32_t tensor_id, float std_dev,
                            void* stream);
/* The host-side operand check the launchers run when the environment sets
 * HAI_CHECK_BOUNDS=1, applied here unconditionally and without launching
 * anything: HAI_OK when [p, p + bytes) lies inside one device allocation,
 * HAI_ERR_INVALID_ARGUMENT otherwise. */
int hai_debug_check_extent(const void* p, size_t bytes);
/* Evaluates one canonical primitive elementwise (0 exp, 1 log1p, 2 sigmoid,
 * 3 silu, 4 sqrt, 5 1/x, 6 bf16 round) so tests can pin device bits. */
int hai_debug_math_f32(float* y, const float* x, int64_t n, int fn, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HAI_KERNELS_H */
