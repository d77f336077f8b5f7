// engine.h -- MI355X verify engine: a synthetic Qwen3.5-style hybrid model
// resident in HBM plus the speculative MTP decode loop of the reference's
// Generator::generate (src/generator.cc:545-1117).
//
// Host code only: every device action goes through the hai_* C ABI
// (include/hai_kernels.h).  The engine holds B sequences (B = max_batch) that
// run the speculative rounds in lockstep; every per-sequence quantity (cache
// rows, lengths, round state) is indexed by the sequence, and a verify row
// is row b*T + t of the batch.  Layout in HBM:
//   * weights: one arena, each Linear stored [N, K] row-major as in the
//     checkpoint, with the projections of a layer concatenated so that one
//     weight-streaming launch covers them: DeltaNet in_proj = [qkv | z | a | b]
//     rows, attention = [q(+gate) | k | v] rows, MLP gate/up interleaved row by
//     row (gate_f, up_f) for the fused SwiGLU epilogue;
//   * caches: KV [B][cap][nkv][D] per attention layer; DeltaNet conv inputs
//     in a ring [B][ring][C] indexed by position and the fp32 state in slots
//     [nslots][B][nv][dk*dv] (each head column-tiled, as
//     hai_deltanet_verify_bf16 documents), the slot of sequence length L
//     being L % nslots;
//     committed lengths live on the device and are advanced by the accept
//     kernel, so rollback is a length update, never a copy.
#pragma once

#include <cstdlib>

#include <chrono>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "hai_engine.h"

namespace hybridai::mi355x {

// A Linear stored as FP8 E4M3 codes [N, K] with 128x128 fp32 block scales:
// s holds the block grids of the checkpoint tensors concatenated into the
// matrix (each ceil(rows/128) x ceil(K/128)), map[n] the scale row of stored
// row n (hai_gemm_fp8_bf16's scale_rows).
struct Fp8Linear {
    uint8_t* q = nullptr;
    float* s = nullptr;
    int32_t* map = nullptr;
};

// The weight operand of one linear layer: bf16 rows (w) or FP8 (q, s, map).
struct Lin {
    const uint16_t* w = nullptr;
    const uint8_t* q = nullptr;
    const float* s = nullptr;
    const int32_t* map = nullptr;
    Lin() = default;
    Lin(const uint16_t* bf16) : w(bf16) {}  // NOLINT: bf16 pointers convert implicitly
    explicit Lin(const Fp8Linear& f) : q(f.q), s(f.s), map(f.map) {}
    // rows [r0, ...) of a [N, K] matrix
    Lin rows(int64_t r0, int64_t K) const {
        Lin o = *this;
        if (w) o.w = w + r0 * K;
        if (q) {
            o.q = q + r0 * K;
            o.map = map + r0;
        }
        return o;
    }
};

struct LayerWeights {
    bool attn = false;
    uint16_t* in_ln = nullptr;
    uint16_t* post_ln = nullptr;
    // Gated DeltaNet
    uint16_t* w_in = nullptr;     // [C + nv*dv + 2*nv, H]
    uint16_t* conv_w = nullptr;   // [C, Kc]
    uint16_t* a_log = nullptr;    // [nv]
    uint16_t* dt_bias = nullptr;  // [nv]
    uint16_t* lin_norm = nullptr; // [dv]
    uint16_t* w_out = nullptr;    // [H, nv*dv]
    // gated GQA
    uint16_t* w_qkv = nullptr;    // [nq*2D + 2*nkv*D, H]
    uint16_t* q_norm = nullptr;   // [D]
    uint16_t* k_norm = nullptr;   // [D]
    uint16_t* w_o = nullptr;      // [H, nq*D]
    // SwiGLU MLP
    uint16_t* w_gu = nullptr;     // [2F, H], rows interleaved gate/up
    uint16_t* w_down = nullptr;   // [H, F]
    // FP8 weight format: the same matrices as E4M3 (in_proj without a|b),
    // in_proj_a | in_proj_b kept bf16 as the reference loads them
    Fp8Linear f_in;               // [C + nv*dv, H]
    uint16_t* w_ab = nullptr;     // [2*nv, H]
    Fp8Linear f_out, f_qkv, f_o, f_gu, f_down;
    // caches
    uint16_t* k_cache = nullptr;  // [B][cap][nkv][D]
    uint16_t* v_cache = nullptr;
    uint16_t* ring = nullptr;     // [B][ring][C]
    float* state = nullptr;       // [nslots][B][nv][dk*dv], column-tiled heads
    float* rec = nullptr;         // [nslots][B][nv][dk + dv + 4] rollback records of verify tokens
};

// Tensor ids shared with the synthetic generator, the CPU oracle and the
// checkpoint names: slot * 64 + kind (slot 0 shared, 1 MTP shared, 2 + i
// decoder layer i, 1024 the MTP decoder layer).
enum Kind : uint32_t {
    kInputLN = 0, kPostLN = 1, kInQKV = 2, kInZ = 3, kInA = 4, kInB = 5, kConv = 6, kALog = 7,
    kDtBias = 8, kLinNorm = 9, kOutProj = 10, kQProj = 11, kKProj = 12, kVProj = 13, kOProj = 14,
    kQNorm = 15, kKNorm = 16, kGate = 17, kUp = 18, kDown = 19,
};
constexpr uint32_t tid(uint32_t slot, uint32_t kind) { return slot * 64u + kind; }
constexpr uint32_t kSlotShared = 0, kSlotMtpShared = 1, kSlotLayer0 = 2, kSlotMtpLayer0 = 1024;

class SafeTensors;

struct TensorEntry {
    uint32_t id;
    uint16_t* ptr;
    int64_t rows, cols, ld;
};

// One checkpoint tensor held as FP8: where its codes and scale grid live.
struct QuantEntry {
    uint32_t id;
    uint8_t* q;
    int64_t ldq;
    float* s;
    int64_t rows, cols;
};

struct Dims {
    int64_t H, F, V, nq, nkv, D, R, nk, nv, dk, dv, Kc, C, Nin, Nqkv, qw, kvw, vw;
};

// Tokens per DeltaNet kernel launch, and the largest verify (width 16 + 1,
// the reference's widest proposal, generator.cc:124-137).
constexpr int64_t kDeltaNetMaxT = 16;
constexpr int64_t kMaxVerifyRows = 17;

class Engine {
public:
    Engine(const hai_model_config& cfg, const hai_engine_options& opt);
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    bool ok() const { return ok_; }
    const std::string& error() const { return error_; }
    int set_error(int rc, const std::string& what) { return fail(rc, what); }

    int init_synthetic(uint64_t seed, float std_dev);
    // Every weight from a Qwen checkpoint (models/qwen3_weights.cc:196-380):
    // each engine tensor read under its checkpoint name, shape and dtype
    // checked (BF16, or F32 whose values are all bf16 numbers; FP8 E4M3 codes
    // with their weight_scale_inv grid when the engine stores FP8), and
    // copied into the engine's stacked / interleaved layout.
    // include_mtp = false leaves the MTP weights unloaded (a checkpoint
    // without them decodes greedily only).
    int load_checkpoint(const SafeTensors& st, bool include_mtp = true);
    int64_t read_tensor(uint32_t id, uint16_t* out, int64_t capacity);
    uint64_t weight_bytes() const { return weight_bytes_; }
    const Dims& dims() const { return d_; }
    int64_t batch() const { return B_; }
    bool fp8_weights() const { return fp8_; }
    const hai_model_config& config() const { return cfg_; }

    // Per-sequence arrays below are [B][...]: prompts [B][P], ids [B][T],
    // hidden [B][T][H], logits [B][T][V], out [B][max_new or cap], n_out [B],
    // stats [B], round_log [B][round_log_cap][HAI_ROUND_RECORD],
    // override_tokens [B][n_override].
    int forward_rows(const int32_t* ids, int64_t T, uint16_t* hidden, uint16_t* logits);
    int generate_greedy(const int32_t* prompt, int64_t P, int64_t max_new, const int32_t* eos,
                        int64_t n_eos, int32_t* out, int64_t* n_out);
    int generate_speculative(const int32_t* prompts, int64_t P, int64_t max_new, int64_t width,
                             const int32_t* eos, int64_t n_eos, const int32_t* override_tokens,
                             int64_t n_override, int32_t* out, hai_spec_stats* stats,
                             int32_t* round_log, int64_t round_log_cap, int64_t* n_out);

    // benchmark split of generate_speculative; spec_rounds sums the stats of
    // all sequences
    int prefill(const int32_t* prompts, int64_t P, int64_t max_new);
    // draft overrides for spec_rounds, uploaded once: tokens [B][n] replace
    // the MTP proposal for output position pos < n of each sequence (the
    // device copies them into the verify ids, no host round trip); n = 0 or
    // null tokens clears them
    int set_draft_override(const int32_t* tokens, int64_t n);
    int set_prefill_rows(int64_t rows);
    bool fast_prefill_buffers() const { return dn_ws_ != nullptr; }
    int spec_rounds(int64_t rounds, int64_t width, int32_t* out, int64_t cap, int64_t* n_out,
                    hai_spec_stats* stats);
    int profile_verify(int64_t T, int64_t iters, hai_verify_profile* out);

private:
    struct RoundState {
        int64_t max_new = 0;
        int64_t emitted = 0;
        int64_t next_target = 0;
        int64_t target_len = 0;  // host mirror of the device committed length
        int64_t mtp_len = 0;
        bool done = false;
    };
    // Inputs of one lockstep round that vary per sequence.
    struct RoundIo {
        const int32_t* eos = nullptr;              // host copy (round-start and correction checks)
        int64_t n_eos = 0;                         // > 0: the draft chains end on the device (d_eos_)
        const int64_t* ov = nullptr;               // device [B][n_ov] draft overrides, or null
        int64_t n_ov = 0;
        int32_t* out = nullptr;                    // [B][out_ld]
        int64_t out_ld = 0;
        hai_spec_stats* stats = nullptr;           // [B]
        int32_t* round_log = nullptr;              // [B][log_cap][HAI_ROUND_RECORD]
        int64_t log_cap = 0;
        int64_t* n_log = nullptr;                  // [B] records written
    };

    int fail(int rc, const std::string& what);       // the engine's own message
    int lib_fail(int rc, const std::string& what);   // what + the kernel library's last error
    int propagate(int rc, const char* what, uint64_t seq_before);
    // every id in [0, vocab): token ids index the embedding table
    int check_ids(const int32_t* ids, int64_t n, const char* what);
    int alloc_all();
    int reset_state();
    int upload_rope_tables();

    // device pieces of a step
    // M rows of any count: launches of <= 16 rows on the bit-exact kernels,
    // or one MFMA launch per <= 128 rows when the engine runs in tolerance
    // mode (hai_engine_options::mfma) and M >= kMfmaMinRows.
    static constexpr int64_t kMfmaMinRows = 4;
    // above this many rows a matrix-core GEMM tiles both operands
    // (hai_gemm_*_tiled) instead of streaming the weights once per 128 rows
    static constexpr int64_t kTiledMinRows = 128;
    bool use_mfma(int64_t M) const { return (mfma_ || fast_) && M >= kMfmaMinRows; }
    // which rows of a forward get lm_head logits
    enum class Logits { kAll, kLast, kNone };
    // A residual MFMA GEMM whose K-split partials wait in the workspace: the
    // RMSNorm of the same rows completes them (hai_mfma_residual_rmsnorm_bf16)
    // in one launch; anything else completes them first (flush_pending).
    struct PendingResidual {
        uint16_t* h = nullptr;
        int64_t ld = 0, M = 0, N = 0;
        int splits = 0;
    };
    PendingResidual pending_;
    int flush_pending();
    int gemm(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const Lin& w, int64_t M, int64_t N,
             int64_t K, int epi, const uint16_t* res, int64_t ldres);
    // RMSNorm(+1) of the H-wide rows x (norm weight nw) fused into the linear
    // layer W [N, H]; xn_out (optional) receives the normalised rows.
    int norm_gemm(uint16_t* y, int64_t ldy, const uint16_t* x, const uint16_t* nw, uint16_t* xn_out,
                  const Lin& w, int64_t M, int64_t N, int epi, const uint16_t* res, int64_t ldres);
    Lin lin(const uint16_t* w, const Fp8Linear& f) const { return fp8_ ? Lin(f) : Lin(w); }
    // DeltaNet state writes of a forward: the final state only (prompt rows,
    // greedy steps), rollback records of a verify (final state + one record
    // per token, start positions in d_vbase_), or a correction that first
    // re-applies the kept records of the verify's accepted prefix
    enum class StateWrites { kFinal, kRecord, kReplay };
    int forward_target(const int64_t* d_ids, int64_t T, StateWrites sw, Logits logits = Logits::kAll);
    int deltanet(const LayerWeights& L, int64_t T, StateWrites sw, int64_t off_a, int64_t off_b, const uint16_t* xn,
                 const uint16_t* w_ab);
    int attention_layer(const LayerWeights& L, int64_t T, uint16_t* h, const int32_t* lens,
                        uint16_t* kc, uint16_t* vc);
    int mlp(const LayerWeights& L, int64_t T, uint16_t* h);
    int mtp_kv_rows(const int64_t* d_ids, const uint16_t* d_hidden, int64_t T, bool add_len);
    int mtp_draft_step(const int64_t* d_id, const uint16_t* d_hin, uint16_t* d_mh, int64_t* d_cand);
    int prefill_chunks(const int32_t* ids, int64_t P, uint16_t* hidden_out, uint16_t* logits_out);
    // One lockstep round of every live sequence; returns false in *any_live
    // when every sequence has finished.
    int one_round(int64_t width, const RoundIo& io, bool* any_live);
    int sync();
    int read_i64(const int64_t* d, int64_t* h, int64_t n);
    int64_t* read_ids() const {  // the int64 part of h_read_, after the [4B] results
        return reinterpret_cast<int64_t*>(static_cast<char*>(h_read_) + 16 * B_);
    }
    // ids (int32, host) widened into an engine-owned device table that grows on demand
    int upload_ids(int64_t** table, int64_t* cap, const int32_t* ids, int64_t n);
    // Replays the captured graph in *slot (capturing `enqueue` on first use)
    // when graphs are enabled; otherwise launches `enqueue` directly.
    template <typename F>
    int replay(void** slot, F&& enqueue);
    int draft_step_at(int64_t i, int64_t T);
    int verify_step(int64_t T);
    int correction_step();

    hai_model_config cfg_{};
    hai_engine_options opt_{};
    Dims d_{};
    bool ok_ = false;
    std::string error_;
    uint64_t err_seq_ = 0;  // bumped by every failure report

    void* stream_ = nullptr;
    void* weights_ = nullptr;
    void* caches_ = nullptr;
    void* work_ = nullptr;
    uint64_t weight_bytes_ = 0;

    int64_t B_ = 1;       // sequences
    int64_t cap_ = 0;     // KV capacity per sequence
    int64_t tmax_ = 0;    // largest verify T (rows per sequence)
    int64_t pchunk_ = 0;  // prompt rows per sequence and prefill forward
    bool fast_prefill_ = false;  // prompts prefill in large chunks on the matrix cores
    int64_t pchunk_cap_ = 0;     // the largest prompt chunk the buffers hold
    bool fast_ = false;          // inside such a chunk: matrix-core GEMMs and attention
    char* dn_ws_ = nullptr;      // prefill DeltaNet outputs before the gated norm
    int64_t dn_ws_bytes_ = 0;
    bool mfma_ = false;   // tolerance mode: MFMA GEMMs (4+ rows) and attention
    int64_t ring_ = 0;
    int64_t nslots_ = 0;

    std::vector<LayerWeights> layers_;
    LayerWeights mtp_;
    uint16_t* embed_ = nullptr;
    uint16_t* final_norm_ = nullptr;
    uint16_t* lm_head_ = nullptr;
    uint16_t* fc_ = nullptr;
    uint16_t* mtp_norm_ = nullptr;
    uint16_t* pre_emb_ = nullptr;
    uint16_t* pre_hid_ = nullptr;
    std::vector<TensorEntry> tensors_;
    bool fp8_ = false;  // quantizable Linears stored FP8 (hai_engine_options::weight_format)
    std::vector<QuantEntry> quant_;
    std::vector<std::pair<int32_t*, std::vector<int32_t>>> maps_;  // scale maps uploaded at init

    // workspace (rows = B * tmax)
    int64_t* d_ids_ = nullptr;    // [rows] prefill / forward ids
    int64_t* d_vids_ = nullptr;   // [B][T] per sequence: next_target, candidates
    int64_t* d_next_ = nullptr;   // [B] next target after the round (accept / correction)
    int64_t* d_dids_ = nullptr;   // [B] draft inputs
    int64_t* d_cand_ = nullptr;   // [B] draft outputs / correction argmax
    int64_t* d_preds_ = nullptr;  // [rows]
    int32_t* d_result_ = nullptr; // [B][4]
    int32_t* d_tlen_ = nullptr;   // [B] committed target lengths
    int32_t* d_vbase_ = nullptr;  // [B] target lengths at the last verify (DeltaNet replay base)
    int32_t* d_mlen_ = nullptr;   // [B] MTP cache lengths
    int32_t* d_ndraft_ = nullptr; // [B] drafts counted per sequence this round
    int32_t* d_delta_ = nullptr;  // [B] MTP length corrections
    int32_t* d_plen_ = nullptr;   // [3B + 4B] profiling scratch lengths/results
    int64_t* d_pnext_ = nullptr;  // [B] profiling scratch tokens
    int64_t* d_override_ = nullptr;  // [B][n_override_] draft overrides of spec_rounds (own allocation)
    int64_t n_override_ = 0;
    int64_t* d_gen_ov_ = nullptr;    // [B][n] draft overrides of one generate_speculative call (own allocation)
    int64_t gen_ov_cap_ = 0;         // int64 entries of d_gen_ov_
    int64_t* d_eos_ = nullptr;       // end-of-sequence ids of the running generate call (own allocation)
    int64_t eos_cap_ = 0;
    int32_t* d_pcap_ = nullptr;      // [B] proposal caps of the round (device chain counting)
    int32_t* h_stage_ = nullptr;     // pinned [3B]: caps, draft counts, MTP length corrections of a round
    void* h_read_ = nullptr;         // pinned read-back of a round: [4B] results | [B·tmax] predictions | [B·tmax] ids | [B] ids
    int64_t syncs_ = 0;              // host synchronisations with the stream so far
    uint16_t* h_ = nullptr;       // [rows, H] residual stream
    uint16_t* xn_ = nullptr;      // [rows, 2H]
    uint16_t* emb_ = nullptr;     // [rows, H]
    uint16_t* proj_ = nullptr;    // [rows, max(Nin, Nqkv)]
    uint16_t* q_ = nullptr;       // [rows, nq*D]
    uint16_t* gate_ = nullptr;
    uint16_t* att_ = nullptr;
    uint16_t* dnout_ = nullptr;   // [rows, nv*dv]
    uint16_t* act_ = nullptr;     // [rows, F]
    uint16_t* hf_ = nullptr;      // [rows, H] post-final-norm hidden
    uint16_t* logits_ = nullptr;  // [rows, V]
    uint16_t* mh_[2] = {nullptr, nullptr};  // [B, H] MTP outputs (chained drafts)
    uint16_t* h_prev_ = nullptr;  // [B, H] target hidden feeding the next draft
    uint16_t* rec_hidden_ = nullptr;  // [B, H]
    void* gqa_scratch_ = nullptr;
    void* mfma_ws_ = nullptr;     // K-split partials of the MFMA GEMMs
    size_t mfma_ws_bytes_ = 0;
    void* argmax_scratch_ = nullptr;
    float* rope_cos_ = nullptr;
    float* rope_sin_ = nullptr;
    int64_t nproj_ = 0;

    // profiling of GEMM launches (profile_verify only)
    // profile_verify: the GEMM launches of one verify step, recorded so that
    // they can be replayed back to back between two events.
    struct GemmCall {
        uint16_t* y;
        int64_t ldy;
        const uint16_t* x;
        int64_t ldx;
        Lin w;
        int64_t M, N, K;
        int epi;
        const uint16_t* res;
        int64_t ldres;
        const uint16_t* nw;  // non-null: RMSNorm-fused launch
        uint16_t* xn;
    };
    bool prof_record_ = false;
    std::vector<GemmCall> prof_calls_;

    std::vector<RoundState> rs_;          // [B]
    std::vector<int32_t> ndraft_host_;    // last uploaded d_ndraft_ contents

    bool use_graphs_ = false;
    std::vector<void*> draft_graphs_;   // by (verify width T, draft index)
    std::vector<void*> verify_graphs_;  // by verify width T
    void* corr_graph_ = nullptr;
};

}  // namespace hybridai::mi355x
