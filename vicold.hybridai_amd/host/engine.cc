// engine.cc -- MI355X verify engine (see engine.h).
#include "engine.h"

#include "checkpoint.h"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "hai_kernels.h"

namespace hybridai::mi355x {

namespace {

constexpr size_t kAlign = 256;
// Widest linear layer that takes its input RMSNorm fused into the GEMM.
constexpr int64_t kFusedNormMaxN = 65536;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Bump allocator over one device arena: first pass sizes, second pass hands
// out pointers.
class Carver {
public:
    explicit Carver(char* base) : base_(base) {}
    template <typename T>
    T* take(size_t count) {
        const size_t off = used_;
        used_ += align_up(count * sizeof(T));
        return base_ ? reinterpret_cast<T*>(base_ + off) : nullptr;
    }
    size_t used() const { return used_; }

private:
    char* base_;
    size_t used_ = 0;
};

bool in_set(const int32_t* s, int64_t n, int64_t v) {
    for (int64_t i = 0; i < n; ++i)
        if (s[i] == v) return true;
    return false;
}

using Clock = std::chrono::steady_clock;
double seconds_since(Clock::time_point t) {
    return std::chrono::duration<double>(Clock::now() - t).count();
}

}  // namespace

// A failing call is reported with its expression, followed by the engine's
// own message when the callee set one (an argument check) and otherwise by
// the kernel library's last error.
#define HAI_TRY(expr)                                                 \
    do {                                                              \
        const uint64_t _seq = err_seq_;                               \
        const int _rc = (expr);                                       \
        if (_rc != HAI_OK) return propagate(_rc, #expr, _seq);        \
    } while (0)

Engine::Engine(const hai_model_config& cfg, const hai_engine_options& opt) : cfg_(cfg), opt_(opt) {
    d_.H = cfg.hidden;
    d_.F = cfg.ffn;
    d_.V = cfg.vocab;
    d_.nq = cfg.num_q_heads;
    d_.nkv = cfg.num_kv_heads;
    d_.D = cfg.head_dim;
    d_.R = cfg.rope_dim;
    d_.nk = cfg.lin_qk_heads;
    d_.nv = cfg.lin_v_heads;
    d_.dk = cfg.lin_k_dim;
    d_.dv = cfg.lin_v_dim;
    d_.Kc = cfg.conv_kernel;
    d_.C = 2 * d_.nk * d_.dk + d_.nv * d_.dv;
    d_.vw = d_.nv * d_.dv;
    d_.Nin = d_.C + d_.vw + 2 * d_.nv;
    d_.qw = d_.nq * d_.D;
    d_.kvw = d_.nkv * d_.D;
    d_.Nqkv = 2 * d_.qw + 2 * d_.kvw;
    B_ = std::max<int64_t>(1, opt.max_batch);
    // verify rows per sequence: up to 17 (width 16, the reference's largest,
    // generator.cc:124-137) for one sequence; batches keep 16 (one DeltaNet
    // launch per forward)
    tmax_ = std::max<int64_t>(2, std::min<int64_t>(B_ == 1 ? kMaxVerifyRows : kDeltaNetMaxT, opt.max_verify_tokens));
    pchunk_ = std::min<int64_t>(tmax_, kDeltaNetMaxT);
    if (opt.prefill_rows > tmax_) {
        pchunk_ = opt.prefill_rows;
        fast_prefill_ = true;
    }
    pchunk_cap_ = pchunk_;
    cap_ = std::max<int64_t>(opt.max_context, tmax_ + 1);
    ring_ = 32;
    nslots_ = tmax_ + 1;
    use_graphs_ = opt.use_graphs != 0;
    fp8_ = opt.weight_format == HAI_WEIGHTS_FP8_BLOCK128;
    mfma_ = opt.mfma != 0;
    draft_graphs_.assign(static_cast<size_t>((tmax_ + 1) * tmax_), nullptr);
    verify_graphs_.assign(static_cast<size_t>(tmax_ + 1), nullptr);
    rs_.assign(static_cast<size_t>(B_), RoundState{});
    if (cfg.hidden <= 0 || cfg.hidden % 8 != 0 || cfg.num_layers <= 0 || cfg.full_attention_interval <= 0 ||
        cfg.num_kv_heads <= 0 || cfg.num_q_heads % cfg.num_kv_heads != 0 || cfg.lin_qk_heads <= 0 ||
        cfg.lin_v_heads % cfg.lin_qk_heads != 0 || cfg.ffn % 8 != 0 || cfg.mtp_layers != 1 ||
        cfg.rope_dim > cfg.head_dim || cfg.rope_dim % 2 != 0 || cfg.conv_kernel < 2 || cfg.conv_kernel > 8 ||
        d_.vw % 8 != 0 || d_.qw % 8 != 0) {
        error_ = "unsupported model configuration";
        return;
    }
    if (opt.weight_format != HAI_WEIGHTS_BF16 && opt.weight_format != HAI_WEIGHTS_FP8_BLOCK128) {
        error_ = "unknown weight_format";
        return;
    }
    if (B_ > 64) {
        error_ = "max_batch above 64";
        return;
    }
    if (opt.prefill_rows < 0 || opt.prefill_rows > 8192 || B_ * pchunk_ > 65536) {
        error_ = "prefill_rows outside 0..8192 (or more than 65536 rows per chunk over the batch)";
        return;
    }
    if (hai_set_device(opt.device) != HAI_OK || hai_stream_create(&stream_) != HAI_OK) {
        error_ = std::string("device setup failed: ") + hai_last_error();
        return;
    }
    if (alloc_all() != HAI_OK) return;
    if (upload_rope_tables() != HAI_OK) return;
    ok_ = true;
}

Engine::~Engine() {
    if (stream_) hai_stream_synchronize(stream_);
    for (void* g : draft_graphs_) if (g) hai_graph_destroy(g);
    for (void* g : verify_graphs_) if (g) hai_graph_destroy(g);
    if (corr_graph_) hai_graph_destroy(corr_graph_);
    if (weights_) hai_free(weights_);
    if (caches_) hai_free(caches_);
    if (work_) hai_free(work_);
    if (d_override_) hai_free(d_override_);
    if (d_gen_ov_) hai_free(d_gen_ov_);
    if (d_eos_) hai_free(d_eos_);
    if (h_stage_) hai_host_free(h_stage_);
    if (h_read_) hai_host_free(h_read_);
    if (stream_) hai_stream_destroy(stream_);
}

int Engine::fail(int rc, const std::string& what) {
    error_ = what;
    ++err_seq_;
    return rc;
}

int Engine::lib_fail(int rc, const std::string& what) {
    error_ = what + ": " + hai_last_error();
    ++err_seq_;
    return rc;
}

int Engine::propagate(int rc, const char* what, uint64_t seq_before) {
    error_ = std::string(what) + ": " + (err_seq_ != seq_before ? error_ : std::string(hai_last_error()));
    ++err_seq_;
    return rc;
}

int Engine::alloc_all() {
    const auto& d = d_;
    const int64_t H = d.H;
    layers_.assign(static_cast<size_t>(cfg_.num_layers), LayerWeights{});
    for (int64_t i = 0; i < cfg_.num_layers; ++i)
        layers_[i].attn = (i + 1) % cfg_.full_attention_interval == 0;
    mtp_.attn = true;

    // ---- weights ----
    auto carve_weights = [&](Carver& cv) {
        tensors_.clear();
        quant_.clear();
        maps_.clear();
        auto add = [&](uint16_t*& dst, uint32_t id, int64_t rows, int64_t cols) {
            dst = cv.take<uint16_t>(static_cast<size_t>(rows * cols));
            tensors_.push_back({id, dst, rows, cols, cols});
        };
        // FP8 matrix [sum rows, K] made of checkpoint tensors stacked
        // (interleave: row r of part i is stored row r * nparts + i).
        struct Part {
            uint32_t id;
            int64_t rows;
        };
        auto fp8mat = [&](Fp8Linear& f, int64_t K, std::vector<Part> parts, bool interleave) {
            const int64_t nkb = (K + 127) / 128;
            const int64_t np = static_cast<int64_t>(parts.size());
            int64_t total = 0, grid = 0;
            for (const auto& p : parts) {
                total += p.rows;
                grid += (p.rows + 127) / 128;
            }
            f.q = cv.take<uint8_t>(static_cast<size_t>(total * K));
            f.s = cv.take<float>(static_cast<size_t>(grid * nkb));
            f.map = cv.take<int32_t>(static_cast<size_t>(total));
            if (f.q == nullptr) return;  // sizing pass
            std::vector<int32_t> map(static_cast<size_t>(total));
            int64_t row0 = 0, g0 = 0;
            for (int64_t i = 0; i < np; ++i) {
                const Part& p = parts[static_cast<size_t>(i)];
                for (int64_t r = 0; r < p.rows; ++r)
                    map[static_cast<size_t>(interleave ? r * np + i : row0 + r)] = static_cast<int32_t>(g0 + r / 128);
                quant_.push_back({p.id, interleave ? f.q + i * K : f.q + row0 * K, interleave ? np * K : K,
                                  f.s + g0 * nkb, p.rows, K});
                row0 += p.rows;
                g0 += (p.rows + 127) / 128;
            }
            maps_.emplace_back(f.map, std::move(map));
        };
        auto layer = [&](LayerWeights& L, uint32_t slot) {
            add(L.in_ln, tid(slot, kInputLN), 1, H);
            add(L.post_ln, tid(slot, kPostLN), 1, H);
            if (L.attn) {
                if (fp8_) {
                    fp8mat(L.f_qkv, H, {{tid(slot, kQProj), 2 * d.qw}, {tid(slot, kKProj), d.kvw},
                                        {tid(slot, kVProj), d.kvw}}, false);
                } else {
                    L.w_qkv = cv.take<uint16_t>(static_cast<size_t>(d.Nqkv * H));
                    tensors_.push_back({tid(slot, kQProj), L.w_qkv, 2 * d.qw, H, H});
                    tensors_.push_back(
                        {tid(slot, kKProj), L.w_qkv ? L.w_qkv + 2 * d.qw * H : nullptr, d.kvw, H, H});
                    tensors_.push_back({tid(slot, kVProj), L.w_qkv ? L.w_qkv + (2 * d.qw + d.kvw) * H : nullptr,
                                        d.kvw, H, H});
                }
                add(L.q_norm, tid(slot, kQNorm), 1, d.D);
                add(L.k_norm, tid(slot, kKNorm), 1, d.D);
                if (fp8_) fp8mat(L.f_o, d.qw, {{tid(slot, kOProj), H}}, false);
                else add(L.w_o, tid(slot, kOProj), H, d.qw);
            } else {
                if (fp8_) {
                    fp8mat(L.f_in, H, {{tid(slot, kInQKV), d.C}, {tid(slot, kInZ), d.vw}}, false);
                    L.w_ab = cv.take<uint16_t>(static_cast<size_t>(2 * d.nv * H));
                    tensors_.push_back({tid(slot, kInA), L.w_ab, d.nv, H, H});
                    tensors_.push_back({tid(slot, kInB), L.w_ab ? L.w_ab + d.nv * H : nullptr, d.nv, H, H});
                } else {
                    L.w_in = cv.take<uint16_t>(static_cast<size_t>(d.Nin * H));
                    uint16_t* b = L.w_in;
                    auto at = [&](int64_t row) { return b ? b + row * H : nullptr; };
                    tensors_.push_back({tid(slot, kInQKV), at(0), d.C, H, H});
                    tensors_.push_back({tid(slot, kInZ), at(d.C), d.vw, H, H});
                    tensors_.push_back({tid(slot, kInA), at(d.C + d.vw), d.nv, H, H});
                    tensors_.push_back({tid(slot, kInB), at(d.C + d.vw + d.nv), d.nv, H, H});
                }
                add(L.conv_w, tid(slot, kConv), d.C, d.Kc);
                add(L.a_log, tid(slot, kALog), 1, d.nv);
                add(L.dt_bias, tid(slot, kDtBias), 1, d.nv);
                add(L.lin_norm, tid(slot, kLinNorm), 1, d.dv);
                if (fp8_) fp8mat(L.f_out, d.vw, {{tid(slot, kOutProj), H}}, false);
                else add(L.w_out, tid(slot, kOutProj), H, d.vw);
            }
            if (fp8_) {
                fp8mat(L.f_gu, H, {{tid(slot, kGate), d.F}, {tid(slot, kUp), d.F}}, true);
                fp8mat(L.f_down, d.F, {{tid(slot, kDown), H}}, false);
            } else {
                L.w_gu = cv.take<uint16_t>(static_cast<size_t>(2 * d.F * H));
                tensors_.push_back({tid(slot, kGate), L.w_gu, d.F, H, 2 * H});
                tensors_.push_back({tid(slot, kUp), L.w_gu ? L.w_gu + H : nullptr, d.F, H, 2 * H});
                add(L.w_down, tid(slot, kDown), H, d.F);
            }
        };
        add(embed_, tid(kSlotShared, 0), d.V, H);
        add(final_norm_, tid(kSlotShared, 1), 1, H);
        add(lm_head_, tid(kSlotShared, 2), d.V, H);
        add(fc_, tid(kSlotMtpShared, 0), H, 2 * H);
        add(mtp_norm_, tid(kSlotMtpShared, 1), 1, H);
        add(pre_emb_, tid(kSlotMtpShared, 2), 1, H);
        add(pre_hid_, tid(kSlotMtpShared, 3), 1, H);
        for (size_t i = 0; i < layers_.size(); ++i) layer(layers_[i], kSlotLayer0 + static_cast<uint32_t>(i));
        layer(mtp_, kSlotMtpLayer0);
    };
    {
        Carver sizing(nullptr);
        carve_weights(sizing);
        weight_bytes_ = sizing.used();
        HAI_TRY(hai_malloc(&weights_, weight_bytes_));
        Carver real(static_cast<char*>(weights_));
        carve_weights(real);
        for (const auto& m : maps_)
            HAI_TRY(hai_memcpy_h2d(m.first, m.second.data(), m.second.size() * 4, stream_));
        HAI_TRY(sync());
        maps_.clear();
    }

    // ---- caches ----
    const size_t Bz = static_cast<size_t>(B_);
    auto carve_caches = [&](Carver& cv) {
        for (auto& L : layers_) {
            if (L.attn) {
                L.k_cache = cv.take<uint16_t>(Bz * static_cast<size_t>(cap_ * d.kvw));
                L.v_cache = cv.take<uint16_t>(Bz * static_cast<size_t>(cap_ * d.kvw));
            } else {
                L.ring = cv.take<uint16_t>(Bz * static_cast<size_t>(ring_ * d.C));
                L.state = cv.take<float>(Bz * static_cast<size_t>(nslots_ * d.nv * d.dv * d.dk));
                L.rec = cv.take<float>(hai_deltanet_records_bytes(nslots_, B_, d.nv, d.dk, d.dv) / sizeof(float));
            }
        }
        mtp_.k_cache = cv.take<uint16_t>(Bz * static_cast<size_t>(cap_ * d.kvw));
        mtp_.v_cache = cv.take<uint16_t>(Bz * static_cast<size_t>(cap_ * d.kvw));
    };
    {
        Carver sizing(nullptr);
        carve_caches(sizing);
        HAI_TRY(hai_malloc(&caches_, sizing.used()));
        Carver real(static_cast<char*>(caches_));
        carve_caches(real);
        HAI_TRY(hai_memset(caches_, 0, sizing.used(), stream_));
    }

    // ---- workspace ----
    nproj_ = std::max(d.Nin, d.Nqkv);
    const int64_t T = tmax_;
    const int64_t R = B_ * std::max(tmax_, pchunk_cap_);  // rows of one forward (verify step or prompt chunk)
    auto carve_work = [&](Carver& cv) {
        d_ids_ = cv.take<int64_t>(R);
        d_vids_ = cv.take<int64_t>(R + 1);
        d_next_ = cv.take<int64_t>(B_);
        d_dids_ = cv.take<int64_t>(B_);
        d_cand_ = cv.take<int64_t>(B_);
        d_preds_ = cv.take<int64_t>(R);
        d_result_ = cv.take<int32_t>(4 * B_);
        d_tlen_ = cv.take<int32_t>(B_);
        d_vbase_ = cv.take<int32_t>(B_);
        d_mlen_ = cv.take<int32_t>(B_);
        d_ndraft_ = cv.take<int32_t>(B_);
        d_delta_ = cv.take<int32_t>(B_);
        d_plen_ = cv.take<int32_t>(7 * B_);
        d_pnext_ = cv.take<int64_t>(B_);
        d_pcap_ = cv.take<int32_t>(B_);
        h_ = cv.take<uint16_t>(R * H);
        xn_ = cv.take<uint16_t>(R * 2 * H);
        emb_ = cv.take<uint16_t>(R * H);
        proj_ = cv.take<uint16_t>(R * nproj_);
        q_ = cv.take<uint16_t>(R * d.qw);
        gate_ = cv.take<uint16_t>(R * d.qw);
        att_ = cv.take<uint16_t>(R * d.qw);
        dnout_ = cv.take<uint16_t>(R * d.vw);
        act_ = cv.take<uint16_t>(R * d.F);
        hf_ = cv.take<uint16_t>(R * H);
        logits_ = cv.take<uint16_t>(B_ * tmax_ * d.V);  // verify rows; prompt chunks compute theirs in slices
        mh_[0] = cv.take<uint16_t>(B_ * H);
        mh_[1] = cv.take<uint16_t>(B_ * H);
        h_prev_ = cv.take<uint16_t>(B_ * H);
        rec_hidden_ = cv.take<uint16_t>(B_ * H);
        // a prompt chunk's split plan depends on its row count, and a short
        // last chunk can take more splits (and more scratch) than a full one
        size_t prefill_scratch = 0;
        if (fast_prefill_)
            for (int64_t t = 1; t <= pchunk_cap_; ++t)
                prefill_scratch =
                    std::max(prefill_scratch, hai_gqa_mfma_plan_scratch_bytes(B_, t, d.nq, d.nkv, d.D, cap_));
        gqa_scratch_ = cv.take<char>(std::max({hai_gqa_scratch_bytes(B_, T, d.nq, d.D, cap_),
                                               mfma_ ? hai_gqa_mfma_scratch_bytes(B_, T, d.nq, d.D, cap_) : size_t{0},
                                               prefill_scratch}));
        if (mfma_) {
            const int64_t mrows = std::min<int64_t>(128, R);
            size_t ws = 0;
            for (int64_t n : {d.Nqkv, d.H, d.Nin, d.C + d.vw, 2 * d.nv, 2 * d.F, 2 * d.kvw, d.V})
                ws = std::max(ws, hai_gemm_mfma_workspace_bytes(mrows, n));
            mfma_ws_bytes_ = ws;
            mfma_ws_ = ws > 0 ? cv.take<char>(ws) : nullptr;
        }
        if (fast_prefill_) {
            dn_ws_bytes_ = static_cast<int64_t>(hai_deltanet_prefill_workspace_bytes(B_, pchunk_cap_, d.nv, d.dv));
            dn_ws_ = cv.take<char>(static_cast<size_t>(dn_ws_bytes_));
        }
        argmax_scratch_ = cv.take<char>(hai_argmax_scratch_bytes(R, d.V));
        rope_cos_ = cv.take<float>(cap_ * std::max<int64_t>(1, d.R / 2));
        rope_sin_ = cv.take<float>(cap_ * std::max<int64_t>(1, d.R / 2));
    };
    {
        Carver sizing(nullptr);
        carve_work(sizing);
        HAI_TRY(hai_malloc(&work_, sizing.used()));
        Carver real(static_cast<char*>(work_));
        carve_work(real);
        HAI_TRY(hai_memset(work_, 0, sizing.used(), stream_));
    }
    // Pinned staging for the per-round uploads: a round writes each slice at
    // most once, and the previous round's copies ended with its closing sync.
    void* pin = nullptr;
    HAI_TRY(hai_host_malloc(&pin, static_cast<size_t>(3 * B_) * sizeof(int32_t)));
    h_stage_ = static_cast<int32_t*>(pin);
    // Pinned read-back: copies into pageable memory are staged and wait one
    // by one; into pinned memory they queue behind the round's kernels and
    // the round's one sync covers them all.
    HAI_TRY(hai_host_malloc(&h_read_, static_cast<size_t>(4 * B_) * 4 + static_cast<size_t>(2 * B_ * T + B_) * 8));
    return sync();
}

// cos/sin of theta = pos / base^(2p/R) in double, rounded to fp32
// (partial_rope_kernel, hip_kernels.hip:209-213).
int Engine::upload_rope_tables() {
    const int64_t half = std::max<int64_t>(1, d_.R / 2);
    std::vector<float> c(static_cast<size_t>(cap_ * half)), s(c.size());
    for (int64_t pos = 0; pos < cap_; ++pos)
        for (int64_t p = 0; p < d_.R / 2; ++p) {
            const double theta = static_cast<double>(pos) /
                std::pow(static_cast<double>(cfg_.rope_theta),
                         static_cast<double>(2 * p) / static_cast<double>(d_.R));
            c[pos * half + p] = static_cast<float>(std::cos(theta));
            s[pos * half + p] = static_cast<float>(std::sin(theta));
        }
    HAI_TRY(hai_memcpy_h2d(rope_cos_, c.data(), c.size() * 4, stream_));
    HAI_TRY(hai_memcpy_h2d(rope_sin_, s.data(), s.size() * 4, stream_));
    return sync();
}

int Engine::sync() {
    ++syncs_;
    const int rc = hai_stream_synchronize(stream_);
    if (rc != HAI_OK) return lib_fail(rc, "stream synchronize");
    return HAI_OK;
}

int Engine::read_i64(const int64_t* d, int64_t* h, int64_t n) {
    if (n > B_ || h_read_ == nullptr) {
        HAI_TRY(hai_memcpy_d2h(h, d, static_cast<size_t>(n) * 8, stream_));
        return sync();
    }
    int64_t* pin = read_ids() + 2 * B_ * tmax_;
    HAI_TRY(hai_memcpy_d2h(pin, d, static_cast<size_t>(n) * 8, stream_));
    HAI_TRY(sync());
    std::copy(pin, pin + n, h);
    return HAI_OK;
}

int Engine::upload_ids(int64_t** table, int64_t* cap, const int32_t* ids, int64_t n) {
    if (n <= 0) return HAI_OK;
    if (n > *cap || *table == nullptr) {
        HAI_TRY(sync());  // the old table may still be read by queued work
        if (*table) HAI_TRY(hai_free(*table));
        *table = nullptr;
        *cap = 0;
        void* p = nullptr;
        HAI_TRY(hai_malloc(&p, static_cast<size_t>(n) * 8));
        *table = static_cast<int64_t*>(p);
        *cap = n;
    }
    std::vector<int64_t> wide(ids, ids + n);
    HAI_TRY(hai_memcpy_h2d(*table, wide.data(), wide.size() * 8, stream_));
    return sync();  // wide lives on the host stack
}

int Engine::init_synthetic(uint64_t seed, float std_dev) {
    for (const auto& t : tensors_)
        HAI_TRY(hai_fill_synthetic_bf16(t.ptr, t.rows, t.cols, t.ld, seed, t.id, std_dev, stream_));
    if (quant_.empty()) return sync();
    // FP8 tensors: the bf16 synthetic tensor in a staging buffer, its block
    // scales, then the quantised codes into the stored layout.
    int64_t most = 0;
    for (const auto& e : quant_) most = std::max(most, e.rows * e.cols);
    void* tmp = nullptr;
    HAI_TRY(hai_malloc(&tmp, static_cast<size_t>(most) * 2));
    int rc = HAI_OK;
    for (const auto& e : quant_) {
        const int64_t nblk = ((e.rows + 127) / 128) * ((e.cols + 127) / 128);
        rc = hai_fill_synthetic_bf16(tmp, e.rows, e.cols, e.cols, seed, e.id, std_dev, stream_);
        if (rc == HAI_OK) rc = hai_fill_synthetic_scales_f32(e.s, nblk, seed, e.id, stream_);
        if (rc == HAI_OK) rc = hai_fp8_quantize_bf16(e.q, e.ldq, tmp, e.cols, e.s, e.rows, e.cols, stream_);
        if (rc != HAI_OK) break;
    }
    const int rc_sync = hai_stream_synchronize(stream_);
    hai_free(tmp);
    if (rc != HAI_OK) return lib_fail(rc, "fp8 synthetic weights");
    if (rc_sync != HAI_OK) return lib_fail(rc_sync, "stream synchronize");
    return HAI_OK;
}

int Engine::load_checkpoint(const SafeTensors& st, bool include_mtp) {
    auto is_mtp = [](uint32_t id) { return id / 64u == kSlotMtpShared || id / 64u == kSlotMtpLayer0; };
    std::string err;
    std::vector<unsigned char> host;
    auto missing = [&](const std::string& name) {
        return fail(HAI_ERR_INVALID_MODEL, "Missing Qwen weight: " + name);
    };
    // shape of a checkpoint tensor against the engine's rows x cols: 2-D
    // [rows, cols], a vector [cols] when rows == 1, the depthwise conv as
    // [C, 1, Kc] or [C, Kc]
    auto shape_ok = [](const StTensor& t, int64_t rows, int64_t cols) {
        const auto& s = t.shape;
        if (s.size() == 2) return s[0] == rows && s[1] == cols;
        if (s.size() == 1) return rows == 1 && s[0] == cols;
        if (s.size() == 3) return s[0] == rows && s[1] == 1 && s[2] == cols;
        return false;
    };
    auto shape_text = [](const StTensor& t) {
        std::string r = "[";
        for (size_t i = 0; i < t.shape.size(); ++i) r += (i ? ", " : "") + std::to_string(t.shape[i]);
        return r + "]";
    };
    // BF16 bits of a tensor (F32 accepted when every value is a bf16 number)
    auto read_bf16 = [&](const std::string& name, const StTensor& t, std::vector<uint16_t>* out) -> int {
        out->resize(static_cast<size_t>(t.numel()));
        if (t.dtype == StDType::BF16) {
            if (const int rc = st.read(t, out->data(), &err); rc != HAI_OK) return fail(rc, err);
            return HAI_OK;
        }
        if (t.dtype != StDType::F32)
            return fail(HAI_ERR_UNSUPPORTED_DTYPE,
                        "Qwen weight " + name + " is " + st_dtype_name(t.dtype) + "; the engine stores BF16");
        std::vector<float> f(static_cast<size_t>(t.numel()));
        if (const int rc = st.read(t, f.data(), &err); rc != HAI_OK) return fail(rc, err);
        for (size_t i = 0; i < f.size(); ++i)
            if (!exact_bf16(f[i], &(*out)[i]))
                return fail(HAI_ERR_UNSUPPORTED_DTYPE,
                            "Qwen weight " + name + " is F32 with values that are not bf16 numbers");
        return HAI_OK;
    };
    std::vector<uint16_t> bits;
    for (const auto& e : tensors_) {
        if (!include_mtp && is_mtp(e.id)) continue;
        const std::string name = checkpoint_name(e.id);
        const StTensor* t = st.find(name);
        if (name.empty() || t == nullptr) return missing(name.empty() ? std::to_string(e.id) : name);
        if (!shape_ok(*t, e.rows, e.cols))
            return fail(HAI_ERR_INVALID_MODEL, "Qwen weight " + name + " has shape " + shape_text(*t) + ", expected [" +
                                                   std::to_string(e.rows) + ", " + std::to_string(e.cols) + "]");
        if (const int rc = read_bf16(name, *t, &bits); rc != HAI_OK) return rc;
        HAI_TRY(hai_memcpy_h2d_2d(e.ptr, static_cast<size_t>(e.ld) * 2, bits.data(), static_cast<size_t>(e.cols) * 2,
                                  static_cast<size_t>(e.cols) * 2, static_cast<size_t>(e.rows), stream_));
        HAI_TRY(sync());  // bits is reused
    }
    for (const auto& e : quant_) {
        if (!include_mtp && is_mtp(e.id)) continue;
        const std::string name = checkpoint_name(e.id);
        const StTensor* t = st.find(name);
        if (name.empty() || t == nullptr) return missing(name.empty() ? std::to_string(e.id) : name);
        const std::string sname = name.substr(0, name.size() - 7) + ".weight_scale_inv";
        const StTensor* s = st.find(sname);
        if (t->dtype != StDType::F8_E4M3 || s == nullptr)
            return fail(HAI_ERR_UNSUPPORTED_DTYPE, "Expected scaled FP8 Qwen weight: " + name);
        if (!shape_ok(*t, e.rows, e.cols) || t->shape.size() != 2)
            return fail(HAI_ERR_INVALID_MODEL, "Qwen weight " + name + " has shape " + shape_text(*t));
        const int64_t sr = (e.rows + 127) / 128, sc = (e.cols + 127) / 128;
        if (s->shape.size() != 2 || s->shape[0] != sr || s->shape[1] != sc)
            return fail(HAI_ERR_INVALID_MODEL, "Qwen scale " + sname + " has shape " + shape_text(*s) +
                                                   ", expected the 128 x 128 block grid [" + std::to_string(sr) +
                                                   ", " + std::to_string(sc) + "]");
        host.resize(static_cast<size_t>(t->bytes()));
        if (const int rc = st.read(*t, host.data(), &err); rc != HAI_OK) return fail(rc, err);
        HAI_TRY(hai_memcpy_h2d_2d(e.q, static_cast<size_t>(e.ldq), host.data(), static_cast<size_t>(e.cols),
                                  static_cast<size_t>(e.cols), static_cast<size_t>(e.rows), stream_));
        HAI_TRY(sync());
        // block scales to fp32 (load_as_fp32: BF16 widened exactly)
        std::vector<float> scales(static_cast<size_t>(sr * sc));
        if (s->dtype == StDType::F32) {
            if (const int rc = st.read(*s, scales.data(), &err); rc != HAI_OK) return fail(rc, err);
        } else if (s->dtype == StDType::BF16) {
            std::vector<uint16_t> sb(scales.size());
            if (const int rc = st.read(*s, sb.data(), &err); rc != HAI_OK) return fail(rc, err);
            for (size_t i = 0; i < sb.size(); ++i) {
                const uint32_t u = static_cast<uint32_t>(sb[i]) << 16;
                std::memcpy(&scales[i], &u, 4);
            }
        } else {
            return fail(HAI_ERR_UNSUPPORTED_DTYPE, "Only BF16 and FP32 can be loaded as FP32: " + sname);
        }
        HAI_TRY(hai_memcpy_h2d(e.s, scales.data(), scales.size() * 4, stream_));
        HAI_TRY(sync());
    }
    return HAI_OK;
}

int64_t Engine::read_tensor(uint32_t id, uint16_t* out, int64_t capacity) {
    for (const auto& t : tensors_) {
        if (t.id != id) continue;
        const int64_t n = t.rows * t.cols;
        if (out == nullptr) return n;
        if (capacity < n) return -1;
        std::vector<uint16_t> tmp(static_cast<size_t>((t.rows - 1) * t.ld + t.cols));
        if (hai_memcpy_d2h(tmp.data(), t.ptr, tmp.size() * 2, stream_) != HAI_OK || sync() != HAI_OK) return -1;
        for (int64_t r = 0; r < t.rows; ++r)
            std::memcpy(out + r * t.cols, tmp.data() + r * t.ld, static_cast<size_t>(t.cols) * 2);
        return n;
    }
    return -1;
}

int Engine::flush_pending() {
    if (pending_.h == nullptr) return HAI_OK;
    const PendingResidual p = pending_;
    pending_ = PendingResidual{};
    return hai_mfma_residual_rmsnorm_bf16(p.h, p.ld, mfma_ws_, mfma_ws_bytes_, p.M, p.N, p.splits, nullptr, 0.0f, 0,
                                          nullptr, 0, stream_);
}

int Engine::gemm(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const Lin& w, int64_t M, int64_t N,
                 int64_t K, int epi, const uint16_t* res, int64_t ldres) {
    HAI_TRY(flush_pending());  // the workspace is about to be reused
    if (prof_record_) prof_calls_.push_back({y, ldy, x, ldx, w, M, N, K, epi, res, ldres, nullptr, nullptr});
    if (use_mfma(M) && M > kTiledMinRows && K % 64 == 0) {
        // prompt-sized row counts: both operands tiled on the matrix cores,
        // compute bound (FP8 codes decoded exactly as they are staged)
        if (w.q != nullptr)
            return hai_gemm_fp8_tiled(y, ldy, x, ldx, w.q, w.s, w.map, M, N, K, epi | HAI_FP8_NO_SPECIAL_CODES, res,
                                      ldres, stream_);
        return hai_gemm_bf16_tiled(y, ldy, x, ldx, w.w, M, N, K, epi, res, ldres, stream_);
    }
    if (use_mfma(M) && epi == HAI_EPI_RESIDUAL && res == y && ldres == ldy && M <= 128 && N % 8 == 0 && N <= 8192 &&
        !prof_record_) {
        // residual in place: leave the split partials for the next RMSNorm
        const int splits = hai_gemm_mfma_splits(M, N, K, mfma_ws_, mfma_ws_bytes_);
        if (splits > 1) {
            const int keep = HAI_EPI_RESIDUAL | HAI_MFMA_KEEP_PARTIALS;
            if (w.q != nullptr)
                HAI_TRY(hai_gemm_fp8_mfma(y, ldy, x, ldx, w.q, w.s, w.map, M, N, K, keep | HAI_FP8_NO_SPECIAL_CODES,
                                          res, ldres, mfma_ws_, mfma_ws_bytes_, stream_));
            else
                HAI_TRY(hai_gemm_bf16_mfma(y, ldy, x, ldx, w.w, M, N, K, keep, res, ldres, mfma_ws_,
                                           mfma_ws_bytes_, stream_));
            pending_ = PendingResidual{y, ldy, M, N, splits};
            return HAI_OK;
        }
    }
    if (use_mfma(M)) {
        for (int64_t m0 = 0; m0 < M; m0 += 128) {
            const int64_t mm = std::min<int64_t>(128, M - m0);
            const uint16_t* rm = res ? res + m0 * ldres : nullptr;
            if (w.q != nullptr)
                HAI_TRY(hai_gemm_fp8_mfma(y + m0 * ldy, ldy, x + m0 * ldx, ldx, w.q, w.s, w.map, mm, N, K,
                                          epi | HAI_FP8_NO_SPECIAL_CODES, rm, ldres, mfma_ws_, mfma_ws_bytes_,
                                          stream_));
            else
                HAI_TRY(hai_gemm_bf16_mfma(y + m0 * ldy, ldy, x + m0 * ldx, ldx, w.w, mm, N, K, epi, rm, ldres,
                                           mfma_ws_, mfma_ws_bytes_, stream_));
        }
        return HAI_OK;
    }
    // bf16 weights: one launch for any M (16-row batches inside it);
    // the FP8 skinny kernel takes 16 rows per launch.  Rows are
    // independent, so neither split changes a bit.
    if (w.q == nullptr) return hai_gemm_bf16(y, ldy, x, ldx, w.w, M, N, K, epi, res, ldres, stream_);
    for (int64_t m0 = 0; m0 < M; m0 += 16) {
        const int64_t mm = std::min<int64_t>(16, M - m0);
        uint16_t* ym = y + m0 * ldy;
        const uint16_t* xm = x + m0 * ldx;
        const uint16_t* rm = res ? res + m0 * ldres : nullptr;
        // the engine's codes come from the saturating quantiser: never 0x7F / 0xFF
        HAI_TRY(hai_gemm_fp8_bf16(ym, ldy, xm, ldx, w.q, w.s, w.map, mm, N, K, epi | HAI_FP8_NO_SPECIAL_CODES, rm,
                                  ldres, stream_));
    }
    return HAI_OK;
}

int Engine::norm_gemm(uint16_t* y, int64_t ldy, const uint16_t* x, const uint16_t* nw, uint16_t* xn_out,
                      const Lin& w, int64_t M, int64_t N, int epi, const uint16_t* res, int64_t ldres) {
    const int64_t H = d_.H;
    // lm_head-sized outputs stream faster from the plain kernel than the norm
    // prologue saves (measured on MI355X), so they normalise separately; so
    // do launches of more than 16 rows.
    if (N > kFusedNormMaxN || M > 16 || use_mfma(M)) {
        uint16_t* xn = xn_out != nullptr ? xn_out : xn_;
        if (pending_.h != nullptr && pending_.h == x && pending_.M == M && pending_.N == H && pending_.ld == H) {
            // the previous residual GEMM's split sum, residual add and this norm in one launch
            const PendingResidual p = pending_;
            pending_ = PendingResidual{};
            HAI_TRY(hai_mfma_residual_rmsnorm_bf16(p.h, p.ld, mfma_ws_, mfma_ws_bytes_, M, H, p.splits, nw,
                                                   cfg_.rms_eps, 1, xn, H, stream_));
        } else {
            HAI_TRY(flush_pending());
            HAI_TRY(hai_rmsnorm_bf16(xn, H, x, H, nw, M, H, cfg_.rms_eps, 1, stream_));
        }
        return gemm(y, ldy, xn, H, w, M, N, H, epi, res, ldres);
    }
    HAI_TRY(flush_pending());
    // Above the fused limit the call runs RMSNorm then GEMM through xn_.
    if (xn_out == nullptr && M * H > HAI_GEMM_RMSNORM_FUSED_MAX) xn_out = xn_;
    if (prof_record_) prof_calls_.push_back({y, ldy, x, H, w, M, N, H, epi, res, ldres, nw, xn_out});
    if (w.q != nullptr)
        HAI_TRY(hai_gemm_rmsnorm_fp8_bf16(y, ldy, x, H, nw, cfg_.rms_eps, 1, xn_out, H, w.q, w.s, w.map, M, N, H,
                                          epi | HAI_FP8_NO_SPECIAL_CODES, res, ldres, stream_));
    else
        HAI_TRY(hai_gemm_rmsnorm_bf16(y, ldy, x, H, nw, cfg_.rms_eps, 1, xn_out, H, w.w, M, N, H, epi, res, ldres,
                                      stream_));
    return HAI_OK;
}

int Engine::reset_state() {
    // Committed lengths to zero; the DeltaNet state slot 0 of every layer and
    // sequence must start at zero (conv history before position 0 is read as
    // zero).
    HAI_TRY(hai_memset(d_tlen_, 0, static_cast<size_t>(B_) * 4, stream_));
    HAI_TRY(hai_memset(d_mlen_, 0, static_cast<size_t>(B_) * 4, stream_));
    const size_t slot_bytes = static_cast<size_t>(B_ * d_.nv * d_.dv * d_.dk) * 4;
    for (auto& L : layers_)
        if (!L.attn) HAI_TRY(hai_memset(L.state, 0, slot_bytes, stream_));
    rs_.assign(static_cast<size_t>(B_), RoundState{});
    ndraft_host_.clear();
    return HAI_OK;
}

// One gated-GQA sub-layer over T rows of each sequence: input RMSNorm fused
// into the q|gate,k,v projection, residual added into h
// (qwen_attention_reference -> GatedGQAAttention::forward_impl,
// attention.cc:301-599).
int Engine::attention_layer(const LayerWeights& L, int64_t T, uint16_t* h, const int32_t* lens, uint16_t* kc,
                            uint16_t* vc) {
    const auto& d = d_;
    const int64_t rows = B_ * T;
    HAI_TRY(norm_gemm(proj_, d.Nqkv, h, L.in_ln, nullptr, lin(L.w_qkv, L.f_qkv), rows, d.Nqkv, HAI_EPI_STORE,
                      nullptr, 0));
    if (mfma_ || fast_) {
        // tolerance mode: Q.K^T and P.V on the matrix cores
        HAI_TRY(hai_qkv_rmsnorm_rope_append_bf16(q_, gate_, kc, vc, cap_, proj_, d.Nqkv, L.q_norm, L.k_norm,
                                                 rope_cos_, rope_sin_, cap_, B_, T, d.nq, d.nkv, d.D, d.R, lens, 0,
                                                 cfg_.rms_eps, stream_));
        HAI_TRY(hai_gqa_verify_mfma_bf16(att_, q_, gate_, kc, vc, cap_, gqa_scratch_, B_, T, d.nq, d.nkv, d.D, lens,
                                         static_cast<int32_t>(T), cap_, stream_));
    } else {
        // the q / k norms, RoPE and the cache append inside the attention's
        // partial pass (bit-identical to the two launches)
        HAI_TRY(hai_gqa_verify_fused_bf16(att_, gate_, proj_, d.Nqkv, L.q_norm, L.k_norm, rope_cos_, rope_sin_, cap_,
                                          d.R, cfg_.rms_eps, kc, vc, cap_, gqa_scratch_, B_, T, d.nq, d.nkv, d.D,
                                          lens, static_cast<int32_t>(T), cap_, stream_));
    }
    return gemm(h, d.H, att_, d.qw, lin(L.w_o, L.f_o), rows, d.H, d.qw, HAI_EPI_RESIDUAL, h, d.H);
}

// qwen_mlp_reference (qwen_reference.cc:146-175): post-norm, SwiGLU, down
// projection with the residual add fused.
int Engine::mlp(const LayerWeights& L, int64_t T, uint16_t* h) {
    const auto& d = d_;
    const int64_t rows = B_ * T;
    HAI_TRY(norm_gemm(act_, d.F, h, L.post_ln, nullptr, lin(L.w_gu, L.f_gu), rows, 2 * d.F, HAI_EPI_SILU_MUL,
                      nullptr, 0));
    return gemm(h, d.H, act_, d.F, lin(L.w_down, L.f_down), rows, d.H, d.F, HAI_EPI_RESIDUAL, h, d.H);
}

// The fused DeltaNet verify layer over the T rows in proj_ (a|b from proj
// columns off_a / off_b, or formed from the normalised rows xn and w_ab) into
// dnout_, with the state writes sw asks for.
int Engine::deltanet(const LayerWeights& L, int64_t T, StateWrites sw, int64_t off_a, int64_t off_b,
                     const uint16_t* xn, const uint16_t* w_ab) {
    const auto& d = d_;
    if (sw == StateWrites::kFinal) {
        if (w_ab != nullptr)
            return hai_deltanet_verify_ab_bf16(dnout_, d.vw, proj_, d.Nin, 0, d.C, xn, d.H, w_ab, d.H, L.conv_w,
                                               L.ring, ring_, L.state, nslots_, 0, L.a_log, L.dt_bias, L.lin_norm,
                                               d_tlen_, 0, B_, T, d.nk, d.nv, d.dk, d.dv, d.Kc, cfg_.rms_eps, stream_);
        return hai_deltanet_verify_bf16(dnout_, d.vw, proj_, d.Nin, 0, d.C, off_a, off_b, L.conv_w, L.ring, ring_,
                                        L.state, nslots_, 0, L.a_log, L.dt_bias, L.lin_norm, d_tlen_, 0, B_, T, d.nk,
                                        d.nv, d.dk, d.dv, d.Kc, cfg_.rms_eps, stream_);
    }
    return hai_deltanet_verify_rec_bf16(dnout_, d.vw, proj_, d.Nin, 0, d.C, off_a, off_b, xn, d.H, w_ab,
                                        w_ab != nullptr ? d.H : 0, L.conv_w, L.ring, ring_, L.state, nslots_, L.rec,
                                        d_vbase_, sw == StateWrites::kReplay ? 1 : 0, L.a_log, L.dt_bias,
                                        L.lin_norm, d_tlen_, 0, B_, T, d.nk, d.nv, d.dk, d.dv, d.Kc, cfg_.rms_eps,
                                        stream_);
}

// target_forward (generator.cc:550-634): T rows of every sequence (row b*T+t)
// on top of its committed caches; hf_ = post-final-norm hidden, logits_ =
// lm_head.  Committed lengths are not advanced here.
int Engine::forward_target(const int64_t* d_ids, int64_t T, StateWrites sw, Logits logits) {
    pending_ = PendingResidual{};  // a forward ends with a norm, which completes any residual; only
                                   // a failed one leaves a record, for rows this forward overwrites
    const auto& d = d_;
    const int64_t rows = B_ * T;
    HAI_TRY(hai_embedding_gather_bf16(h_, embed_, d_ids, rows, d.V, d.H, stream_));
    for (auto& L : layers_) {
        if (L.attn) {
            HAI_TRY(attention_layer(L, T, h_, d_tlen_, L.k_cache, L.v_cache));
        } else {
            // qwen_deltanet_reference (qwen_reference.cc:205-258).  The
            // DeltaNet kernel takes at most 16 tokens per launch: a verify
            // of 17 rows (width 16, one sequence) or a prompt chunk runs as
            // launches of 16, each starting from the state the previous one
            // left in slot (L + 16) % nslots and reading its conv history
            // from the ring (the library issues them).
            if (fast_) {
                // a prompt chunk: the whole in_proj [qkv | z | a | b] on the
                // tiled GEMMs (FP8: the bf16 a|b rows as a GEMM of their own
                // over the normalised rows), then the prefill DeltaNet kernel
                if (fp8_) {
                    HAI_TRY(norm_gemm(proj_, d.Nin, h_, L.in_ln, xn_, Lin(L.f_in), rows, d.C + d.vw, HAI_EPI_STORE,
                                      nullptr, 0));
                    HAI_TRY(gemm(proj_ + d.C + d.vw, d.Nin, xn_, d.H, L.w_ab, rows, 2 * d.nv, d.H, HAI_EPI_STORE,
                                 nullptr, 0));
                } else {
                    HAI_TRY(norm_gemm(proj_, d.Nin, h_, L.in_ln, nullptr, L.w_in, rows, d.Nin, HAI_EPI_STORE, nullptr,
                                      0));
                }
                HAI_TRY(flush_pending());
                HAI_TRY(hai_deltanet_prefill_bf16(dnout_, d.vw, proj_, d.Nin, 0, d.C, d.C + d.vw, d.C + d.vw + d.nv,
                                                  L.conv_w, L.ring, ring_, L.state, nslots_, L.a_log, L.dt_bias,
                                                  L.lin_norm, d_tlen_, 0, B_, T, d.nk, d.nv, d.dk, d.dv, d.Kc,
                                                  cfg_.rms_eps, dn_ws_, dn_ws_bytes_, stream_));
            } else if (fp8_) {
                // FP8 qkv|z with the norm fused, writing the normalised rows;
                // the bf16 a|b projection of each head is formed from them
                // inside the DeltaNet kernel (no launch of its own)
                HAI_TRY(norm_gemm(proj_, d.Nin, h_, L.in_ln, xn_, Lin(L.f_in), rows, d.C + d.vw, HAI_EPI_STORE,
                                  nullptr, 0));
                HAI_TRY(flush_pending());
                HAI_TRY(deltanet(L, T, sw, 0, 0, xn_, L.w_ab));
            } else if (use_mfma(rows)) {
                // matrix-core mode: the qkv|z rows only (16384 rows at the 27B
                // shape, whole 64-row tiles that load every CU alike, where
                // [qkv|z|a|b] leaves a half tile); a|b formed in the DeltaNet
                // kernel from the normalised rows, as with FP8 weights
                HAI_TRY(norm_gemm(proj_, d.Nin, h_, L.in_ln, xn_, L.w_in, rows, d.C + d.vw, HAI_EPI_STORE, nullptr,
                                  0));
                HAI_TRY(flush_pending());
                HAI_TRY(deltanet(L, T, sw, 0, 0, xn_, L.w_in + (d.C + d.vw) * d.H));
            } else {
                HAI_TRY(norm_gemm(proj_, d.Nin, h_, L.in_ln, nullptr, L.w_in, rows, d.Nin, HAI_EPI_STORE, nullptr,
                                  0));
                HAI_TRY(deltanet(L, T, sw, d.C + d.vw, d.C + d.vw + d.nv, nullptr, nullptr));
            }
            HAI_TRY(gemm(h_, d.H, dnout_, d.vw, lin(L.w_out, L.f_out), rows, d.H, d.vw, HAI_EPI_RESIDUAL, h_, d.H));
        }
        HAI_TRY(mlp(L, T, h_));
    }
    if (logits == Logits::kAll)
        return norm_gemm(logits_, d.V, h_, final_norm_, hf_, lm_head_, rows, d.V, HAI_EPI_STORE, nullptr, 0);
    // a prompt chunk: the final norm of every row (the MTP rows read them),
    // lm_head for the last row of each sequence (rows 0..B-1 of logits_) or none
    HAI_TRY(flush_pending());
    HAI_TRY(hai_rmsnorm_bf16(hf_, d.H, h_, d.H, final_norm_, rows, d.H, cfg_.rms_eps, 1, stream_));
    if (logits == Logits::kNone) return HAI_OK;
    return gemm(logits_, d.V, hf_ + (T - 1) * d.H, T * d.H, lm_head_, B_, d.V, d.H, HAI_EPI_STORE, nullptr, 0);
}

// MTP input rows x = fc([RMSNorm(emb) | RMSNorm(hidden)]) (generator.cc:152-160)
// followed by only the part of the MTP decoder layer that the cache keeps:
// input RMSNorm, the K/V projection rows and the K RMSNorm+RoPE append.  The
// reference's prompt prefill and correction recovery discard the MTP output
// (generator.cc:673-699, 977-1003), so the cache state is identical.  T rows
// per sequence; add_len advances every MTP length by T.
int Engine::mtp_kv_rows(const int64_t* d_ids, const uint16_t* d_hidden, int64_t T, bool add_len) {
    pending_ = PendingResidual{};  // a forward ends with a norm, which completes any residual; only
                                   // a failed one leaves a record, for rows this forward overwrites
    const auto& d = d_;
    const int64_t rows = B_ * T;
    HAI_TRY(hai_embedding_gather_bf16(emb_, embed_, d_ids, rows, d.V, d.H, stream_));
    HAI_TRY(hai_rmsnorm_bf16(xn_, 2 * d.H, emb_, d.H, pre_emb_, rows, d.H, cfg_.rms_eps, 1, stream_));
    HAI_TRY(hai_rmsnorm_bf16(xn_ + d.H, 2 * d.H, d_hidden, d.H, pre_hid_, rows, d.H, cfg_.rms_eps, 1, stream_));
    HAI_TRY(gemm(h_, d.H, xn_, 2 * d.H, fc_, rows, d.H, 2 * d.H, HAI_EPI_STORE, nullptr, 0));
    // K and V rows of the fused attention projection only.
    HAI_TRY(norm_gemm(proj_, 2 * d.kvw, h_, mtp_.in_ln, nullptr, lin(mtp_.w_qkv, mtp_.f_qkv).rows(2 * d.qw, d.H),
                      rows, 2 * d.kvw, HAI_EPI_STORE, nullptr, 0));
    HAI_TRY(hai_kv_rmsnorm_rope_append_bf16(mtp_.k_cache, mtp_.v_cache, cap_, proj_, proj_ + d.kvw, 2 * d.kvw,
                                            mtp_.k_norm, rope_cos_, rope_sin_, cap_, B_, T, d.nkv, d.D, d.R, d_mlen_,
                                            0, cfg_.rms_eps, stream_));
    if (add_len) HAI_TRY(hai_add_i32(d_mlen_, nullptr, static_cast<int32_t>(T), B_, stream_));
    return HAI_OK;
}

// One draft step of every sequence: the full MTP forward
// (qwen_mtp_forward_reference, generator.cc:139-183) of one row per
// sequence, lm_head and argmax (generator.cc:784-811).  d_id / d_cand are
// [B], d_hin / d_mh [B][H]; every MTP cache grows by one row.
int Engine::mtp_draft_step(const int64_t* d_id, const uint16_t* d_hin, uint16_t* d_mh, int64_t* d_cand) {
    pending_ = PendingResidual{};  // a forward ends with a norm, which completes any residual; only
                                   // a failed one leaves a record, for rows this forward overwrites
    const auto& d = d_;
    HAI_TRY(hai_embedding_gather_bf16(emb_, embed_, d_id, B_, d.V, d.H, stream_));
    HAI_TRY(hai_rmsnorm_bf16(xn_, 2 * d.H, emb_, d.H, pre_emb_, B_, d.H, cfg_.rms_eps, 1, stream_));
    HAI_TRY(hai_rmsnorm_bf16(xn_ + d.H, 2 * d.H, d_hin, d.H, pre_hid_, B_, d.H, cfg_.rms_eps, 1, stream_));
    HAI_TRY(gemm(h_, d.H, xn_, 2 * d.H, fc_, B_, d.H, 2 * d.H, HAI_EPI_STORE, nullptr, 0));
    HAI_TRY(attention_layer(mtp_, 1, h_, d_mlen_, mtp_.k_cache, mtp_.v_cache));
    HAI_TRY(mlp(mtp_, 1, h_));
    HAI_TRY(norm_gemm(logits_, d.V, h_, mtp_norm_, d_mh, lm_head_, B_, d.V, HAI_EPI_STORE, nullptr, 0));
    HAI_TRY(hai_argmax_rows_bf16(d_cand, logits_, d.V, B_, d.V, argmax_scratch_, stream_));
    HAI_TRY(hai_add_i32(d_mlen_, nullptr, 1, B_, stream_));
    return HAI_OK;
}

// Prompt prefill in chunks of pchunk_ rows per sequence (rows are independent
// and the recurrences are sequential, so chunking does not change a bit),
// each chunk followed by its MTP prompt rows (emb(t_i) paired with the
// hidden of t_i).  ids [B][P]; hidden_out [B][P][H], logits_out [B][P][V].
int Engine::prefill_chunks(const int32_t* ids, int64_t P, uint16_t* hidden_out, uint16_t* logits_out) {
    // fast prefill: every GEMM and the attention of the chunks on the matrix cores
    struct FastScope {
        bool& flag;
        FastScope(bool& f, bool on) : flag(f) { flag = on; }
        ~FastScope() { flag = false; }
    } scope(fast_, fast_prefill_);
    const auto& d = d_;
    std::vector<int64_t> chunk(static_cast<size_t>(B_ * pchunk_));
    for (int64_t off = 0; off < P; off += pchunk_) {
        const int64_t T = std::min<int64_t>(pchunk_, P - off);
        for (int64_t b = 0; b < B_; ++b)
            for (int64_t t = 0; t < T; ++t) chunk[static_cast<size_t>(b * T + t)] = ids[b * P + off + t];
        HAI_TRY(hai_memcpy_h2d(d_ids_, chunk.data(), static_cast<size_t>(B_ * T) * 8, stream_));
        // the verify-step prefill keeps every row's logits (one weight
        // stream serves all rows); a fast chunk computes only the last row's,
        // and only in the last chunk (lm_head of the other rows in slices
        // when the caller asks for them)
        const bool last_chunk = off + T == P;
        const Logits lg = !fast_prefill_ ? Logits::kAll : last_chunk ? Logits::kLast : Logits::kNone;
        HAI_TRY(forward_target(d_ids_, T, StateWrites::kFinal, lg));
        HAI_TRY(hai_add_i32(d_tlen_, nullptr, static_cast<int32_t>(T), B_, stream_));
        if (last_chunk) {
            // the last prompt row of every sequence: its argmax is the first target
            if (lg == Logits::kLast)
                HAI_TRY(hai_argmax_rows_bf16(d_next_, logits_, d.V, B_, d.V, argmax_scratch_, stream_));
            else
                HAI_TRY(hai_argmax_rows_bf16(d_next_, logits_ + (T - 1) * d.V, T * d.V, B_, d.V, argmax_scratch_,
                                             stream_));
        }
        for (int64_t b = 0; b < B_; ++b) {
            if (hidden_out)
                HAI_TRY(hai_memcpy_d2h(hidden_out + (b * P + off) * d.H, hf_ + b * T * d.H,
                                       static_cast<size_t>(T * d.H) * 2, stream_));
            if (logits_out && lg == Logits::kAll) {
                HAI_TRY(hai_memcpy_d2h(logits_out + (b * P + off) * d.V, logits_ + b * T * d.V,
                                       static_cast<size_t>(T * d.V) * 2, stream_));
            } else if (logits_out) {
                const int64_t slice = B_ * tmax_;
                for (int64_t t0 = 0; t0 < T; t0 += slice) {
                    const int64_t n = std::min(slice, T - t0);
                    HAI_TRY(gemm(logits_, d.V, hf_ + (b * T + t0) * d.H, d.H, lm_head_, n, d.V, d.H, HAI_EPI_STORE,
                                 nullptr, 0));
                    HAI_TRY(hai_memcpy_d2h(logits_out + (b * P + off + t0) * d.V, logits_,
                                           static_cast<size_t>(n * d.V) * 2, stream_));
                    HAI_TRY(sync());  // logits_ is rewritten by the next slice
                }
            }
        }
        HAI_TRY(mtp_kv_rows(d_ids_, hf_, T, true));
        if (last_chunk) {
            // and its hidden feeds the first draft
            for (int64_t b = 0; b < B_; ++b)
                HAI_TRY(hai_memcpy_d2d(h_prev_ + b * d.H, hf_ + (b * T + T - 1) * d.H, static_cast<size_t>(d.H) * 2,
                                       stream_));
        }
        if (hidden_out || logits_out) HAI_TRY(sync());
    }
    for (auto& r : rs_) {
        r.target_len = P;
        r.mtp_len = P;
    }
    return HAI_OK;
}

int Engine::check_ids(const int32_t* ids, int64_t n, const char* what) {
    if (n > 0 && ids == nullptr) return fail(HAI_ERR_INVALID_ARGUMENT, std::string(what) + ": null token ids");
    for (int64_t i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= d_.V)
            return fail(HAI_ERR_INVALID_ARGUMENT, std::string(what) + ": token id " + std::to_string(ids[i]) +
                                                      " outside the vocabulary");
    return HAI_OK;
}

int Engine::forward_rows(const int32_t* ids, int64_t T, uint16_t* hidden, uint16_t* logits) {
    if (T <= 0 || T > cap_) return fail(HAI_ERR_INVALID_ARGUMENT, "forward_rows: T out of range");
    HAI_TRY(check_ids(ids, B_ * T, "forward"));
    HAI_TRY(reset_state());
    HAI_TRY(prefill_chunks(ids, T, hidden, logits));
    return sync();
}

int Engine::prefill(const int32_t* prompts, int64_t P, int64_t max_new) {
    if (P <= 0 || max_new <= 0 || P + max_new + tmax_ > cap_)
        return fail(HAI_ERR_INVALID_ARGUMENT, "prefill: prompt + max_new exceeds max_context");
    HAI_TRY(check_ids(prompts, B_ * P, "prefill"));
    HAI_TRY(reset_state());
    HAI_TRY(prefill_chunks(prompts, P, nullptr, nullptr));
    std::vector<int64_t> next(static_cast<size_t>(B_));
    HAI_TRY(read_i64(d_next_, next.data(), B_));
    for (int64_t b = 0; b < B_; ++b) {
        auto& r = rs_[static_cast<size_t>(b)];
        r.next_target = next[static_cast<size_t>(b)];
        r.max_new = max_new;
        r.emitted = 0;
        r.done = false;
    }
    return HAI_OK;
}

int Engine::generate_greedy(const int32_t* prompt, int64_t P, int64_t max_new, const int32_t* eos, int64_t n_eos,
                            int32_t* out, int64_t* n_out) {
    if (B_ != 1) return fail(HAI_ERR_INVALID_ARGUMENT, "generate_greedy: one sequence only");
    HAI_TRY(prefill(prompt, P, max_new));
    int64_t emitted = 0;
    int64_t next = rs_[0].next_target;
    while (true) {
        out[emitted++] = static_cast<int32_t>(next);
        if (emitted >= max_new || in_set(eos, n_eos, next)) break;
        HAI_TRY(forward_target(d_next_, 1, StateWrites::kFinal));
        HAI_TRY(hai_add_i32(d_tlen_, nullptr, 1, 1, stream_));
        HAI_TRY(hai_argmax_rows_bf16(d_next_, logits_, d_.V, 1, d_.V, argmax_scratch_, stream_));
        HAI_TRY(read_i64(d_next_, &next, 1));
    }
    *n_out = emitted;
    return HAI_OK;
}

template <typename F>
int Engine::replay(void** slot, F&& enqueue) {
    if (!use_graphs_) return enqueue();
    if (*slot == nullptr) {
        HAI_TRY(hai_graph_begin_capture(stream_));
        const int rc = enqueue();
        void* exec = nullptr;
        const int rc_end = hai_graph_end_capture(stream_, &exec);
        if (rc != HAI_OK) return rc;
        if (rc_end != HAI_OK) return lib_fail(rc_end, "graph capture");
        *slot = exec;
    }
    HAI_TRY(hai_graph_launch(*slot, stream_));
    return HAI_OK;
}

// Draft i of a round of verify width T reads candidate i of every sequence
// (vids[b*T + i]; column 0 is next_target) and the hidden that produced it,
// and writes candidate i+1.
int Engine::draft_step_at(int64_t i, int64_t T) {
    const uint16_t* hin = i == 0 ? h_prev_ : mh_[(i - 1) % 2];
    return replay(&draft_graphs_[static_cast<size_t>(T * tmax_ + i)], [&]() -> int {
        if (B_ == 1) return mtp_draft_step(d_vids_ + i, hin, mh_[i % 2], d_vids_ + i + 1);
        HAI_TRY(hai_copy_i64_strided(d_dids_, 1, d_vids_ + i, T, B_, stream_));
        HAI_TRY(mtp_draft_step(d_dids_, hin, mh_[i % 2], d_cand_));
        HAI_TRY(hai_copy_i64_strided(d_vids_ + i + 1, T, d_cand_, 1, B_, stream_));
        return HAI_OK;
    });
}

// Verify forward of T rows per sequence + fused argmax/acceptance (commits on
// device).  The next target of every sequence lands in d_next_.
int Engine::verify_step(int64_t T) {
    return replay(&verify_graphs_[static_cast<size_t>(T)], [&]() -> int {
        HAI_TRY(forward_target(d_vids_, T, StateWrites::kRecord));
        HAI_TRY(hai_verify_argmax_accept_bf16(logits_, d_.V, hf_, d_.H, d_vids_, d_ndraft_, B_, T, d_preds_,
                                              d_result_, d_tlen_, d_mlen_, d_next_, rec_hidden_, h_prev_,
                                              argmax_scratch_, stream_));
        return HAI_OK;
    });
}

// Mismatch path, batched over every sequence: MTP recovery row (emb(corr),
// hidden of the last accepted row), then the forward of corr on the
// committed prefix; for the sequences whose round ended in a rejection its
// argmax becomes the next target and its hidden feeds the next draft, and
// both rows are committed (hai_correction_commit_bf16).  Fully accepted
// sequences compute a row past their committed length that the next round
// overwrites.
int Engine::correction_step() {
    return replay(&corr_graph_, [&]() -> int {
        HAI_TRY(mtp_kv_rows(d_next_, rec_hidden_, 1, false));
        HAI_TRY(forward_target(d_next_, 1, StateWrites::kReplay));
        HAI_TRY(hai_argmax_rows_bf16(d_cand_, logits_, d_.V, B_, d_.V, argmax_scratch_, stream_));
        HAI_TRY(hai_correction_commit_bf16(d_result_, d_cand_, hf_, d_.H, B_, d_next_, h_prev_, d_tlen_, d_mlen_,
                                           stream_));
        return HAI_OK;
    });
}

// One lockstep round of the reference loop body (generator.cc:720-1028) for
// every sequence still generating.
int Engine::one_round(int64_t width, const RoundIo& io, bool* any_live) {
    const size_t Bz = static_cast<size_t>(B_);
    // sequences whose next target ends the generation emit it without a round
    std::vector<int64_t> pc(Bz, 0);
    int64_t k = 0;
    bool live = false;
    for (size_t b = 0; b < Bz; ++b) {
        auto& st = rs_[b];
        if (st.done) continue;
        const int64_t remaining = st.max_new - st.emitted;
        if (in_set(io.eos, io.n_eos, st.next_target) || remaining <= 1) {
            io.out[static_cast<int64_t>(b) * io.out_ld + st.emitted++] = static_cast<int32_t>(st.next_target);
            st.done = true;
            continue;
        }
        pc[b] = std::min<int64_t>(width, remaining - 1);  // width <= tmax_ - 1, checked by the callers
        k = std::max(k, pc[b]);
        live = true;
    }
    *any_live = live;
    if (!live) return HAI_OK;
    const int64_t T = k + 1;
    std::vector<int64_t> mtp_len0(Bz), target_len0(Bz);
    for (size_t b = 0; b < Bz; ++b) {
        mtp_len0[b] = rs_[b].mtp_len;
        target_len0[b] = rs_[b].target_len;
    }
    // this round's next targets into column 0 of the [B][T] id block
    HAI_TRY(hai_copy_i64_strided(d_vids_, T, d_next_, 1, B_, stream_));

    // ---- draft (chained MTP proposals) ----
    // With an EOS set a chain can end early (generator.cc:845-847); the
    // counts then live on the device (hai_draft_chain_count) and come back
    // with the verify result, so the round still syncs once.  Without one
    // every chain runs to its cap and the host knows the counts.
    auto t0 = Clock::now();
    const int64_t syncs0 = syncs_;
    const bool chain_on_device = io.n_eos > 0;
    int32_t* h_cap = h_stage_;
    int32_t* h_nd = h_stage_ + Bz;
    int32_t* h_delta = h_stage_ + 2 * Bz;
    if (chain_on_device) {
        for (size_t b = 0; b < Bz; ++b) h_cap[b] = static_cast<int32_t>(pc[b]);
        HAI_TRY(hai_memcpy_h2d(d_pcap_, h_cap, Bz * 4, stream_));
    }
    for (int64_t i = 0; i < k; ++i) {
        HAI_TRY(draft_step_at(i, T));
        if (io.ov != nullptr)
            for (size_t b = 0; b < Bz; ++b) {
                const int64_t pos = rs_[b].emitted + 1 + i;
                if (i < pc[b] && pos < io.n_ov)
                    HAI_TRY(hai_copy_i64_strided(d_vids_ + static_cast<int64_t>(b) * T + i + 1, 1,
                                                 io.ov + static_cast<int64_t>(b) * io.n_ov + pos, 1, 1, stream_));
            }
        if (chain_on_device)
            HAI_TRY(hai_draft_chain_count(i, d_vids_, T, d_pcap_, d_eos_, io.n_eos, d_ndraft_, B_, stream_));
    }
    // Drafts beyond a sequence's own count leave MTP rows the accept kernel
    // must not see: roll the lengths back (mtp_len += count - k) and pass
    // the counts.
    std::vector<int64_t> kd(Bz);
    if (chain_on_device) {
        HAI_TRY(hai_add_i32(d_mlen_, d_ndraft_, static_cast<int32_t>(-k), B_, stream_));
        ndraft_host_.clear();  // the device counts are read back with the verify result
    } else {
        std::vector<int32_t> nd(Bz);
        bool uneven = false;
        for (size_t b = 0; b < Bz; ++b) {
            kd[b] = pc[b];
            nd[b] = static_cast<int32_t>(pc[b]);
            h_delta[b] = static_cast<int32_t>(pc[b] - k);
            uneven = uneven || h_delta[b] != 0;
        }
        if (uneven) {
            HAI_TRY(hai_memcpy_h2d(d_delta_, h_delta, Bz * 4, stream_));
            HAI_TRY(hai_add_i32(d_mlen_, d_delta_, 0, B_, stream_));
        }
        if (nd != ndraft_host_) {
            std::copy(nd.begin(), nd.end(), h_nd);
            HAI_TRY(hai_memcpy_h2d(d_ndraft_, h_nd, Bz * 4, stream_));
            ndraft_host_ = nd;
        }
    }
    const double draft_s = seconds_since(t0);

    // ---- verify + fused argmax/accept ----
    t0 = Clock::now();
    HAI_TRY(verify_step(T));
    const int32_t* res = static_cast<const int32_t*>(h_read_);
    const int64_t* preds = read_ids();
    const int64_t* ids = preds + Bz * static_cast<size_t>(T);
    HAI_TRY(hai_memcpy_d2h(h_read_, d_result_, 4 * Bz * 4, stream_));
    HAI_TRY(hai_memcpy_d2h(read_ids(), d_preds_, Bz * static_cast<size_t>(T) * 8, stream_));
    HAI_TRY(hai_memcpy_d2h(read_ids() + Bz * static_cast<size_t>(T), d_vids_, Bz * static_cast<size_t>(T) * 8,
                           stream_));
    if (chain_on_device) HAI_TRY(hai_memcpy_d2h(h_nd, d_ndraft_, Bz * 4, stream_));
    HAI_TRY(sync());
    if (chain_on_device)
        for (size_t b = 0; b < Bz; ++b) kd[b] = h_nd[b];
    const double verify_s = seconds_since(t0);

    std::vector<bool> correct(Bz, false);
    std::vector<int32_t*> recs(Bz, nullptr);
    bool any_correct = false;
    for (size_t b = 0; b < Bz; ++b) {
        if (pc[b] == 0) continue;  // finished before this round
        auto& st = rs_[b];
        hai_spec_stats& stats = io.stats[b];
        int32_t* out = io.out + static_cast<int64_t>(b) * io.out_ld;
        const int64_t kb = kd[b];
        stats.max_proposal_width = std::max(stats.max_proposal_width, pc[b]);
        stats.proposed += kb;
        ++stats.rounds;
        stats.draft_seconds += draft_s;
        stats.verify_seconds += verify_s;
        int32_t* rec = nullptr;
        if (io.round_log != nullptr && io.n_log[b] < io.log_cap)
            rec = io.round_log + (static_cast<int64_t>(b) * io.log_cap + io.n_log[b]++) * HAI_ROUND_RECORD;
        recs[b] = rec;
        const int64_t a = res[4 * b];
        const bool full = res[4 * b + 1] != 0;
        const int64_t* cands = ids + b * static_cast<size_t>(T) + 1;
        const int64_t* pr = preds + b * static_cast<size_t>(T);
        if (rec != nullptr) {
            std::fill(rec, rec + HAI_ROUND_RECORD, -1);
            rec[0] = static_cast<int32_t>(kb);
            rec[1] = static_cast<int32_t>(a);
            rec[4] = static_cast<int32_t>(st.next_target);
            rec[5] = static_cast<int32_t>(st.emitted);
            for (int64_t i = 0; i < kb && i < 8; ++i) rec[8 + i] = static_cast<int32_t>(cands[i]);
        }
        out[st.emitted++] = static_cast<int32_t>(st.next_target);
        if (full) {
            for (int64_t i = 0; i < kb; ++i) out[st.emitted++] = static_cast<int32_t>(cands[i]);
            stats.accepted += a;
            st.next_target = pr[kb];
            st.target_len = target_len0[b] + kb + 1;
            st.mtp_len = mtp_len0[b] + kb;
            if (rec) { rec[2] = 1; rec[3] = -1; }
        } else {
            const int64_t corr = pr[a];
            stats.rejected += kb - a;
            ++stats.corrections;
            for (int64_t i = 0; i < a; ++i) out[st.emitted++] = static_cast<int32_t>(cands[i]);
            if (st.emitted < st.max_new) out[st.emitted++] = static_cast<int32_t>(corr);
            stats.accepted += a;
            if (rec) { rec[2] = 0; rec[3] = static_cast<int32_t>(corr); }
            // The reference replays [next, accepted..., corr] on the committed
            // caches; the rows before corr are already committed above.
            st.target_len = target_len0[b] + a + 2;
            // the reference's replay count (generator.cc:941-950): next,
            // the accepted candidates and the correction
            stats.replay_tokens += a + 2;
            if (st.emitted >= st.max_new || in_set(io.eos, io.n_eos, corr)) {
                st.mtp_len = mtp_len0[b];  // the reference stops before restoring the MTP checkpoint
                st.done = true;
            } else {
                correct[b] = true;
                any_correct = true;
                ++stats.mtp_recovery_tokens;
                st.mtp_len = mtp_len0[b] + a + 1;
            }
        }
    }
    if (any_correct) {
        // MTP checkpoint[a] (length already rolled back by the accept kernel)
        // plus the recovery row (emb(corr), hidden of row a)
        t0 = Clock::now();
        HAI_TRY(correction_step());
        std::vector<int64_t> next(Bz);
        HAI_TRY(read_i64(d_next_, next.data(), B_));
        const double corr_s = seconds_since(t0);
        for (size_t b = 0; b < Bz; ++b) {
            if (!correct[b]) continue;
            rs_[b].next_target = next[b];
            io.stats[b].correction_seconds += corr_s;
        }
    }
    for (size_t b = 0; b < Bz; ++b) {
        if (pc[b] == 0) continue;
        auto& st = rs_[b];
        if (recs[b] != nullptr) {
            recs[b][6] = static_cast<int32_t>(st.mtp_len);
            recs[b][7] = static_cast<int32_t>(st.target_len);
        }
        const int32_t* out = io.out + static_cast<int64_t>(b) * io.out_ld;
        if (!st.done && (st.emitted >= st.max_new || in_set(io.eos, io.n_eos, out[st.emitted - 1]))) st.done = true;
        io.stats[b].host_syncs += syncs_ - syncs0;
    }
    return HAI_OK;
}

int Engine::generate_speculative(const int32_t* prompts, int64_t P, int64_t max_new, int64_t width,
                                 const int32_t* eos, int64_t n_eos, const int32_t* override_tokens,
                                 int64_t n_override, int32_t* out, hai_spec_stats* stats, int32_t* round_log,
                                 int64_t round_log_cap, int64_t* n_out) {
    if (width < 1) return fail(HAI_ERR_INVALID_ARGUMENT, "width must be >= 1");
    if (width > tmax_ - 1)
        return fail(HAI_ERR_INVALID_ARGUMENT, "width " + std::to_string(width) + " needs max_verify_tokens >= " +
                                                  std::to_string(width + 1) + " (this engine verifies " +
                                                  std::to_string(tmax_) + " rows)");
    if (override_tokens != nullptr) HAI_TRY(check_ids(override_tokens, B_ * n_override, "draft override"));
    // a finished sequence keeps running with the batch: leave room for its
    // rows until the slowest sequence ends
    if (B_ > 1 && P + (width + 2) * max_new + tmax_ > cap_)
        return fail(HAI_ERR_INVALID_ARGUMENT, "generate_speculative: batched decode needs max_context >= "
                                              "P + (width + 2) * max_new + max_verify_tokens");
    const size_t Bz = static_cast<size_t>(B_);
    std::vector<hai_spec_stats> st(Bz, hai_spec_stats{});
    auto t0 = Clock::now();
    HAI_TRY(prefill(prompts, P, max_new));
    const double prefill_s = seconds_since(t0);
    auto t1 = Clock::now();
    std::vector<int64_t> nlog(Bz, 0);
    RoundIo io;
    io.eos = eos;
    io.n_eos = n_eos;
    if (override_tokens != nullptr && n_override > 0) {
        HAI_TRY(upload_ids(&d_gen_ov_, &gen_ov_cap_, override_tokens, B_ * n_override));
        io.ov = d_gen_ov_;
        io.n_ov = n_override;
    }
    HAI_TRY(upload_ids(&d_eos_, &eos_cap_, eos, n_eos));
    io.out = out;
    io.out_ld = max_new;
    io.stats = st.data();
    io.round_log = round_log;
    io.log_cap = round_log_cap;
    io.n_log = nlog.data();
    bool live = true;
    while (live) HAI_TRY(one_round(width, io, &live));
    const double decode_s = seconds_since(t1);
    for (size_t b = 0; b < Bz; ++b) {
        st[b].prefill_seconds = prefill_s;
        st[b].decode_seconds = decode_s;
        st[b].emitted = rs_[b].emitted;
        if (stats) stats[b] = st[b];
        n_out[b] = rs_[b].emitted;
    }
    return HAI_OK;
}

int Engine::set_prefill_rows(int64_t rows) {
    if (rows < 0 || rows > std::max(pchunk_cap_, tmax_))
        return fail(HAI_ERR_INVALID_ARGUMENT, "set_prefill_rows: above the prompt chunk the engine was created for (" +
                                                  std::to_string(pchunk_cap_) + " rows)");
    if (rows > tmax_) {
        if (!fast_prefill_buffers()) return fail(HAI_ERR_INVALID_ARGUMENT, "set_prefill_rows: the engine was created "
                                                                           "without fast-prefill buffers");
        pchunk_ = rows;
        fast_prefill_ = true;
    } else {
        pchunk_ = std::min<int64_t>(tmax_, kDeltaNetMaxT);
        fast_prefill_ = false;
    }
    return HAI_OK;
}

int Engine::set_draft_override(const int32_t* tokens, int64_t n) {
    if (n < 0) return fail(HAI_ERR_INVALID_ARGUMENT, "set_draft_override: negative length");
    if (tokens == nullptr || n == 0) {
        n_override_ = 0;
        return HAI_OK;
    }
    HAI_TRY(check_ids(tokens, B_ * n, "draft override"));
    if (n > n_override_ || d_override_ == nullptr) {
        HAI_TRY(sync());
        if (d_override_) HAI_TRY(hai_free(d_override_));
        d_override_ = nullptr;
        void* p = nullptr;
        HAI_TRY(hai_malloc(&p, static_cast<size_t>(B_ * n) * 8));
        d_override_ = static_cast<int64_t*>(p);
    }
    std::vector<int64_t> wide(static_cast<size_t>(B_ * n));
    for (size_t i = 0; i < wide.size(); ++i) wide[i] = tokens[i];
    HAI_TRY(hai_memcpy_h2d(d_override_, wide.data(), wide.size() * 8, stream_));
    n_override_ = n;
    return sync();  // wide lives on the host stack
}

int Engine::spec_rounds(int64_t rounds, int64_t width, int32_t* out, int64_t cap, int64_t* n_out,
                        hai_spec_stats* stats) {
    if (width < 1 || width > tmax_ - 1)
        return fail(HAI_ERR_INVALID_ARGUMENT, "spec_rounds: width must be in 1 .. max_verify_tokens - 1");
    for (const auto& r : rs_)
        if (out == nullptr || cap < r.max_new) return fail(HAI_ERR_INVALID_ARGUMENT, "spec_rounds: out capacity < max_new");
    const size_t Bz = static_cast<size_t>(B_);
    std::vector<hai_spec_stats> st(Bz, hai_spec_stats{});
    std::vector<int64_t> start(Bz);
    for (size_t b = 0; b < Bz; ++b) start[b] = rs_[b].emitted;
    RoundIo io;
    io.out = out;
    io.out_ld = cap;
    io.stats = st.data();
    if (n_override_ > 0) {
        io.ov = d_override_;
        io.n_ov = n_override_;
    }
    auto t0 = Clock::now();
    bool live = true;
    for (int64_t r = 0; r < rounds && live; ++r) HAI_TRY(one_round(width, io, &live));
    HAI_TRY(sync());
    const double dt = seconds_since(t0);
    hai_spec_stats sum{};
    for (size_t b = 0; b < Bz; ++b) {
        const auto& s = st[b];
        sum.rounds = std::max(sum.rounds, s.rounds);
        sum.proposed += s.proposed;
        sum.accepted += s.accepted;
        sum.rejected += s.rejected;
        sum.corrections += s.corrections;
        sum.replay_tokens += s.replay_tokens;
        sum.mtp_recovery_tokens += s.mtp_recovery_tokens;
        sum.max_proposal_width = std::max(sum.max_proposal_width, s.max_proposal_width);
        sum.host_syncs = std::max(sum.host_syncs, s.host_syncs);
        sum.emitted += rs_[b].emitted - start[b];
        if (n_out) n_out[b] = rs_[b].emitted;
    }
    sum.decode_seconds = dt;
    if (stats) {
        stats->rounds += sum.rounds;
        stats->proposed += sum.proposed;
        stats->accepted += sum.accepted;
        stats->rejected += sum.rejected;
        stats->corrections += sum.corrections;
        stats->replay_tokens += sum.replay_tokens;
        stats->mtp_recovery_tokens += sum.mtp_recovery_tokens;
        stats->max_proposal_width = std::max(stats->max_proposal_width, sum.max_proposal_width);
        stats->emitted += sum.emitted;
        stats->host_syncs += sum.host_syncs;
        stats->decode_seconds += dt;
    }
    return HAI_OK;
}

// Replays verify steps of T rows per sequence at the current committed
// context without committing them (the accept kernel runs on scratch
// lengths), timing the whole step with events and every GEMM launch
// individually.
int Engine::profile_verify(int64_t T, int64_t iters, hai_verify_profile* out) {
    if (T < 1 || T > tmax_ || iters < 1) return fail(HAI_ERR_INVALID_ARGUMENT, "profile_verify: T or iters");
    const auto& d = d_;
    void *e0 = nullptr, *e1 = nullptr;
    HAI_TRY(hai_event_create(&e0));
    HAI_TRY(hai_event_create(&e1));
    // scratch lengths: target [B], MTP [B], result [4B]; the real ones stay untouched
    int32_t* s_tlen = d_plen_;
    int32_t* s_mlen = d_plen_ + B_;
    int32_t* s_res = d_plen_ + 3 * B_;
    std::vector<int64_t> ids(static_cast<size_t>(B_ * T), 1);
    HAI_TRY(hai_memcpy_h2d(d_ids_, ids.data(), ids.size() * 8, stream_));
    double verify_ms = 0.0, gemm_ms = 0.0, draft_ms = 0.0;
    for (int64_t it = 0; it < iters + 1; ++it) {  // first iteration warms up and records the GEMMs
        prof_record_ = it == 0;
        if (prof_record_) prof_calls_.clear();
        HAI_TRY(hai_event_record(e0, stream_));
        HAI_TRY(forward_target(d_ids_, T, StateWrites::kRecord));
        HAI_TRY(hai_memcpy_d2d(s_tlen, d_tlen_, static_cast<size_t>(B_) * 4, stream_));
        HAI_TRY(hai_memcpy_d2d(s_mlen, d_mlen_, static_cast<size_t>(B_) * 4, stream_));
        HAI_TRY(hai_verify_argmax_accept_bf16(logits_, d.V, hf_, d.H, d_ids_, nullptr, B_, T, d_preds_, s_res,
                                              s_tlen, s_mlen, d_pnext_, nullptr, nullptr, argmax_scratch_,
                                              stream_));
        HAI_TRY(hai_event_record(e1, stream_));
        prof_record_ = false;
        HAI_TRY(sync());
        float ms = 0.0f;
        HAI_TRY(hai_event_elapsed_ms(e0, e1, &ms));
        if (it > 0) verify_ms += ms;
    }
    // The step's GEMM launches replayed back to back (same shapes, weights and
    // buffers; the outputs are scratch here), two events around each replay.
    double gemm_bytes = 0.0;
    for (const auto& c : prof_calls_) {
        // weights (+ the FP8 scale grid rows and scale map)
        gemm_bytes += static_cast<double>(c.N) * static_cast<double>(c.K) * (c.w.q ? 1.0 : 2.0);
        if (c.w.q) gemm_bytes += static_cast<double>((c.N + 127) / 128 * ((c.K + 127) / 128)) * 4.0 + c.N * 4.0;
    }
    for (int64_t it = 0; it < iters + 1; ++it) {
        HAI_TRY(hai_event_record(e0, stream_));
        for (const auto& c : prof_calls_) {
            if (c.nw != nullptr && c.w.q != nullptr)
                HAI_TRY(hai_gemm_rmsnorm_fp8_bf16(c.y, c.ldy, c.x, c.ldx, c.nw, cfg_.rms_eps, 1, c.xn, c.ldx, c.w.q,
                                                  c.w.s, c.w.map, c.M, c.N, c.K, c.epi | HAI_FP8_NO_SPECIAL_CODES,
                                                  c.res, c.ldres, stream_));
            else if (c.nw != nullptr)
                HAI_TRY(hai_gemm_rmsnorm_bf16(c.y, c.ldy, c.x, c.ldx, c.nw, cfg_.rms_eps, 1, c.xn, c.ldx, c.w.w,
                                              c.M, c.N, c.K, c.epi, c.res, c.ldres, stream_));
            else
                HAI_TRY(gemm(c.y, c.ldy, c.x, c.ldx, c.w, c.M, c.N, c.K, c.epi, c.res, c.ldres));
        }
        HAI_TRY(hai_event_record(e1, stream_));
        HAI_TRY(sync());
        float ms = 0.0f;
        HAI_TRY(hai_event_elapsed_ms(e0, e1, &ms));
        if (it > 0) gemm_ms += ms;
    }
    // one entry per GEMM call of the engine; a call of more than 16 rows is
    // several launches on the bit-exact kernels
    double launches = 0.0;
    for (const auto& c : prof_calls_)
        launches += use_mfma(c.M) ? static_cast<double>((c.M + 127) / 128) : static_cast<double>((c.M + 15) / 16);
    // Draft step timing (one MTP forward + lm_head + argmax per sequence)
    // without events inside, on scratch MTP lengths.
    for (int64_t it = 0; it < iters + 1; ++it) {
        HAI_TRY(hai_memcpy_d2d(s_mlen, d_mlen_, static_cast<size_t>(B_) * 4, stream_));
        HAI_TRY(hai_event_record(e0, stream_));
        HAI_TRY(mtp_draft_step(d_ids_, h_prev_, mh_[0], d_pnext_));
        HAI_TRY(hai_event_record(e1, stream_));
        HAI_TRY(hai_memcpy_d2d(d_mlen_, s_mlen, static_cast<size_t>(B_) * 4, stream_));
        HAI_TRY(sync());
        float ms = 0.0f;
        HAI_TRY(hai_event_elapsed_ms(e0, e1, &ms));
        if (it > 0) draft_ms += ms;
    }
    hai_event_destroy(e0);
    hai_event_destroy(e1);
    const double n = static_cast<double>(iters);
    out->verify_ms = verify_ms / n;
    out->gemm_ms = gemm_ms / n;
    out->gemm_bytes = gemm_bytes;
    out->gemm_launches = launches;
    // algorithmic bytes of one verify step: weights streamed + KV read +
    // DeltaNet state read and T states written, per sequence.
    int64_t n_attn = 0, n_dn = 0;
    for (const auto& L : layers_) (L.attn ? n_attn : n_dn) += 1;
    double kv = 0.0;
    for (const auto& r : rs_)
        kv += static_cast<double>(n_attn) * 2.0 * static_cast<double>(r.target_len + T) *
              static_cast<double>(d.kvw) * 2.0;
    const double state = static_cast<double>(B_) * static_cast<double>(n_dn) *
                         static_cast<double>(d.nv * d.dk * d.dv) * 4.0 * (1.0 + static_cast<double>(T));
    out->step_bytes = out->gemm_bytes + kv + state;
    out->draft_ms = draft_ms / n;
    out->draft_bytes = static_cast<double>(d.H) * 2 * d.H * 2.0 +
                       static_cast<double>(d.Nqkv + d.qw + 3 * d.F) * d.H * (fp8_ ? 1.0 : 2.0) +
                       static_cast<double>(d.V) * d.H * 2.0;
    return HAI_OK;
}

}  // namespace hybridai::mi355x
