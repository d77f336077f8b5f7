// oracle_model.cpp -- TEST INFRASTRUCTURE ONLY: synthetic Qwen3.5-style
// hybrid model and the reference's speculative MTP state machine, restated
// on the CPU for parity tests.
//
//   target forward      generator.cc:550-634 (qwen_reference.cc:108-258)
//   MTP forward         generator.cc:139-183
//   speculative loop    generator.cc:648-1028
//   cache semantics     attention.cc:19-92, delta_net.cc:19-100 (deep clones)
#include "oracle.h"
#include "oracle_numerics.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <vector>

using namespace orc;

namespace {

// ---- synthetic data ----------------------------------------------------
// A counter-based generator: splitmix64 of (seed, tensor id, element index),
// the four 16-bit fields summed (Irwin-Hall of order 4, mean 0 after
// centring, unit variance after the sqrt(3)/65536 scale), times std, then
// bf16 RNE.  Pure integer work plus one fp32 multiply, so every platform
// produces the same bits.
inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint32_t id) {
    return splitmix64(seed ^ (static_cast<uint64_t>(id) << 32));
}

inline float gen_value(uint64_t key, uint64_t index, float scale) {
    const uint64_t h = splitmix64(key + index);
    const int32_t s = static_cast<int32_t>((h & 0xffffu) + ((h >> 16) & 0xffffu) +
                                           ((h >> 32) & 0xffffu) + (h >> 48));
    return static_cast<float>(s - 131070) * scale;
}

inline float gen_scale(float std_dev) {
    return static_cast<float>(static_cast<double>(std_dev) * 1.7320508075688772 / 65536.0);
}

// Tensor ids: slot * 64 + kind.  Slot 0 = shared, 1 = MTP shared,
// 2 + i = target layer i, 1024 + j = MTP layer j.
enum Kind : uint32_t {
    kInputLN = 0, kPostLN = 1, kInQKV = 2, kInZ = 3, kInA = 4, kInB = 5,
    kConv = 6, kALog = 7, kDtBias = 8, kLinNorm = 9, kOutProj = 10,
    kQProj = 11, kKProj = 12, kVProj = 13, kOProj = 14, kQNorm = 15,
    kKNorm = 16, kGate = 17, kUp = 18, kDown = 19,
};
enum SharedKind : uint32_t { kEmbed = 0, kFinalNorm = 1, kLmHead = 2 };
enum MtpKind : uint32_t { kFc = 0, kMtpNorm = 1, kPreEmb = 2, kPreHid = 3 };

inline uint32_t tid(uint32_t slot, uint32_t kind) { return slot * 64u + kind; }

struct AttnCache {  // AttentionKVCache (attention.h:11-42)
    std::vector<float> k, v;
    int64_t len = 0, cap = 0;
};

struct Layer {
    bool attn = false;
    std::vector<float> in_ln, post_ln;
    std::vector<float> qkv, z, a, b, conv, a_log, dt_bias, lin_norm, out_proj;
    std::vector<float> q, k, v, o, q_norm, k_norm;
    std::vector<float> gate, up, down;
};

struct Model {
    orc_config c{};
    uint64_t seed = 0;
    float std_dev = 0.02f;
    std::vector<float> embed, final_norm, lm_head;
    std::vector<float> fc, mtp_norm, pre_emb, pre_hid;
    std::vector<Layer> layers, mtp;
    std::vector<std::pair<uint32_t, std::vector<float>*>> registry;
    // MTP cache left by the last orc_generate_speculative call (inspection
    // for the cache-protocol tests)
    mutable std::vector<AttnCache> last_mtp;
};

void fill(Model& m, std::vector<float>& dst, uint32_t id, int64_t n) {
    dst.resize(static_cast<size_t>(n));
    const uint64_t key = stream_key(m.seed, id);
    const float sc = gen_scale(m.std_dev);
    for (int64_t i = 0; i < n; ++i) dst[i] = bf(gen_value(key, static_cast<uint64_t>(i), sc));
    m.registry.emplace_back(id, &dst);
}

void build_layer(Model& m, Layer& L, uint32_t slot, bool attn) {
    const auto& c = m.c;
    const int64_t H = c.hidden;
    L.attn = attn;
    fill(m, L.in_ln, tid(slot, kInputLN), H);
    fill(m, L.post_ln, tid(slot, kPostLN), H);
    if (attn) {
        fill(m, L.q, tid(slot, kQProj), int64_t(c.num_q_heads) * 2 * c.head_dim * H);
        fill(m, L.k, tid(slot, kKProj), int64_t(c.num_kv_heads) * c.head_dim * H);
        fill(m, L.v, tid(slot, kVProj), int64_t(c.num_kv_heads) * c.head_dim * H);
        fill(m, L.o, tid(slot, kOProj), H * c.num_q_heads * c.head_dim);
        fill(m, L.q_norm, tid(slot, kQNorm), c.head_dim);
        fill(m, L.k_norm, tid(slot, kKNorm), c.head_dim);
    } else {
        const int64_t kw = int64_t(c.lin_qk_heads) * c.lin_k_dim;
        const int64_t vw = int64_t(c.lin_v_heads) * c.lin_v_dim;
        const int64_t C = 2 * kw + vw;
        fill(m, L.qkv, tid(slot, kInQKV), C * H);
        fill(m, L.z, tid(slot, kInZ), vw * H);
        fill(m, L.a, tid(slot, kInA), int64_t(c.lin_v_heads) * H);
        fill(m, L.b, tid(slot, kInB), int64_t(c.lin_v_heads) * H);
        fill(m, L.conv, tid(slot, kConv), C * c.conv_kernel);
        fill(m, L.a_log, tid(slot, kALog), c.lin_v_heads);
        fill(m, L.dt_bias, tid(slot, kDtBias), c.lin_v_heads);
        fill(m, L.lin_norm, tid(slot, kLinNorm), c.lin_v_dim);
        fill(m, L.out_proj, tid(slot, kOutProj), H * vw);
    }
    fill(m, L.gate, tid(slot, kGate), int64_t(c.ffn) * H);
    fill(m, L.up, tid(slot, kUp), int64_t(c.ffn) * H);
    fill(m, L.down, tid(slot, kDown), H * c.ffn);
}

// qwen3_config.cc:166-176: layer i is full attention iff (i+1) % interval == 0.
bool is_attention_layer(const orc_config& c, int64_t i) {
    return (i + 1) % c.full_attention_interval == 0;
}

// ---- caches (reference semantics: deep-copied on clone) -----------------
struct DeltaCache {  // DeltaNetCache (delta_net.h:11-55)
    std::vector<float> conv, state;
    int64_t len = 0;
    bool init = false;
};
struct Caches {
    std::vector<AttnCache> attn;
    std::vector<DeltaCache> delta;
};

std::vector<float> gemm(const std::vector<float>& x, const std::vector<float>& w,
                        int64_t M, int64_t N, int64_t K) {
    std::vector<float> y(static_cast<size_t>(M * N));
    orc_gemm(x.data(), w.data(), y.data(), M, N, K, 1);
    return y;
}

std::vector<float> rmsnorm(const Model& m, const std::vector<float>& x,
                           const std::vector<float>& w, int64_t rows) {
    std::vector<float> y(x.size());
    orc_rmsnorm(x.data(), w.data(), y.data(), rows, m.c.hidden, m.c.rms_eps, 1, 1);
    return y;
}

void residual(std::vector<float>& h, const std::vector<float>& d) {
    orc_add(h.data(), d.data(), h.data(), static_cast<int64_t>(h.size()), 1);
}

// GatedGQAAttention::forward_impl with a cache (attention.cc:301-599).
bool attention_layer(const Model& m, const Layer& L, const std::vector<float>& x,
                     int64_t T, AttnCache& cache, int64_t cap,
                     std::vector<float>& out) {
    const auto& c = m.c;
    const int64_t H = c.hidden, nq = c.num_q_heads, nkv = c.num_kv_heads,
                  D = c.head_dim;
    if (cache.cap == 0) {
        cache.cap = cap;
        cache.k.assign(static_cast<size_t>(cap * nkv * D), 0.0f);
        cache.v.assign(static_cast<size_t>(cap * nkv * D), 0.0f);
    }
    if (cache.len + T > cache.cap) return false;  // attention.cc:326-330
    std::vector<float> pq = gemm(x, L.q, T, nq * 2 * D, H);
    std::vector<float> pk = gemm(x, L.k, T, nkv * D, H);
    std::vector<float> pv = gemm(x, L.v, T, nkv * D, H);
    std::vector<float> qr(static_cast<size_t>(T * nq * D)), gt(qr.size());
    std::vector<float> kr(static_cast<size_t>(T * nkv * D));
    const int64_t pos0 = cache.len;
    orc_q_gate_rmsnorm_rope(pq.data(), L.q_norm.data(), qr.data(), gt.data(), T,
                            nq, D, c.rope_dim, pos0, c.rope_theta, c.rms_eps, 1, 1);
    orc_k_rmsnorm_rope(pk.data(), L.k_norm.data(), kr.data(), T, nkv, D,
                       c.rope_dim, pos0, c.rope_theta, c.rms_eps, 1);
    // append_kv_cache_kernel (hip_kernels.hip:295-308).
    std::memcpy(cache.k.data() + pos0 * nkv * D, kr.data(), kr.size() * 4);
    std::memcpy(cache.v.data() + pos0 * nkv * D, pv.data(), pv.size() * 4);
    const int64_t new_len = pos0 + T;
    std::vector<float> att(static_cast<size_t>(T * nq * D));
    orc_attention(qr.data(), gt.data(), cache.k.data(), cache.v.data(), att.data(),
                  T, new_len, nq, nkv, D, 1);
    cache.len = new_len;
    out = gemm(att, L.o, T, H, nq * D);
    return true;
}

// qwen_deltanet_reference (qwen_reference.cc:205-258).
void deltanet_layer(const Model& m, const Layer& L, const std::vector<float>& x,
                    int64_t T, DeltaCache& cache, std::vector<float>& out) {
    const auto& c = m.c;
    const int64_t H = c.hidden, nk = c.lin_qk_heads, nv = c.lin_v_heads,
                  dk = c.lin_k_dim, dv = c.lin_v_dim, Kc = c.conv_kernel;
    const int64_t kw = nk * dk, vw = nv * dv, C = 2 * kw + vw;
    if (!cache.init) {
        cache.conv.assign(static_cast<size_t>(C * (Kc - 1)), 0.0f);
        cache.state.assign(static_cast<size_t>(nv * dk * dv), 0.0f);
        cache.init = true;
    }
    std::vector<float> pqkv = gemm(x, L.qkv, T, C, H);
    std::vector<float> pz = gemm(x, L.z, T, vw, H);
    std::vector<float> pa = gemm(x, L.a, T, nv, H);
    std::vector<float> pb = gemm(x, L.b, T, nv, H);
    std::vector<float> q(static_cast<size_t>(T * kw)), k(q.size()),
        v(static_cast<size_t>(T * vw));
    orc_deltanet_conv(pqkv.data(), L.conv.data(), cache.conv.data(), q.data(),
                      k.data(), v.data(), T, nk, nv, dk, dv, Kc, 1);
    std::vector<float> rec(static_cast<size_t>(T * vw));
    orc_deltanet_recurrent(q.data(), k.data(), v.data(), pa.data(), pb.data(),
                           pz.data(), L.a_log.data(), L.dt_bias.data(),
                           L.lin_norm.data(), cache.state.data(), rec.data(), T,
                           nk, nv, dk, dv, c.rms_eps, 1);
    cache.len += T;
    out = gemm(rec, L.out_proj, T, H, vw);
}

// qwen_mlp_reference (qwen_reference.cc:146-175).
std::vector<float> mlp(const Model& m, const Layer& L, const std::vector<float>& x,
                       int64_t T) {
    const int64_t H = m.c.hidden, F = m.c.ffn;
    std::vector<float> g = gemm(x, L.gate, T, F, H);
    std::vector<float> u = gemm(x, L.up, T, F, H);
    std::vector<float> act(g.size());
    orc_silu_mul(g.data(), u.data(), act.data(), static_cast<int64_t>(g.size()), 1);
    return gemm(act, L.down, T, H, F);
}

std::vector<float> embed(const Model& m, const int32_t* ids, int64_t T) {
    const int64_t H = m.c.hidden;
    std::vector<float> out(static_cast<size_t>(T * H));
    std::vector<int64_t> ids64(ids, ids + T);
    orc_embedding(m.embed.data(), ids64.data(), out.data(), T, m.c.vocab, H);
    return out;
}

// target_forward lambda (generator.cc:550-634).
bool target_forward(const Model& m, const int32_t* ids, int64_t T, Caches& cs,
                    int64_t cap, std::vector<float>& hidden,
                    std::vector<float>& logits) {
    const int64_t H = m.c.hidden;
    std::vector<float> h = embed(m, ids, T);
    for (size_t li = 0; li < m.layers.size(); ++li) {
        const Layer& L = m.layers[li];
        std::vector<float> xn = rmsnorm(m, h, L.in_ln, T);
        std::vector<float> mixed;
        if (L.attn) {
            if (!attention_layer(m, L, xn, T, cs.attn[li], cap, mixed)) return false;
        } else {
            deltanet_layer(m, L, xn, T, cs.delta[li], mixed);
        }
        residual(h, mixed);
        xn = rmsnorm(m, h, L.post_ln, T);
        residual(h, mlp(m, L, xn, T));
    }
    hidden = rmsnorm(m, h, m.final_norm, T);
    logits = gemm(hidden, m.lm_head, T, m.c.vocab, H);
    return true;
}

// qwen_mtp_forward_reference (generator.cc:139-183) + concat_mtp_inputs
// (generator.cc:24-66).
bool mtp_forward(const Model& m, const std::vector<float>& emb,
                 const std::vector<float>& hid, int64_t rows,
                 std::vector<AttnCache>& caches, int64_t cap,
                 std::vector<float>& out) {
    const int64_t H = m.c.hidden;
    std::vector<float> en = rmsnorm(m, emb, m.pre_emb, rows);
    std::vector<float> hn = rmsnorm(m, hid, m.pre_hid, rows);
    std::vector<float> cat(static_cast<size_t>(rows * 2 * H));
    for (int64_t r = 0; r < rows; ++r) {
        std::memcpy(cat.data() + r * 2 * H, en.data() + r * H, H * 4);
        std::memcpy(cat.data() + r * 2 * H + H, hn.data() + r * H, H * 4);
    }
    std::vector<float> cur = gemm(cat, m.fc, rows, H, 2 * H);
    caches.resize(m.mtp.size());
    for (size_t j = 0; j < m.mtp.size(); ++j) {
        const Layer& L = m.mtp[j];
        std::vector<float> xn = rmsnorm(m, cur, L.in_ln, rows);
        std::vector<float> mixed;
        if (!attention_layer(m, L, xn, rows, caches[j], cap, mixed)) return false;
        residual(cur, mixed);
        xn = rmsnorm(m, cur, L.post_ln, rows);
        residual(cur, mlp(m, L, xn, rows));
    }
    out = rmsnorm(m, cur, m.mtp_norm, rows);
    return true;
}

int64_t argmax_row(const std::vector<float>& logits, int64_t row, int64_t V) {
    int64_t idx = 0;
    orc_argmax_rows(logits.data() + row * V, &idx, 1, V);
    return idx;
}

std::vector<float> row_of(const std::vector<float>& x, int64_t row, int64_t W) {
    return std::vector<float>(x.begin() + row * W, x.begin() + (row + 1) * W);
}

bool in_set(const int32_t* s, int64_t n, int64_t v) {
    for (int64_t i = 0; i < n; ++i) if (s[i] == v) return true;
    return false;
}

Caches fresh_caches(const Model& m) {
    Caches cs;
    cs.attn.resize(m.layers.size());
    cs.delta.resize(m.layers.size());
    return cs;
}


// Synthetic FP8 scales: U(0.5, 2)/448 from the top 24 bits of the stream.
void fp8_scales(uint64_t seed, uint32_t id, int64_t n, float* out) {
    const uint64_t key = stream_key(seed, id + (1u << 20));
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t h = splitmix64(key + static_cast<uint64_t>(i));
        const float u = static_cast<float>(static_cast<uint32_t>(h >> 40)) * 0x1p-24f;
        out[i] = (0.5f + 1.5f * u) / 448.0f;
    }
}

// One tensor [rows, cols] of the bf16 model -> decode(encode(w / s)) * s.
void quantize_tensor(const Model& m, std::vector<float>& w, uint32_t id, int64_t rows, int64_t cols) {
    const int64_t nbr = (rows + 127) / 128, nbc = (cols + 127) / 128;
    std::vector<float> s(static_cast<size_t>(nbr * nbc));
    fp8_scales(m.seed, id, nbr * nbc, s.data());
    std::vector<float> t(static_cast<size_t>(cols));
    std::vector<uint8_t> q(static_cast<size_t>(cols));
    for (int64_t r = 0; r < rows; ++r) {
        float* row = w.data() + r * cols;
        for (int64_t c = 0; c < cols; ++c) t[c] = row[c] / s[(r / 128) * nbc + c / 128];
        orc_fp8_encode_array(t.data(), q.data(), cols);
        for (int64_t c = 0; c < cols; ++c) row[c] = orc_fp8_decode(q[c]) * s[(r / 128) * nbc + c / 128];
    }
}

void quantize_layer(Model& m, Layer& L, uint32_t slot) {
    const auto& c = m.c;
    const int64_t H = c.hidden, F = c.ffn;
    if (L.attn) {
        const int64_t qw = int64_t(c.num_q_heads) * c.head_dim, kvw = int64_t(c.num_kv_heads) * c.head_dim;
        quantize_tensor(m, L.q, tid(slot, kQProj), 2 * qw, H);
        quantize_tensor(m, L.k, tid(slot, kKProj), kvw, H);
        quantize_tensor(m, L.v, tid(slot, kVProj), kvw, H);
        quantize_tensor(m, L.o, tid(slot, kOProj), H, qw);
    } else {
        const int64_t kw = int64_t(c.lin_qk_heads) * c.lin_k_dim, vw = int64_t(c.lin_v_heads) * c.lin_v_dim;
        quantize_tensor(m, L.qkv, tid(slot, kInQKV), 2 * kw + vw, H);
        quantize_tensor(m, L.z, tid(slot, kInZ), vw, H);
        quantize_tensor(m, L.out_proj, tid(slot, kOutProj), H, vw);
    }
    quantize_tensor(m, L.gate, tid(slot, kGate), F, H);
    quantize_tensor(m, L.up, tid(slot, kUp), F, H);
    quantize_tensor(m, L.down, tid(slot, kDown), H, F);
}

}  // namespace

extern "C" {

void orc_fp8_synthetic_scales(uint64_t seed, uint32_t tensor_id, int64_t n, float* out) {
    fp8_scales(seed, tensor_id, n, out);
}

int orc_model_quantize_fp8(void* model) {
    auto* m = static_cast<Model*>(model);
    if (m == nullptr) return 1;
    for (size_t i = 0; i < m->layers.size(); ++i) quantize_layer(*m, m->layers[i], 2 + static_cast<uint32_t>(i));
    for (size_t j = 0; j < m->mtp.size(); ++j) quantize_layer(*m, m->mtp[j], 1024 + static_cast<uint32_t>(j));
    return 0;
}

uint16_t orc_synthetic_weight_bits(uint64_t seed, uint32_t tensor_id,
                                   uint64_t index, float std_dev) {
    return bf16_bits(gen_value(stream_key(seed, tensor_id), index, gen_scale(std_dev)));
}

// Prompt ids: splitmix64 stream 0xFFFF of the seed, reduced mod vocab.
void orc_synthetic_prompt(uint64_t seed, int64_t n, int64_t vocab, int32_t* out) {
    const uint64_t key = stream_key(seed, 0xFFFFu);
    for (int64_t i = 0; i < n; ++i)
        out[i] = static_cast<int32_t>(splitmix64(key + static_cast<uint64_t>(i)) %
                                      static_cast<uint64_t>(vocab));
}

void* orc_model_create(const orc_config* cfg, uint64_t seed, float std_dev) {
    auto m = std::make_unique<Model>();
    m->c = *cfg;
    m->seed = seed;
    m->std_dev = std_dev;
    const int64_t H = cfg->hidden, V = cfg->vocab;
    m->layers.resize(static_cast<size_t>(cfg->num_layers));
    m->mtp.resize(static_cast<size_t>(cfg->mtp_layers));
    m->registry.reserve(64 * (m->layers.size() + m->mtp.size() + 2));
    fill(*m, m->embed, tid(0, kEmbed), V * H);
    fill(*m, m->final_norm, tid(0, kFinalNorm), H);
    fill(*m, m->lm_head, tid(0, kLmHead), V * H);
    fill(*m, m->fc, tid(1, kFc), H * 2 * H);
    fill(*m, m->mtp_norm, tid(1, kMtpNorm), H);
    fill(*m, m->pre_emb, tid(1, kPreEmb), H);
    fill(*m, m->pre_hid, tid(1, kPreHid), H);
    for (int64_t i = 0; i < cfg->num_layers; ++i)
        build_layer(*m, m->layers[i], static_cast<uint32_t>(2 + i),
                    is_attention_layer(*cfg, i));
    for (int64_t j = 0; j < cfg->mtp_layers; ++j)
        build_layer(*m, m->mtp[j], static_cast<uint32_t>(1024 + j), true);
    return m.release();
}

void orc_model_destroy(void* model) { delete static_cast<Model*>(model); }

int64_t orc_model_tensor(void* model, uint32_t tensor_id, float* out,
                         int64_t capacity) {
    const Model& m = *static_cast<Model*>(model);
    for (const auto& e : m.registry) {
        if (e.first != tensor_id) continue;
        const int64_t n = static_cast<int64_t>(e.second->size());
        if (out != nullptr) std::memcpy(out, e.second->data(), std::min(n, capacity) * 4);
        return n;
    }
    return -1;
}

int orc_forward(void* model, const int32_t* ids, int64_t T, float* hidden,
                float* logits) {
    const Model& m = *static_cast<Model*>(model);
    Caches cs = fresh_caches(m);
    std::vector<float> hid, lg;
    if (!target_forward(m, ids, T, cs, T, hid, lg)) return -1;
    if (hidden) std::memcpy(hidden, hid.data(), hid.size() * 4);
    if (logits) std::memcpy(logits, lg.data(), lg.size() * 4);
    return 0;
}

int orc_generate_greedy(void* model, const int32_t* prompt, int64_t P,
                        int64_t max_new, const int32_t* eos, int64_t n_eos,
                        int32_t* out_tokens) {
    const Model& m = *static_cast<Model*>(model);
    const int64_t cap = P + max_new, V = m.c.vocab;
    Caches cs = fresh_caches(m);
    std::vector<float> hid, lg;
    if (!target_forward(m, prompt, P, cs, cap, hid, lg)) return -1;
    int32_t next = static_cast<int32_t>(argmax_row(lg, P - 1, V));
    int64_t emitted = 0;
    while (true) {
        out_tokens[emitted++] = next;
        if (emitted >= max_new || in_set(eos, n_eos, next)) break;
        if (!target_forward(m, &next, 1, cs, cap, hid, lg)) return -1;
        next = static_cast<int32_t>(argmax_row(lg, 0, V));
    }
    return static_cast<int>(emitted);
}

// Generator::generate speculative branch (generator.cc:648-1028).
int orc_generate_speculative(void* model, const int32_t* prompt, int64_t P,
                             int64_t max_new, int64_t width,
                             const int32_t* eos, int64_t n_eos,
                             const int32_t* draft_override,
                             int64_t n_override, int32_t* out_tokens,
                             orc_spec_stats* stats, int32_t* round_log,
                             int64_t round_log_cap) {
    const Model& m = *static_cast<Model*>(model);
    const int64_t H = m.c.hidden, V = m.c.vocab;
    const int64_t cap = P + max_new;
    orc_spec_stats st{};
    Caches committed = fresh_caches(m);
    std::vector<AttnCache> mtp_cache;
    int64_t emitted = 0;
    auto emit = [&](int32_t t) { out_tokens[emitted++] = t; };

    // Prefill (generator.cc:648-664).
    std::vector<float> hid, lg;
    std::vector<int32_t> prompt_ids(prompt, prompt + P);
    if (!target_forward(m, prompt, P, committed, cap, hid, lg)) return -1;
    int32_t next = static_cast<int32_t>(argmax_row(lg, P - 1, V));
    std::vector<float> target_hidden = row_of(hid, P - 1, H);
    // MTP prompt prefill pairs emb(t_i) with the post-norm hidden of t_i
    // (unshifted, generator.cc:673-699).
    {
        std::vector<float> pe = embed(m, prompt, P), out;
        std::vector<AttnCache> fresh;
        if (!mtp_forward(m, pe, hid, P, fresh, cap, out)) return -1;
        mtp_cache.swap(fresh);
    }
    int64_t rounds_logged = 0;
    while (emitted < max_new) {
        const int64_t remaining = max_new - emitted;
        if (in_set(eos, n_eos, next) || remaining == 1) {
            emit(next);
            break;
        }
        const int64_t pc = std::min<int64_t>(width, remaining - 1);
        st.max_proposal_width = std::max(st.max_proposal_width, pc);
        ++st.rounds;
        std::vector<AttnCache> scratch = mtp_cache;           // clone
        std::vector<std::vector<AttnCache>> ckpt{mtp_cache};  // checkpoint[0]
        st.mtp_cache_clones += 2;
        std::vector<int32_t> cands;
        std::vector<float> ph = target_hidden;
        int32_t pin = next;
        for (int64_t i = 0; i < pc; ++i) {
            std::vector<float> e = embed(m, &pin, 1), mh;
            if (!mtp_forward(m, e, ph, 1, scratch, cap, mh)) return -1;
            std::vector<float> ml = gemm(mh, m.lm_head, 1, V, H);
            int32_t cand = static_cast<int32_t>(argmax_row(ml, 0, V));
            const int64_t pos = emitted + 1 + i;
            if (draft_override != nullptr && pos < n_override) cand = draft_override[pos];
            cands.push_back(cand);
            pin = cand;
            ph = mh;
            ++st.proposed;
            ckpt.push_back(scratch);
            ++st.mtp_cache_clones;
            if (in_set(eos, n_eos, cand)) break;
        }
        Caches verification = committed;  // clone_decoder_caches
        ++st.target_cache_clones;
        std::vector<int32_t> vids{next};
        vids.insert(vids.end(), cands.begin(), cands.end());
        std::vector<float> vh, vl;
        if (!target_forward(m, vids.data(), static_cast<int64_t>(vids.size()),
                            verification, cap, vh, vl)) return -1;
        std::vector<int64_t> preds(vids.size());
        orc_argmax_rows(vl.data(), preds.data(), static_cast<int64_t>(vids.size()), V);
        size_t acc = 0;
        while (acc < cands.size() && preds[acc] == cands[acc]) ++acc;
        int32_t* rec = nullptr;
        if (round_log != nullptr && rounds_logged < round_log_cap) {
            rec = round_log + rounds_logged * ORC_ROUND_RECORD;
            std::fill(rec, rec + ORC_ROUND_RECORD, -1);
            rec[0] = static_cast<int32_t>(cands.size());
            rec[1] = static_cast<int32_t>(acc);
            rec[4] = next;
            rec[5] = static_cast<int32_t>(emitted);
            for (size_t i = 0; i < cands.size() && i < 8; ++i) rec[8 + i] = cands[i];
            ++rounds_logged;
        }
        bool stop = false;
        if (acc == cands.size()) {
            committed = std::move(verification);
            mtp_cache = std::move(scratch);
            emit(next);
            for (int32_t cnd : cands) emit(cnd);
            st.accepted += static_cast<int64_t>(acc);
            next = static_cast<int32_t>(preds.back());
            target_hidden = row_of(vh, static_cast<int64_t>(vids.size()) - 1, H);
            if (rec) { rec[2] = 1; rec[3] = -1; }
        } else {
            const int32_t corr = static_cast<int32_t>(preds[acc]);
            st.rejected += static_cast<int64_t>(cands.size() - acc);
            ++st.corrections;
            std::vector<int32_t> rids{next};
            rids.insert(rids.end(), cands.begin(), cands.begin() + acc);
            rids.push_back(corr);
            std::vector<float> rh, rl;
            if (!target_forward(m, rids.data(), static_cast<int64_t>(rids.size()),
                                committed, cap, rh, rl)) return -1;
            st.replay_tokens += static_cast<int64_t>(rids.size());
            emit(next);
            for (size_t i = 0; i < acc; ++i) emit(cands[i]);
            if (emitted < max_new) emit(corr);
            st.accepted += static_cast<int64_t>(acc);
            if (rec) { rec[2] = 0; rec[3] = corr; }
            if (emitted >= max_new || in_set(eos, n_eos, corr)) {
                stop = true;
            } else {
                mtp_cache = ckpt[acc];
                std::vector<float> cih = row_of(rh, static_cast<int64_t>(rids.size()) - 2, H);
                std::vector<float> ce = embed(m, &corr, 1), rec_out;
                if (!mtp_forward(m, ce, cih, 1, mtp_cache, cap, rec_out)) return -1;
                ++st.mtp_recovery_tokens;
                next = static_cast<int32_t>(
                    argmax_row(rl, static_cast<int64_t>(rids.size()) - 1, V));
                target_hidden = row_of(rh, static_cast<int64_t>(rids.size()) - 1, H);
            }
        }
        if (rec) {
            rec[6] = mtp_cache.empty() ? 0 : static_cast<int32_t>(mtp_cache[0].len);
            rec[7] = committed.attn.empty() ? 0 : [&]() {
                for (const auto& a : committed.attn) if (a.cap) return static_cast<int32_t>(a.len);
                return static_cast<int32_t>(committed.delta[0].len);
            }();
        }
        if (stop) break;
        if (emitted >= max_new || (emitted > 0 && in_set(eos, n_eos, out_tokens[emitted - 1])))
            break;
    }
    if (stats) *stats = st;
    m.last_mtp = mtp_cache;
    return static_cast<int>(emitted);
}

int orc_model_set_tensor(void* model, uint32_t tensor_id, const float* data, int64_t n) {
    auto* m = static_cast<Model*>(model);
    if (m == nullptr || data == nullptr) return -1;
    for (auto& e : m->registry) {
        if (e.first != tensor_id) continue;
        if (static_cast<int64_t>(e.second->size()) != n) return -1;
        std::memcpy(e.second->data(), data, static_cast<size_t>(n) * 4);
        return 0;
    }
    return -1;
}

// qwen_mtp_forward_reference (generator.cc:139-183) on a fresh MTP cache of
// `rows` rows, as the MTP prompt prefill calls it (generator.cc:673-699):
// row r pairs emb(ids[r]) with hidden[r] at RoPE position r.
int orc_mtp_forward(void* model, const int32_t* ids, const float* hidden, int64_t rows, float* out,
                    float* k_cache, float* v_cache) {
    const Model& m = *static_cast<Model*>(model);
    if (rows <= 0 || m.mtp.empty()) return -1;
    const int64_t H = m.c.hidden;
    std::vector<float> e = embed(m, ids, rows), h(hidden, hidden + rows * H), o;
    std::vector<AttnCache> caches;
    if (!mtp_forward(m, e, h, rows, caches, rows, o)) return -1;
    if (out) std::memcpy(out, o.data(), o.size() * 4);
    const size_t kv = static_cast<size_t>(rows) * m.c.num_kv_heads * m.c.head_dim;
    if (k_cache) std::memcpy(k_cache, caches[0].k.data(), kv * 4);
    if (v_cache) std::memcpy(v_cache, caches[0].v.data(), kv * 4);
    return 0;
}

int64_t orc_last_mtp_cache(void* model, float* k, float* v, int64_t cap_rows) {
    const Model& m = *static_cast<Model*>(model);
    if (m.last_mtp.empty()) return 0;
    const AttnCache& c = m.last_mtp[0];
    const int64_t row = static_cast<int64_t>(m.c.num_kv_heads) * m.c.head_dim;
    const int64_t n = std::min(c.len, cap_rows);
    if (k) std::memcpy(k, c.k.data(), static_cast<size_t>(n * row) * 4);
    if (v) std::memcpy(v, c.v.data(), static_cast<size_t>(n * row) * 4);
    return c.len;
}

}  // extern "C"
