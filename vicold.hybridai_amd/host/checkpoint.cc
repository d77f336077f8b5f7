// checkpoint.cc -- see checkpoint.h.
#include "checkpoint.h"

#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <limits>

#include "engine.h"
#include "hai_kernels.h"
#include "json.h"

namespace hybridai::mi355x {

namespace {

int fail(std::string* err, int code, const std::string& what) {
    if (err) *err = what;
    return code;
}

bool file_exists(const std::string& p) {
    struct stat st{};
    return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

bool dir_exists(const std::string& p) {
    struct stat st{};
    return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

int64_t file_size(const std::string& p) {
    struct stat st{};
    if (stat(p.c_str(), &st) != 0) return -1;
    return static_cast<int64_t>(st.st_size);
}

std::string join(const std::string& dir, const std::string& name) {
    if (dir.empty() || dir.back() == '/') return dir + name;
    return dir + "/" + name;
}

// safetensors dtype strings (safetensor_loader.cc:16-34)
bool parse_dtype(const std::string& s, StDType* t) {
    static const std::pair<const char*, StDType> kTable[] = {
        {"F32", StDType::F32},         {"F16", StDType::F16},           {"BF16", StDType::BF16},
        {"F8_E4M3", StDType::F8_E4M3}, {"F8_E4M3FN", StDType::F8_E4M3}, {"F8_E5M2", StDType::F8_E5M2},
        {"I8", StDType::I8},           {"I32", StDType::I32},           {"I64", StDType::I64},
        {"U8", StDType::U8},           {"BOOL", StDType::BOOL}};
    for (const auto& e : kTable)
        if (s == e.first) {
            *t = e.second;
            return true;
        }
    return false;
}

bool read_file(const std::string& path, std::string* out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    if (n < 0) return false;
    f.seekg(0, std::ios::beg);
    out->resize(static_cast<size_t>(n));
    if (n > 0) f.read(out->data(), n);
    return static_cast<bool>(f);
}

}  // namespace

size_t st_dtype_size(StDType t) {
    switch (t) {
        case StDType::F32: case StDType::I32: return 4;
        case StDType::F16: case StDType::BF16: return 2;
        case StDType::I64: return 8;
        default: return 1;
    }
}

const char* st_dtype_name(StDType t) {
    switch (t) {
        case StDType::F32: return "F32";
        case StDType::F16: return "F16";
        case StDType::BF16: return "BF16";
        case StDType::F8_E4M3: return "F8_E4M3";
        case StDType::F8_E5M2: return "F8_E5M2";
        case StDType::I8: return "I8";
        case StDType::I32: return "I32";
        case StDType::I64: return "I64";
        case StDType::U8: return "U8";
        case StDType::BOOL: return "BOOL";
    }
    return "?";
}

int64_t StTensor::numel() const {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0 || (d != 0 && n > std::numeric_limits<int64_t>::max() / d)) return -1;  // invalid / overflow
        n *= d;
    }
    return n;
}

int SafeTensors::parse_shard(const std::string& path, int shard, std::map<std::string, StTensor>* out,
                             std::string* err) {
    if (!file_exists(path)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Safetensors file does not exist: " + path);
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Failed to open safetensors file: " + path);
    unsigned char len_bytes[8];
    f.read(reinterpret_cast<char*>(len_bytes), 8);
    if (!f) return fail(err, HAI_ERR_INVALID_MODEL, "Safetensors file is missing its header length: " + path);
    uint64_t header_len = 0;
    for (int i = 0; i < 8; ++i) header_len |= static_cast<uint64_t>(len_bytes[i]) << (8 * i);
    const int64_t total = file_size(path);
    if (total < 8 || header_len > static_cast<uint64_t>(total - 8))
        return fail(err, HAI_ERR_INVALID_MODEL, "Safetensors header length exceeds file size: " + path);
    std::string header(static_cast<size_t>(header_len), '\0');
    if (header_len > 0) f.read(header.data(), static_cast<std::streamsize>(header_len));
    if (!f) return fail(err, HAI_ERR_INVALID_MODEL, "Failed to read safetensors header: " + path);
    Json meta;
    std::string jerr;
    if (!Json::parse(header, &meta, &jerr) || !meta.is_object())
        return fail(err, HAI_ERR_INVALID_MODEL, "Invalid safetensors JSON header (" + path + "): " + jerr);
    const uint64_t data_size = static_cast<uint64_t>(total) - 8 - header_len;
    for (const auto& [name, e] : meta.members()) {
        if (name == "__metadata__") continue;
        const Json* dt = e.find("dtype");
        const Json* sh = e.find("shape");
        const Json* off = e.find("data_offsets");
        if (!e.is_object() || dt == nullptr || sh == nullptr || off == nullptr || !dt->is_string() ||
            !sh->is_array() || !off->is_array())
            return fail(err, HAI_ERR_INVALID_MODEL, "Invalid tensor metadata for: " + name);
        StTensor t;
        t.shard = shard;
        if (!parse_dtype(dt->as_string(), &t.dtype))
            return fail(err, HAI_ERR_UNSUPPORTED_DTYPE, "Unsupported safetensors dtype: " + dt->as_string());
        for (const Json& d : sh->items()) {
            int64_t v = 0;
            if (!d.to_int64(&v)) return fail(err, HAI_ERR_INVALID_MODEL, "Invalid tensor fields for " + name);
            if (v < 0) return fail(err, HAI_ERR_INVALID_MODEL, "Negative tensor dimension for: " + name);
            t.shape.push_back(v);
        }
        if (off->items().size() != 2 || !off->items()[0].to_uint64(&t.begin) || !off->items()[1].to_uint64(&t.end) ||
            t.begin > t.end || t.end > data_size)
            return fail(err, HAI_ERR_INVALID_MODEL, "Invalid data offsets for tensor: " + name);
        const int64_t n = t.numel();
        if (n < 0 || static_cast<uint64_t>(n) > std::numeric_limits<uint64_t>::max() / 8 ||
            static_cast<uint64_t>(n) * st_dtype_size(t.dtype) != t.bytes())
            return fail(err, HAI_ERR_INVALID_MODEL, "Tensor byte size does not match shape for: " + name);
        (*out)[name] = std::move(t);
    }
    shard_data_[static_cast<size_t>(shard)] = 8 + header_len;
    return HAI_OK;
}

int SafeTensors::open(const std::string& path, std::string* err) {
    shard_path_.clear();
    shard_data_.clear();
    tensors_.clear();
    if (!dir_exists(path)) {
        shard_path_.push_back(path);
        shard_data_.push_back(0);
        return parse_shard(path, 0, &tensors_, err);
    }
    const std::string index = join(path, "model.safetensors.index.json");
    if (!file_exists(index)) {
        const std::string single = join(path, "model.safetensors");
        if (file_exists(single)) return open(single, err);
        return fail(err, HAI_ERR_FILE_NOT_FOUND, "Neither safetensors index nor model.safetensors exists: " + path);
    }
    std::string text, jerr;
    if (!read_file(index, &text)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Failed to open safetensors index: " + index);
    Json root;
    if (!Json::parse(text, &root, &jerr))
        return fail(err, HAI_ERR_INVALID_MODEL, "Invalid safetensors index JSON: " + jerr);
    const Json* map = root.find("weight_map");
    if (map == nullptr || !map->is_object())
        return fail(err, HAI_ERR_INVALID_MODEL, "Safetensors index has no valid weight_map");
    std::map<std::string, int> shard_ids;
    std::vector<std::map<std::string, StTensor>> shard_tensors;
    for (const auto& [name, file] : map->members()) {
        if (!file.is_string()) return fail(err, HAI_ERR_INVALID_MODEL, "Invalid shard name for tensor: " + name);
        auto it = shard_ids.find(file.as_string());
        if (it == shard_ids.end()) {
            const int id = static_cast<int>(shard_path_.size());
            shard_path_.push_back(join(path, file.as_string()));
            shard_data_.push_back(0);
            shard_tensors.emplace_back();
            const int rc = parse_shard(shard_path_.back(), id, &shard_tensors.back(), err);
            if (rc != HAI_OK) return rc;
            it = shard_ids.emplace(file.as_string(), id).first;
        }
        const auto& st = shard_tensors[static_cast<size_t>(it->second)];
        const auto t = st.find(name);
        if (t == st.end())
            return fail(err, HAI_ERR_INVALID_MODEL, "Tensor listed in index is missing from shard: " + name);
        tensors_[name] = t->second;
    }
    return HAI_OK;
}

const StTensor* SafeTensors::find(const std::string& name) const {
    const auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

std::vector<std::string> SafeTensors::names() const {
    std::vector<std::string> n;
    n.reserve(tensors_.size());
    for (const auto& kv : tensors_) n.push_back(kv.first);
    return n;
}

int SafeTensors::read(const StTensor& t, void* dst, std::string* err) const {
    if (t.shard < 0 || static_cast<size_t>(t.shard) >= shard_path_.size())
        return fail(err, HAI_ERR_INVALID_MODEL, "tensor from an unknown shard");
    const std::string& path = shard_path_[static_cast<size_t>(t.shard)];
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Failed to reopen safetensors file: " + path);
    f.seekg(static_cast<std::streamoff>(shard_data_[static_cast<size_t>(t.shard)] + t.begin));
    if (!f) return fail(err, HAI_ERR_INVALID_MODEL, "Failed to seek to tensor data in " + path);
    if (t.bytes() > 0) f.read(static_cast<char*>(dst), static_cast<std::streamsize>(t.bytes()));
    if (!f) return fail(err, HAI_ERR_INVALID_MODEL, "Failed to read tensor data from " + path);
    return HAI_OK;
}

// ---------------------------------------------------------------- config.json

int read_model_config(const std::string& dir, hai_model_config* cfg, std::vector<int64_t>* eos, std::string* err,
                      int64_t* max_positions) {
    const std::string path = join(dir, "config.json");
    if (!file_exists(path)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Qwen3 config does not exist: " + path);
    std::string text, jerr;
    if (!read_file(path, &text)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Failed to open Qwen3 config: " + path);
    Json root;
    if (!Json::parse(text, &root, &jerr) || !root.is_object())
        return fail(err, HAI_ERR_INVALID_MODEL, "Invalid Qwen3 config JSON: " + jerr);

    // the reference's defaults (qwen3_config.h:16-47)
    int64_t hidden = 5120, layers = 64, heads = 24, kv_heads = 4, head_dim = 256, rope_dim = 64, ffn = 17408,
            vocab = 248320, max_pos = 262144, lin_k = 16, lin_v = 48, lin_kd = 128, lin_vd = 128, conv = 4,
            interval = 4, mtp = 0, bos = -1, pad = -1;
    double theta = 10000000.0, eps = 1.0e-6;
    bool gate = true, use_cache = true, tie = false, mtp_dedicated = false;
    std::string gate_type = "swish", ssm_dtype = "float32";

    // text_config fields first, then the root's, field by field
    const Json* tc = root.find("text_config");
    if (tc != nullptr && !tc->is_object()) tc = nullptr;
    auto field = [&](const char* key) -> const Json* {
        if (tc != nullptr) {
            if (const Json* v = tc->find(key)) return v;
        }
        return root.find(key);
    };
    auto rd_i64 = [&](const char* key, int64_t* t) {
        const Json* v = field(key);
        int64_t x = 0;
        if (v != nullptr && v->to_int64(&x)) *t = x;
    };
    auto rd_f = [&](const char* key, double* t) {
        const Json* v = field(key);
        if (v != nullptr && v->is_number()) *t = v->to_double();
    };
    auto rd_b = [&](const char* key, bool* t) {
        const Json* v = field(key);
        if (v != nullptr && v->is_bool()) *t = v->as_bool();
    };
    auto rd_s = [&](const char* key, std::string* t) {
        const Json* v = field(key);
        if (v != nullptr && v->is_string()) *t = v->as_string();
    };
    rd_i64("hidden_size", &hidden);
    rd_i64("num_hidden_layers", &layers);
    rd_i64("num_attention_heads", &heads);
    rd_i64("num_key_value_heads", &kv_heads);
    rd_i64("head_dim", &head_dim);
    rd_i64("intermediate_size", &ffn);
    rd_i64("vocab_size", &vocab);
    rd_i64("max_position_embeddings", &max_pos);
    rd_f("rope_theta", &theta);
    rd_f("rms_norm_eps", &eps);
    rd_i64("linear_num_key_heads", &lin_k);
    rd_i64("linear_num_value_heads", &lin_v);
    rd_i64("linear_key_head_dim", &lin_kd);
    rd_i64("linear_value_head_dim", &lin_vd);
    rd_i64("linear_conv_kernel_dim", &conv);
    rd_i64("full_attention_interval", &interval);
    rd_b("attn_output_gate", &gate);
    rd_s("output_gate_type", &gate_type);
    rd_s("mamba_ssm_dtype", &ssm_dtype);
    rd_b("use_cache", &use_cache);
    rd_i64("bos_token_id", &bos);
    rd_i64("pad_token_id", &pad);
    rd_b("tie_word_embeddings", &tie);
    rd_i64("mtp_num_hidden_layers", &mtp);
    rd_b("mtp_use_dedicated_embeddings", &mtp_dedicated);
    if (mtp < 0 || mtp > std::numeric_limits<int32_t>::max())
        return fail(err, HAI_ERR_INVALID_MODEL, "mtp_num_hidden_layers must be non-negative");

    eos->clear();
    if (const Json* e = field("eos_token_id")) {
        int64_t id = 0;
        if (e->to_int64(&id)) {
            eos->push_back(id);
        } else if (e->is_array()) {
            for (const Json& x : e->items()) {
                if (!x.to_int64(&id))
                    return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 eos_token_id contains a non-integer value");
                eos->push_back(id);
            }
        } else if (!e->is_null()) {
            return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 eos_token_id must be an integer or array");
        }
    }
    // head_dim from hidden size and heads when absent; rope_theta and the
    // rotary fraction from rope_parameters when present
    if (field("head_dim") == nullptr && heads > 0) head_dim = hidden / heads;
    if (const Json* rp = field("rope_parameters"); rp != nullptr && rp->is_object()) {
        if (const Json* t = rp->find("rope_theta"); t != nullptr && t->is_number()) theta = t->to_double();
        if (const Json* f = rp->find("partial_rotary_factor"); f != nullptr && f->is_number())
            rope_dim = static_cast<int64_t>(static_cast<float>(head_dim) * static_cast<float>(f->to_double()));
    }
    // layer schedule: layer_types if present, else from the interval; it
    // must agree with (i + 1) % interval == 0 for full attention
    std::vector<bool> full;
    if (const Json* lt = field("layer_types")) {
        if (!lt->is_array()) return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 layer_types must be an array");
        for (size_t i = 0; i < lt->items().size(); ++i) {
            const Json& v = lt->items()[i];
            if (!v.is_string()) return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 layer_types contains a non-string value");
            if (v.as_string() == "linear_attention") full.push_back(false);
            else if (v.as_string() == "full_attention") full.push_back(true);
            else
                return fail(err, HAI_ERR_INVALID_MODEL,
                            "Unknown Qwen3 layer type at index " + std::to_string(i) + ": " + v.as_string());
        }
    } else if (interval > 0) {
        for (int64_t i = 0; i < layers; ++i) full.push_back((i + 1) % interval == 0);
    }
    const float theta_f = static_cast<float>(theta), eps_f = static_cast<float>(eps);
    if (hidden <= 0 || layers <= 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || rope_dim <= 0 || ffn <= 0 ||
        vocab <= 0 || max_pos <= 0 || !(theta_f > 0.0f) || !(eps_f > 0.0f) || lin_k <= 0 || lin_v <= 0 ||
        lin_kd <= 0 || lin_vd <= 0 || conv <= 0 || lin_v % lin_k != 0 || heads % kv_heads != 0 ||
        rope_dim > head_dim || rope_dim % 2 != 0 || interval <= 0 || full.size() != static_cast<size_t>(layers))
        return fail(err, HAI_ERR_INVALID_MODEL, "Invalid dimensions in Qwen3 config");
    for (int64_t i = 0; i < layers; ++i)
        if (full[static_cast<size_t>(i)] != ((i + 1) % interval == 0))
            return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 layer_types conflicts with full_attention_interval");
    if (!gate || gate_type != "swish" || ssm_dtype != "float32")
        return fail(err, HAI_ERR_INVALID_MODEL, "Unsupported Qwen3 attention gate or SSM state configuration");
    for (int64_t v : {hidden, layers, heads, kv_heads, head_dim, rope_dim, ffn, vocab, lin_k, lin_v, lin_kd, lin_vd,
                      conv, interval, mtp})
        if (v > std::numeric_limits<int32_t>::max())
            return fail(err, HAI_ERR_INVALID_MODEL, "Qwen3 config dimension beyond 32 bits");
    hai_model_config c{};
    c.hidden = static_cast<int32_t>(hidden);
    c.num_layers = static_cast<int32_t>(layers);
    c.full_attention_interval = static_cast<int32_t>(interval);
    c.num_q_heads = static_cast<int32_t>(heads);
    c.num_kv_heads = static_cast<int32_t>(kv_heads);
    c.head_dim = static_cast<int32_t>(head_dim);
    c.rope_dim = static_cast<int32_t>(rope_dim);
    c.lin_qk_heads = static_cast<int32_t>(lin_k);
    c.lin_v_heads = static_cast<int32_t>(lin_v);
    c.lin_k_dim = static_cast<int32_t>(lin_kd);
    c.lin_v_dim = static_cast<int32_t>(lin_vd);
    c.conv_kernel = static_cast<int32_t>(conv);
    c.ffn = static_cast<int32_t>(ffn);
    c.vocab = static_cast<int32_t>(vocab);
    c.mtp_layers = static_cast<int32_t>(mtp);
    c.rms_eps = eps_f;
    c.rope_theta = theta_f;
    *cfg = c;
    if (max_positions != nullptr) *max_positions = max_pos;
    return HAI_OK;
}

// ---------------------------------------------------------------- names

std::string checkpoint_name(uint32_t id) {
    const uint32_t slot = id / 64u, kind = id % 64u;
    if (slot == kSlotShared) {
        static const char* kShared[] = {"model.language_model.embed_tokens.weight", "model.language_model.norm.weight",
                                        "lm_head.weight"};
        return kind < 3 ? kShared[kind] : "";
    }
    if (slot == kSlotMtpShared) {
        static const char* kMtp[] = {"mtp.fc.weight", "mtp.norm.weight", "mtp.pre_fc_norm_embedding.weight",
                                     "mtp.pre_fc_norm_hidden.weight"};
        return kind < 4 ? kMtp[kind] : "";
    }
    std::string prefix;
    if (slot == kSlotMtpLayer0) prefix = "mtp.layers.0.";
    else if (slot >= kSlotLayer0 && slot < kSlotMtpLayer0)
        prefix = "model.language_model.layers." + std::to_string(slot - kSlotLayer0) + ".";
    else return "";
    static const char* kLayer[] = {
        "input_layernorm.weight",        "post_attention_layernorm.weight", "linear_attn.in_proj_qkv.weight",
        "linear_attn.in_proj_z.weight",  "linear_attn.in_proj_a.weight",    "linear_attn.in_proj_b.weight",
        "linear_attn.conv1d.weight",     "linear_attn.A_log",               "linear_attn.dt_bias",
        "linear_attn.norm.weight",       "linear_attn.out_proj.weight",     "self_attn.q_proj.weight",
        "self_attn.k_proj.weight",       "self_attn.v_proj.weight",         "self_attn.o_proj.weight",
        "self_attn.q_norm.weight",       "self_attn.k_norm.weight",         "mlp.gate_proj.weight",
        "mlp.up_proj.weight",            "mlp.down_proj.weight"};
    return kind < sizeof(kLayer) / sizeof(kLayer[0]) ? prefix + kLayer[kind] : "";
}

int detect_weight_format(const SafeTensors& st, const hai_model_config& cfg, int32_t* format, std::string* err) {
    int dense = 0, fp8 = 0;
    auto check = [&](const std::string& name) -> int {
        const StTensor* t = st.find(name);
        if (t == nullptr) return fail(err, HAI_ERR_INVALID_MODEL, "Missing Qwen weight: " + name);
        const std::string scale = name.substr(0, name.size() - 7) + ".weight_scale_inv";
        if (t->dtype == StDType::BF16) {
            ++dense;
        } else if (t->dtype == StDType::F8_E4M3 && st.find(scale) != nullptr) {
            ++fp8;
        } else {
            return fail(err, HAI_ERR_UNSUPPORTED_DTYPE,
                        "Expected dense BF16 or scaled FP8 Qwen weight: " + name + " (" + st_dtype_name(t->dtype) + ")");
        }
        return HAI_OK;
    };
    auto layer = [&](const std::string& prefix, bool attn) -> int {
        const char* lin[] = {"linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight",
                             "linear_attn.out_proj.weight"};
        const char* att[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                             "self_attn.o_proj.weight"};
        const char* mlp[] = {"mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"};
        if (attn) {
            for (const char* s : att)
                if (const int rc = check(prefix + s); rc != HAI_OK) return rc;
        } else {
            for (const char* s : lin)
                if (const int rc = check(prefix + s); rc != HAI_OK) return rc;
        }
        for (const char* s : mlp)
            if (const int rc = check(prefix + s); rc != HAI_OK) return rc;
        return HAI_OK;
    };
    for (int32_t i = 0; i < cfg.num_layers; ++i)
        if (const int rc = layer("model.language_model.layers." + std::to_string(i) + ".",
                                 (i + 1) % cfg.full_attention_interval == 0);
            rc != HAI_OK)
            return rc;
    if (cfg.mtp_layers > 0)
        if (const int rc = layer("mtp.layers.0.", true); rc != HAI_OK) return rc;
    if (dense > 0 && fp8 > 0)
        return fail(err, HAI_ERR_NOT_IMPLEMENTED,
                    "checkpoint mixes dense BF16 and FP8 Linears; this engine stores them all one way");
    // The other tensors (embedding, norms, conv, A_log, dt_bias, in_proj_a|b,
    // lm_head, the MTP fc) are stored as BF16, the dtype the reference's GPU
    // ops take them in (delta_net.cc:477-478 requires a_log and dt_bias in
    // the activations' dtype): BF16, or F32 whose every value is a bf16
    // number.  Small F32 tensors are checked here; the engine checks the
    // large ones as it loads them.
    auto dense_ok = [&](const std::string& name) -> int {
        const StTensor* t = st.find(name);
        if (t == nullptr || t->dtype == StDType::BF16) return HAI_OK;  // a missing one is the load's error
        if (t->dtype != StDType::F32)
            return fail(err, HAI_ERR_UNSUPPORTED_DTYPE,
                        "Qwen weight " + name + " is " + st_dtype_name(t->dtype) +
                            "; this engine stores it as BF16 (BF16, or F32 holding bf16 values)");
        if (t->numel() > (int64_t{1} << 20)) return HAI_OK;
        std::vector<float> f(static_cast<size_t>(t->numel()));
        if (const int rc = st.read(*t, f.data(), err); rc != HAI_OK) return rc;
        uint16_t bits = 0;
        for (float v : f)
            if (!exact_bf16(v, &bits))
                return fail(err, HAI_ERR_UNSUPPORTED_DTYPE,
                            "Qwen weight " + name + " is F32 with values that are not bf16 numbers; this engine "
                                                    "stores it as BF16");
        return HAI_OK;
    };
    static const uint32_t kLinearKinds[] = {2, 3, 10, 11, 12, 13, 14, 17, 18, 19};  // checked above
    std::vector<uint32_t> slots = {kSlotShared};
    for (int32_t i = 0; i < cfg.num_layers; ++i) slots.push_back(kSlotLayer0 + static_cast<uint32_t>(i));
    if (cfg.mtp_layers > 0) {
        slots.push_back(kSlotMtpShared);
        slots.push_back(kSlotMtpLayer0);
    }
    for (uint32_t slot : slots)
        for (uint32_t kind = 0; kind < 64; ++kind) {
            const bool layer = slot >= kSlotLayer0;
            if (layer && std::find(std::begin(kLinearKinds), std::end(kLinearKinds), kind) != std::end(kLinearKinds))
                continue;
            const std::string name = checkpoint_name(slot * 64u + kind);
            if (name.empty()) continue;
            if (const int rc = dense_ok(name); rc != HAI_OK) return rc;
        }
    *format = fp8 > 0 ? HAI_WEIGHTS_FP8_BLOCK128 : HAI_WEIGHTS_BF16;
    return HAI_OK;
}

bool exact_bf16(float v, uint16_t* bits) {
    uint32_t u = 0;
    std::memcpy(&u, &v, 4);
    if ((u & 0xFFFFu) != 0) return false;
    *bits = static_cast<uint16_t>(u >> 16);
    return true;
}

bool is_regular_file(const std::string& path) { return file_exists(path); }
bool read_whole_file(const std::string& path, std::string* out) { return read_file(path, out); }
std::string path_join(const std::string& dir, const std::string& name) { return join(dir, name); }

}  // namespace hybridai::mi355x
