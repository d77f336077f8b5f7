// generator.cc -- hybridai::Generator (include/hybrid.h:96-113) on the
// MI355X verify engine: load_model() builds the engine, generate() runs the
// greedy or the MTP speculative decode (GenerationOptions::
// enable_speculative_mtp, generator.cc:545-1117) entirely on the device and
// fills GenerationResult's counters (hybrid.h:65-94).
//
// What this build accepts:
//   * GeneratorOptions::model_dir = a Qwen checkpoint directory
//     (config.json, model.safetensors or its sharded index, tokenizer.json,
//     optionally generation_config.json), loaded as Impl::load does
//     (generator.cc:390-431): prompts are text, wrapped in the chat layout
//     when GenerationOptions::use_chat_template, encoded by the checkpoint's
//     tokenizer; the stop ids are the config's and the generation config's;
//     result.text is the decoded continuation without special tokens;
//   * or model_dir =
//     "synthetic:<tiny|27b>[?seed=S&std=X&context=C&weights=bf16|fp8]"
//     -- the counter-based synthetic weights shared with the CPU oracle
//     (tiny = BASELINE config C1, 27b = the 27B shape of C3; weights=fp8 the
//     C5 format: QuantizedWeight Linears as E4M3 with 128x128 block scales).
//     These have no tokenizer: GenerationOptions::prompt = "ids:1,2,3" gives
//     token ids, result.text holds the generated ids in the same form, and
//     there is no EOS;
//   * GeneratorOptions::backend = "hip" (or "mi355x");
//   * the speculative proposal width is HYBRIDAI_SPECULATIVE_WIDTH (1..16,
//     default 8), read at every generate() as the reference does.
#include <sys/stat.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <sstream>

#include "checkpoint.h"
#include "engine.h"
#include "hai_kernels.h"
#include "refabi/hybrid_api.h"
#include "tokenizer.h"

namespace hybridai {

ApiStatus::ApiStatus(ApiStatusCode code, std::string message) : code_(code), message_(std::move(message)) {}
bool ApiStatus::ok() const noexcept { return code_ == ApiStatusCode::OK; }
ApiStatusCode ApiStatus::code() const noexcept { return code_; }
const std::string& ApiStatus::message() const noexcept { return message_; }

namespace {

hai_model_config tiny_config() {
    hai_model_config c{};
    c.hidden = 256; c.num_layers = 4; c.full_attention_interval = 4; c.num_q_heads = 4; c.num_kv_heads = 2;
    c.head_dim = 64; c.rope_dim = 16; c.lin_qk_heads = 4; c.lin_v_heads = 4; c.lin_k_dim = 64; c.lin_v_dim = 64;
    c.conv_kernel = 4; c.ffn = 768; c.vocab = 4096; c.mtp_layers = 1; c.rms_eps = 1e-6f; c.rope_theta = 1e7f;
    return c;
}

hai_model_config qwen27b_config() {
    hai_model_config c{};
    c.hidden = 5120; c.num_layers = 64; c.full_attention_interval = 4; c.num_q_heads = 24; c.num_kv_heads = 4;
    c.head_dim = 256; c.rope_dim = 64; c.lin_qk_heads = 16; c.lin_v_heads = 48; c.lin_k_dim = 128;
    c.lin_v_dim = 128; c.conv_kernel = 4; c.ffn = 17408; c.vocab = 248320; c.mtp_layers = 1; c.rms_eps = 1e-6f;
    c.rope_theta = 1e7f;
    return c;
}

ApiStatusCode api_code(int hai_rc) {
    switch (hai_rc) {
        case HAI_ERR_INVALID_ARGUMENT: return ApiStatusCode::InvalidArgument;
        case HAI_ERR_OUT_OF_MEMORY: return ApiStatusCode::OutOfMemory;
        case HAI_ERR_NOT_IMPLEMENTED: return ApiStatusCode::NotImplemented;
        case HAI_ERR_INVALID_DEVICE: return ApiStatusCode::InvalidDevice;
        case HAI_ERR_UNSUPPORTED_DTYPE: return ApiStatusCode::InvalidModel;  // no such ApiStatusCode
        case HAI_ERR_FILE_NOT_FOUND: return ApiStatusCode::FileNotFound;
        case HAI_ERR_INVALID_MODEL: return ApiStatusCode::InvalidModel;
        default: return ApiStatusCode::BackendError;
    }
}

// "ids:1,2,3" (commas and/or spaces) -> ids; false on anything else.
bool parse_ids(const std::string& text, std::vector<int32_t>* ids) {
    if (text.rfind("ids:", 0) != 0) return false;
    std::string body = text.substr(4);
    std::replace(body.begin(), body.end(), ',', ' ');
    std::istringstream in(body);
    long long v;
    while (in >> v) {
        if (v < 0 || v > INT32_MAX) return false;
        ids->push_back(static_cast<int32_t>(v));
    }
    return in.eof() && !ids->empty();
}

// speculative_proposal_width (generator.cc:124-137): the MTP proposal width
// comes from HYBRIDAI_SPECULATIVE_WIDTH, a decimal in 1..16; unset, empty or
// anything else gives the default of 8.
int64_t speculative_width_from_env() {
    constexpr int64_t kDefault = 8, kMax = 16;
    const char* v = std::getenv("HYBRIDAI_SPECULATIVE_WIDTH");
    if (v == nullptr || v[0] == '\0') return kDefault;
    char* end = nullptr;
    const unsigned long n = std::strtoul(v, &end, 10);
    if (end == v || *end != '\0' || n == 0 || n > static_cast<unsigned long>(kMax)) return kDefault;
    return static_cast<int64_t>(n);
}

// Positions a checkpoint engine accepts (prompt + max_new_tokens):
// max_position_embeddings, the bound of generator.cc:481-485, unless
// HYBRIDAI_MAX_CONTEXT (a positive integer) caps it to bound the KV memory
// (64 KiB per position at the 27B shape).  0: not set or not a number.
int64_t max_context_from_env() {
    const char* v = std::getenv("HYBRIDAI_MAX_CONTEXT");
    if (v == nullptr || v[0] == '\0') return 0;
    char* end = nullptr;
    const long long n = std::strtoll(v, &end, 10);
    if (end == v || *end != '\0' || n <= 0) return 0;
    return static_cast<int64_t>(n);
}

}  // namespace

class Generator::Impl {
public:
    explicit Impl(GeneratorOptions options) : options_(std::move(options)) {}

    ApiStatus load() {
        if (options_.backend != "hip" && options_.backend != "mi355x")
            return {ApiStatusCode::NotImplemented,
                    "this library provides the MI355X (\"hip\") backend only, not \"" + options_.backend + "\""};
        const std::string& dir = options_.model_dir;
        if (dir.empty()) return {ApiStatusCode::InvalidArgument, "model_dir is empty"};
        tokenizer_ = mi355x::QwenTokenizer();
        if (dir.rfind("synthetic:", 0) != 0) return load_checkpoint_dir(dir);
        std::string spec = dir.substr(10), query;
        if (const auto q = spec.find('?'); q != std::string::npos) {
            query = spec.substr(q + 1);
            spec = spec.substr(0, q);
        }
        if (spec == "tiny") cfg_ = tiny_config();
        else if (spec == "27b") cfg_ = qwen27b_config();
        else return {ApiStatusCode::InvalidModel, "unknown synthetic model \"" + spec + "\" (tiny or 27b)"};
        uint64_t seed = 0;
        float std_dev = 0.02f;
        int32_t context = 4096;
        int32_t weight_format = HAI_WEIGHTS_BF16;
        std::istringstream qs(query);
        for (std::string kv; std::getline(qs, kv, '&');) {
            const auto eq = kv.find('=');
            if (eq == std::string::npos) continue;
            const std::string key = kv.substr(0, eq), val = kv.substr(eq + 1);
            if (key == "seed") seed = std::strtoull(val.c_str(), nullptr, 10);
            else if (key == "std") std_dev = std::strtof(val.c_str(), nullptr);
            else if (key == "context") context = static_cast<int32_t>(std::strtol(val.c_str(), nullptr, 10));
            else if (key == "weights" && (val == "bf16" || val == "fp8"))
                weight_format = val == "fp8" ? HAI_WEIGHTS_FP8_BLOCK128 : HAI_WEIGHTS_BF16;
            else return {ApiStatusCode::InvalidArgument, "unknown model option \"" + kv + "\""};
        }
        hai_engine_options eo{};
        eo.max_context = context;
        eo.max_verify_tokens = static_cast<int32_t>(mi355x::kMaxVerifyRows);  // any width the env var allows
        eo.device = 0;
        eo.use_graphs = 0;
        eo.weight_format = weight_format;
        engine_ = std::make_unique<mi355x::Engine>(cfg_, eo);
        if (!engine_->ok()) {
            const std::string why = engine_->error();
            engine_.reset();
            return {ApiStatusCode::BackendError, "engine creation failed: " + why};
        }
        if (const int rc = engine_->init_synthetic(seed, std_dev); rc != HAI_OK) {
            const std::string why = engine_->error();
            engine_.reset();
            return {api_code(rc), "synthetic weights: " + why};
        }
        context_ = context;
        position_limit_ = 0;
        limit_capped_ = false;
        return {};
    }

    // generator.cc:390-431 for a Qwen checkpoint directory: config.json,
    // the weights (the MTP layer's when enable_mtp), the EOS ids of the
    // config; the engine holds max_position_embeddings positions (or
    // HYBRIDAI_MAX_CONTEXT, when that is smaller) plus the verify rows.
    ApiStatus load_checkpoint_dir(const std::string& dir) {
        struct stat sb{};
        if (dir.empty() || stat(dir.c_str(), &sb) != 0 || !S_ISDIR(sb.st_mode))
            return {ApiStatusCode::FileNotFound, "model directory does not exist: " + dir};
        std::string err;
        std::vector<int64_t> eos;
        int64_t max_pos = 0;
        int rc = mi355x::read_model_config(dir, &cfg_, &eos, &err, &max_pos);
        if (rc != HAI_OK) return {api_code(rc), err};
        mi355x::SafeTensors st;
        rc = st.open(dir, &err);
        int32_t fmt = HAI_WEIGHTS_BF16;
        if (rc == HAI_OK) rc = mi355x::detect_weight_format(st, cfg_, &fmt, &err);
        if (rc != HAI_OK) return {api_code(rc), err};
        if (options_.enable_mtp && cfg_.mtp_layers <= 0)
            return {ApiStatusCode::InvalidModel, "Checkpoint does not contain Qwen MTP layers"};
        if (cfg_.mtp_layers > 1)
            return {ApiStatusCode::NotImplemented, "checkpoints with more than one MTP layer are not supported"};
        const int64_t env_cap = max_context_from_env();
        const int64_t limit = env_cap > 0 ? std::min(max_pos, env_cap) : max_pos;
        if (limit <= 0 || limit > INT32_MAX - mi355x::kMaxVerifyRows)
            return {ApiStatusCode::InvalidModel, "max_position_embeddings out of range"};
        hai_engine_options eo{};
        eo.max_context = static_cast<int32_t>(limit + mi355x::kMaxVerifyRows);
        eo.max_verify_tokens = static_cast<int32_t>(mi355x::kMaxVerifyRows);
        eo.device = 0;
        eo.use_graphs = 0;
        eo.weight_format = fmt;
        engine_ = std::make_unique<mi355x::Engine>(cfg_, eo);
        if (!engine_->ok()) {
            const std::string why = engine_->error();
            engine_.reset();
            return {ApiStatusCode::BackendError, "engine creation failed: " + why};
        }
        if (rc = engine_->load_checkpoint(st, options_.enable_mtp); rc != HAI_OK) {
            const std::string why = engine_->error();
            engine_.reset();
            return {api_code(rc), why};
        }
        // QwenTokenizer::load after the weights (generator.cc:423-424)
        if (rc = tokenizer_.load(dir, &err); rc != HAI_OK) {
            engine_.reset();
            return {ApiStatusCode::InvalidModel, err};
        }
        // stop ids: the config's and the generation config's (generator.cc:476-480)
        eos.insert(eos.end(), tokenizer_.eos_token_ids().begin(), tokenizer_.eos_token_ids().end());
        eos_.clear();
        for (int64_t id : eos)
            if (id >= 0 && id < cfg_.vocab) eos_.push_back(static_cast<int32_t>(id));
        std::sort(eos_.begin(), eos_.end());
        eos_.erase(std::unique(eos_.begin(), eos_.end()), eos_.end());
        context_ = eo.max_context;
        position_limit_ = limit;
        limit_capped_ = limit < max_pos;
        mtp_loaded_ = options_.enable_mtp;
        return {};
    }

    ApiStatus generate(const GenerationOptions& o, GenerationResult* result) {
        // argument checks in the order of generator.cc:452-465
        if (result == nullptr) return {ApiStatusCode::InvalidArgument, "result must not be null"};
        if (!engine_) return {ApiStatusCode::InvalidModel, "load_model() has not succeeded"};
        if (o.prompt.empty() || o.max_new_tokens <= 0)
            return {ApiStatusCode::InvalidArgument, "prompt must be non-empty and max_new_tokens must be positive"};
        if (o.enable_speculative_mtp && !mtp_loaded_)
            return {ApiStatusCode::InvalidArgument, "speculative MTP requires GeneratorOptions::enable_mtp"};
        std::vector<int32_t> prompt;
        if (tokenizer_.loaded()) {
            // chat layout and encode (generator.cc:468-474)
            const std::string text =
                o.use_chat_template ? mi355x::QwenTokenizer::chat_prompt({{"user", o.prompt}}, true, o.enable_thinking)
                                    : o.prompt;
            for (int64_t id : tokenizer_.encode(text)) {
                if (id < 0 || id >= cfg_.vocab)
                    return {ApiStatusCode::InvalidArgument, "prompt token id outside the model's vocabulary"};
                prompt.push_back(static_cast<int32_t>(id));
            }
            if (prompt.empty()) return {ApiStatusCode::InvalidArgument, "the prompt encodes to no tokens"};
        } else if (!parse_ids(o.prompt, &prompt)) {
            return {ApiStatusCode::InvalidArgument, "a model without a tokenizer takes the prompt as \"ids:1,2,3\""};
        }
        for (int32_t id : prompt)
            if (id >= cfg_.vocab) return {ApiStatusCode::InvalidArgument, "prompt id outside the vocabulary"};
        const int64_t positions = static_cast<int64_t>(prompt.size()) + o.max_new_tokens;
        if (position_limit_ > 0) {
            // a checkpoint: the reference's bound and message (generator.cc:481-485)
            if (positions > position_limit_)
                return {ApiStatusCode::InvalidArgument,
                        limit_capped_ ? "prompt + max_new_tokens exceed HYBRIDAI_MAX_CONTEXT (" +
                                            std::to_string(position_limit_) + " positions)"
                                      : std::string("prompt exceeds model context")};
        } else if (positions + mi355x::kMaxVerifyRows > context_) {
            return {ApiStatusCode::InvalidArgument, "prompt + max_new_tokens exceed the model context"};
        }
        *result = GenerationResult{};
        std::vector<int32_t> out(static_cast<size_t>(std::max(1, o.max_new_tokens)));
        int64_t n = 0;
        hai_spec_stats st{};
        const auto t0 = std::chrono::steady_clock::now();
        int rc;
        if (o.enable_speculative_mtp) {
            rc = engine_->generate_speculative(prompt.data(), static_cast<int64_t>(prompt.size()), o.max_new_tokens,
                                               speculative_width_from_env(), eos_.data(),
                                               static_cast<int64_t>(eos_.size()), nullptr, 0, out.data(), &st,
                                               nullptr, 0, &n);
        } else {
            rc = engine_->generate_greedy(prompt.data(), static_cast<int64_t>(prompt.size()), o.max_new_tokens,
                                          eos_.data(), static_cast<int64_t>(eos_.size()), out.data(), &n);
        }
        if (rc != HAI_OK) return {api_code(rc), "generation failed: " + engine_->error()};
        result->elapsed_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        result->token_ids.assign(out.begin(), out.begin() + n);
        if (tokenizer_.loaded()) {
            // decode without special tokens (generator.cc:1032, 1275)
            result->text = tokenizer_.decode(result->token_ids.data(), result->token_ids.size(), true);
        } else {
            std::ostringstream text;
            text << "ids:";
            for (int64_t i = 0; i < n; ++i) text << (i ? "," : "") << out[static_cast<size_t>(i)];
            result->text = text.str();
        }
        result->prompt_tokens = static_cast<int64_t>(prompt.size());
        if (o.enable_speculative_mtp) {
            result->prefill_seconds = st.prefill_seconds;
            result->time_to_first_token_seconds = st.prefill_seconds;
            result->decode_seconds = st.decode_seconds;
            result->mtp_proposed_tokens = st.proposed;
            result->mtp_accepted_tokens = st.accepted;
            result->mtp_acceptance_rate =
                st.proposed > 0 ? static_cast<double>(st.accepted) / static_cast<double>(st.proposed) : 0.0;
            result->speculative_proposal_seconds = st.draft_seconds;
            result->speculative_verification_seconds = st.verify_seconds;
            result->speculative_replay_seconds = st.correction_seconds;
            result->speculative_rounds = st.rounds;
            result->mtp_rejected_tokens = st.rejected;
            result->mtp_correction_tokens = st.corrections;
            result->speculative_replay_tokens = st.replay_tokens;
            result->speculative_mtp_recovery_tokens = st.mtp_recovery_tokens;
            result->speculative_max_proposal_width = st.max_proposal_width;
            // rollback is by committed length: no cache is ever cloned
        } else {
            result->decode_seconds = result->elapsed_seconds;
        }
        if (result->decode_seconds > 0.0)
            result->decode_tokens_per_second = static_cast<double>(n) / result->decode_seconds;
        return {};
    }

    ApiStatus reset() {
        // Every generate() starts from empty caches; the weights stay resident.
        return {};
    }

private:
    GeneratorOptions options_;
    hai_model_config cfg_{};
    int32_t context_ = 0;
    int64_t position_limit_ = 0;  // checkpoints: prompt + max_new_tokens bound (0 for synthetic models)
    bool limit_capped_ = false;   // position_limit_ comes from HYBRIDAI_MAX_CONTEXT
    bool mtp_loaded_ = true;     // synthetic models always carry their MTP layer
    std::vector<int32_t> eos_;   // the checkpoint's stop ids (config and generation config)
    mi355x::QwenTokenizer tokenizer_;  // loaded for checkpoint directories only
    std::unique_ptr<mi355x::Engine> engine_;
};

Generator::Generator(GeneratorOptions options) : impl_(std::make_unique<Impl>(std::move(options))) {}
Generator::~Generator() = default;
Generator::Generator(Generator&&) noexcept = default;
Generator& Generator::operator=(Generator&&) noexcept = default;
ApiStatus Generator::load_model() { return impl_->load(); }
ApiStatus Generator::reset() { return impl_->reset(); }
ApiStatus Generator::generate(const GenerationOptions& options, GenerationResult* result) {
    return impl_->generate(options, result);
}

}  // namespace hybridai
