// capi.cc -- extern "C" surface of the verify engine (include/hai_engine.h).
#include <new>
#include <string>

#include <algorithm>
#include <cstring>
#include <vector>

#include "checkpoint.h"
#include "engine.h"
#include "hai_kernels.h"
#include "hai_tokenizer.h"
#include "tokenizer.h"

using hybridai::mi355x::Engine;

namespace {
thread_local std::string g_create_error;
Engine* as_engine(void* e) { return static_cast<Engine*>(e); }
}  // namespace

extern "C" {

void* hai_engine_create(const hai_model_config* cfg, const hai_engine_options* opt) {
    if (cfg == nullptr || opt == nullptr) {
        g_create_error = "null config";
        return nullptr;
    }
    auto* e = new (std::nothrow) Engine(*cfg, *opt);
    if (e == nullptr) {
        g_create_error = "out of host memory";
        return nullptr;
    }
    if (!e->ok()) {
        g_create_error = e->error();
        delete e;
        return nullptr;
    }
    return e;
}

void hai_engine_destroy(void* engine) { delete as_engine(engine); }

const char* hai_engine_last_error(void* engine) {
    return engine ? as_engine(engine)->error().c_str() : g_create_error.c_str();
}

int hai_engine_init_synthetic(void* engine, uint64_t seed, float std_dev) {
    if (!engine) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->init_synthetic(seed, std_dev);
}

int hai_model_config_load(const char* dir, hai_model_config* cfg, int64_t* eos_ids, int64_t eos_capacity,
                          int64_t* n_eos, int32_t* weight_format, char* message, int64_t message_capacity) {
    auto report = [&](int rc, const std::string& what) {
        if (message != nullptr && message_capacity > 0) {
            const size_t n = std::min(what.size(), static_cast<size_t>(message_capacity - 1));
            std::memcpy(message, what.data(), n);
            message[n] = '\0';
        }
        return rc;
    };
    if (dir == nullptr || cfg == nullptr) return report(HAI_ERR_INVALID_ARGUMENT, "null argument");
    std::string err;
    std::vector<int64_t> eos;
    hai_model_config c{};
    if (const int rc = hybridai::mi355x::read_model_config(dir, &c, &eos, &err); rc != HAI_OK) return report(rc, err);
    if (weight_format != nullptr) {
        hybridai::mi355x::SafeTensors st;
        if (const int rc = st.open(dir, &err); rc != HAI_OK) return report(rc, err);
        if (const int rc = hybridai::mi355x::detect_weight_format(st, c, weight_format, &err); rc != HAI_OK)
            return report(rc, err);
    }
    if (n_eos != nullptr) *n_eos = static_cast<int64_t>(eos.size());
    if (eos_ids != nullptr)
        for (int64_t i = 0; i < eos_capacity && i < static_cast<int64_t>(eos.size()); ++i) eos_ids[i] = eos[i];
    *cfg = c;
    return report(HAI_OK, "");
}

int hai_engine_load_checkpoint(void* engine, const char* dir) {
    if (!engine || !dir) return HAI_ERR_INVALID_ARGUMENT;
    Engine* e = as_engine(engine);
    hybridai::mi355x::SafeTensors st;
    std::string err;
    int rc = st.open(dir, &err);
    int32_t fmt = HAI_WEIGHTS_BF16;
    if (rc == HAI_OK) rc = hybridai::mi355x::detect_weight_format(st, e->config(), &fmt, &err);
    if (rc == HAI_OK && (fmt == HAI_WEIGHTS_FP8_BLOCK128) != e->fp8_weights()) {
        rc = HAI_ERR_INVALID_ARGUMENT;
        err = std::string("the checkpoint stores its Linears as ") + (fmt == HAI_WEIGHTS_FP8_BLOCK128 ? "FP8" : "BF16") +
              " but the engine was created for the other format";
    }
    if (rc != HAI_OK) return e->set_error(rc, "load_checkpoint: " + err);
    return e->load_checkpoint(st);
}

int64_t hai_engine_read_tensor(void* engine, uint32_t tensor_id, uint16_t* out, int64_t capacity) {
    if (!engine) return -1;
    return as_engine(engine)->read_tensor(tensor_id, out, capacity);
}

uint64_t hai_engine_weight_bytes(void* engine) { return engine ? as_engine(engine)->weight_bytes() : 0; }

int hai_engine_forward(void* engine, const int32_t* ids, int64_t T, uint16_t* hidden, uint16_t* logits) {
    if (!engine || !ids || as_engine(engine)->batch() != 1) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->forward_rows(ids, T, hidden, logits);
}

int hai_engine_forward_batch(void* engine, const int32_t* ids, int64_t T, uint16_t* hidden, uint16_t* logits) {
    if (!engine || !ids) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->forward_rows(ids, T, hidden, logits);
}

int64_t hai_engine_batch(void* engine) { return engine ? as_engine(engine)->batch() : 0; }

int hai_engine_generate_greedy(void* engine, const int32_t* prompt, int64_t P, int64_t max_new,
                               const int32_t* eos, int64_t n_eos, int32_t* out_tokens) {
    if (!engine || !prompt || !out_tokens) return -HAI_ERR_INVALID_ARGUMENT;
    int64_t n = 0;
    const int rc = as_engine(engine)->generate_greedy(prompt, P, max_new, eos, n_eos, out_tokens, &n);
    return rc == HAI_OK ? static_cast<int>(n) : -rc;
}

int hai_engine_generate_speculative(void* engine, const int32_t* prompt, int64_t P, int64_t max_new,
                                    int64_t width, const int32_t* eos, int64_t n_eos,
                                    const int32_t* draft_override, int64_t n_override, int32_t* out_tokens,
                                    hai_spec_stats* stats, int32_t* round_log, int64_t round_log_cap) {
    if (!engine || !prompt || !out_tokens || as_engine(engine)->batch() != 1) return -HAI_ERR_INVALID_ARGUMENT;
    int64_t n = 0;
    const int rc = as_engine(engine)->generate_speculative(prompt, P, max_new, width, eos, n_eos, draft_override,
                                                           n_override, out_tokens, stats, round_log,
                                                           round_log_cap, &n);
    return rc == HAI_OK ? static_cast<int>(n) : -rc;
}

int hai_engine_generate_speculative_batch(void* engine, const int32_t* prompts, int64_t P, int64_t max_new,
                                          int64_t width, const int32_t* eos, int64_t n_eos,
                                          const int32_t* draft_override, int64_t n_override, int32_t* out_tokens,
                                          int64_t* n_out, hai_spec_stats* stats, int32_t* round_log,
                                          int64_t round_log_cap) {
    if (!engine || !prompts || !out_tokens || !n_out) return -HAI_ERR_INVALID_ARGUMENT;
    const int rc = as_engine(engine)->generate_speculative(prompts, P, max_new, width, eos, n_eos, draft_override,
                                                           n_override, out_tokens, stats, round_log,
                                                           round_log_cap, n_out);
    return rc == HAI_OK ? 0 : -rc;
}

int hai_engine_prefill(void* engine, const int32_t* prompt, int64_t P, int64_t max_new) {
    if (!engine || !prompt) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->prefill(prompt, P, max_new);
}

int hai_engine_spec_rounds(void* engine, int64_t rounds, int64_t width, int32_t* out_tokens,
                           int64_t out_capacity, int64_t* n_out, hai_spec_stats* stats) {
    if (!engine) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->spec_rounds(rounds, width, out_tokens, out_capacity, n_out, stats);
}

int hai_engine_set_draft_override(void* engine, const int32_t* tokens, int64_t n) {
    if (!engine) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->set_draft_override(tokens, n);
}

int hai_engine_set_prefill_rows(void* engine, int64_t rows) {
    if (!engine) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->set_prefill_rows(rows);
}

int hai_engine_profile_verify(void* engine, int64_t T, int64_t iters, hai_verify_profile* out) {
    if (!engine || !out) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->profile_verify(T, iters, out);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// tokenizer (include/hai_tokenizer.h)

namespace {
using hybridai::mi355x::QwenTokenizer;
QwenTokenizer* as_tokenizer(void* t) { return static_cast<QwenTokenizer*>(t); }

template <typename T>
int32_t emit(const T* src, size_t n, T* out, int64_t capacity, int64_t* n_out) {
    if (n_out == nullptr) return HAI_ERR_INVALID_ARGUMENT;
    *n_out = static_cast<int64_t>(n);
    if (static_cast<int64_t>(n) > capacity) return HAI_ERR_INVALID_ARGUMENT;
    if (n > 0) {
        if (out == nullptr) return HAI_ERR_INVALID_ARGUMENT;
        std::memcpy(out, src, n * sizeof(T));
    }
    return HAI_OK;
}

int32_t emit_text(const std::string& s, char* out, int64_t capacity, int64_t* n_out) {
    const int32_t rc = emit(s.data(), s.size(), out, capacity, n_out);
    if (rc == HAI_OK && out != nullptr && capacity > static_cast<int64_t>(s.size())) out[s.size()] = '\0';
    return rc;
}
}  // namespace

extern "C" {

void* hai_tokenizer_open(const char* dir, int32_t* status, char* message, int64_t message_capacity) {
    auto report = [&](int32_t rc, const std::string& what) {
        if (status != nullptr) *status = rc;
        if (message != nullptr && message_capacity > 0) {
            const size_t n = std::min(what.size(), static_cast<size_t>(message_capacity - 1));
            std::memcpy(message, what.data(), n);
            message[n] = '\0';
        }
    };
    if (dir == nullptr) {
        report(HAI_ERR_INVALID_ARGUMENT, "null directory");
        return nullptr;
    }
    auto* t = new (std::nothrow) QwenTokenizer();
    if (t == nullptr) {
        report(HAI_ERR_OUT_OF_MEMORY, "out of host memory");
        return nullptr;
    }
    std::string err;
    if (const int rc = t->load(dir, &err); rc != HAI_OK) {
        delete t;
        report(rc, err);
        return nullptr;
    }
    report(HAI_OK, "");
    return t;
}

void hai_tokenizer_close(void* tokenizer) { delete as_tokenizer(tokenizer); }

int32_t hai_tokenizer_encode(void* tokenizer, const char* text, int64_t text_bytes, int64_t* ids, int64_t capacity,
                             int64_t* n_out) {
    if (tokenizer == nullptr || text_bytes < 0 || (text == nullptr && text_bytes > 0)) return HAI_ERR_INVALID_ARGUMENT;
    const std::vector<int64_t> v =
        as_tokenizer(tokenizer)->encode(std::string(text ? text : "", static_cast<size_t>(text_bytes)));
    return emit(v.data(), v.size(), ids, capacity, n_out);
}

int32_t hai_tokenizer_decode(void* tokenizer, const int64_t* ids, int64_t n_ids, int32_t skip_special, char* out,
                             int64_t capacity, int64_t* n_out) {
    if (tokenizer == nullptr || n_ids < 0 || (ids == nullptr && n_ids > 0)) return HAI_ERR_INVALID_ARGUMENT;
    return emit_text(as_tokenizer(tokenizer)->decode(ids, static_cast<size_t>(n_ids), skip_special != 0), out,
                     capacity, n_out);
}

int32_t hai_tokenizer_chat_prompt(const char* const* roles, const char* const* contents, int64_t n_messages,
                                  int32_t add_generation_prompt, int32_t enable_thinking, char* out,
                                  int64_t capacity, int64_t* n_out) {
    if (n_messages < 0 || (n_messages > 0 && (roles == nullptr || contents == nullptr))) return HAI_ERR_INVALID_ARGUMENT;
    std::vector<std::pair<std::string, std::string>> m;
    for (int64_t i = 0; i < n_messages; ++i) {
        if (roles[i] == nullptr || contents[i] == nullptr) return HAI_ERR_INVALID_ARGUMENT;
        m.emplace_back(roles[i], contents[i]);
    }
    return emit_text(QwenTokenizer::chat_prompt(m, add_generation_prompt != 0, enable_thinking != 0), out, capacity,
                     n_out);
}

int32_t hai_tokenizer_special_ids(void* tokenizer, int64_t* eos, int64_t eos_capacity, int64_t* n_eos, int64_t* pad,
                                  int64_t* bos) {
    if (tokenizer == nullptr) return HAI_ERR_INVALID_ARGUMENT;
    const QwenTokenizer* t = as_tokenizer(tokenizer);
    if (pad != nullptr) *pad = t->pad_token_id();
    if (bos != nullptr) *bos = t->bos_token_id();
    return emit(t->eos_token_ids().data(), t->eos_token_ids().size(), eos, eos_capacity, n_eos);
}

int32_t hai_tokenizer_pieces(void* tokenizer, const char* text, int64_t text_bytes, int64_t* bounds,
                             int64_t capacity, int64_t* n_out) {
    if (tokenizer == nullptr || text_bytes < 0 || (text == nullptr && text_bytes > 0)) return HAI_ERR_INVALID_ARGUMENT;
    const auto p = as_tokenizer(tokenizer)->pieces(std::string(text ? text : "", static_cast<size_t>(text_bytes)));
    std::vector<int64_t> flat;
    flat.reserve(2 * p.size());
    for (const auto& r : p) {
        flat.push_back(static_cast<int64_t>(r.first));
        flat.push_back(static_cast<int64_t>(r.second));
    }
    const int32_t rc = emit(flat.data(), flat.size(), bounds, capacity, n_out);
    if (n_out != nullptr) *n_out = static_cast<int64_t>(p.size());
    return rc;
}

}  // extern "C"
