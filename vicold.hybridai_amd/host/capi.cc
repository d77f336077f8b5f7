// capi.cc -- extern "C" surface of the verify engine (include/hai_engine.h).
#include <new>
#include <string>

#include "engine.h"
#include "hai_kernels.h"

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

int hai_engine_profile_verify(void* engine, int64_t T, int64_t iters, hai_verify_profile* out) {
    if (!engine || !out) return HAI_ERR_INVALID_ARGUMENT;
    return as_engine(engine)->profile_verify(T, iters, out);
}

}  // extern "C"
