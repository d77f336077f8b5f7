// generator_run.cc -- drives hybridai::Generator (include/hybrid.h) the way a
// caller such as demo/generate does, against this library.
//
//   generator_run --cpu                      error paths that need no device
//   generator_run <model_dir> <greedy|spec> <prompt> <max_new> [plain|chat|chat-think]
//       prints "tokens <id> <id> ...", "stats <name>=<value> ..." and
//       "text_hex <result text as hex, - when empty>"; the last argument sets
//       GenerationOptions::use_chat_template / enable_thinking (default: the
//       struct's defaults, chat without thinking).
#include <cstdio>
#include <cstring>
#include <string>

#include "refabi/hybrid_api.h"

using namespace hybridai;

namespace {

int fails = 0;

void expect_code(const ApiStatus& st, ApiStatusCode want, const char* what) {
    if (st.code() != want) {
        std::printf("FAIL %s: code %d (%s)\n", what, static_cast<int>(st.code()), st.message().c_str());
        ++fails;
    }
}

int cpu_checks() {
    {
        Generator g(GeneratorOptions{"synthetic:tiny", "cpu", 1, false});
        expect_code(g.load_model(), ApiStatusCode::NotImplemented, "cpu backend");
    }
    {
        Generator g(GeneratorOptions{"/nonexistent/model", "hip", 1, false});
        expect_code(g.load_model(), ApiStatusCode::FileNotFound, "missing model dir");
    }
    {
        Generator g(GeneratorOptions{"/tmp", "hip", 1, false});
        expect_code(g.load_model(), ApiStatusCode::FileNotFound, "checkpoint dir without config.json");
    }
    {
        Generator g(GeneratorOptions{"synthetic:huge", "hip", 1, false});
        expect_code(g.load_model(), ApiStatusCode::InvalidModel, "unknown synthetic model");
    }
    {
        Generator g(GeneratorOptions{"synthetic:tiny?flavour=1", "hip", 1, false});
        expect_code(g.load_model(), ApiStatusCode::InvalidArgument, "unknown model option");
    }
    {
        Generator g;
        GenerationResult r;
        expect_code(g.generate(GenerationOptions{}, &r), ApiStatusCode::InvalidModel, "generate before load");
        expect_code(g.reset(), ApiStatusCode::OK, "reset");
    }
    std::printf("generator (cpu): %d failed\n", fails);
    return fails == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--cpu") == 0) return cpu_checks();
    if (argc != 5 && argc != 6) {
        std::fprintf(stderr, "usage: %s <model_dir> <greedy|spec> <prompt> <max_new> [plain|chat|chat-think]\n",
                     argv[0]);
        return 2;
    }
    const std::string layout = argc == 6 ? argv[5] : "chat";
    Generator g(GeneratorOptions{argv[1], "hip", 1, true});
    ApiStatus st = g.load_model();
    if (!st.ok()) {
        std::printf("load_model failed: %d %s\n", static_cast<int>(st.code()), st.message().c_str());
        return 1;
    }
    GenerationOptions o;
    o.prompt = argv[3];
    o.max_new_tokens = std::atoi(argv[4]);
    o.enable_speculative_mtp = std::strcmp(argv[2], "spec") == 0;
    o.use_chat_template = layout != "plain";
    o.enable_thinking = layout == "chat-think";
    GenerationResult r;
    st = g.generate(o, &r);
    if (!st.ok()) {
        std::printf("generate failed: %d %s\n", static_cast<int>(st.code()), st.message().c_str());
        return 1;
    }
    // bad arguments after a successful load are rejected (generator.cc:458-461),
    // and a model without a tokenizer refuses text prompts
    GenerationResult bad;
    GenerationOptions ob = o;
    ob.prompt = "";
    const bool empty_refused = g.generate(ob, &bad).code() == ApiStatusCode::InvalidArgument;
    ob = o;
    ob.max_new_tokens = 0;
    const bool zero_refused = g.generate(ob, &bad).code() == ApiStatusCode::InvalidArgument;
    ob = o;
    ob.prompt = "hello";
    const bool ids_model = o.prompt.rfind("ids:", 0) == 0;
    const bool text_refused = g.generate(ob, &bad).code() == ApiStatusCode::InvalidArgument;
    if (!empty_refused || !zero_refused || (ids_model && !text_refused)) {
        std::printf("FAIL bad arguments accepted (empty %d, zero %d, text %d)\n", empty_refused, zero_refused,
                    text_refused);
        return 1;
    }
    std::printf("tokens");
    for (int64_t t : r.token_ids) std::printf(" %lld", static_cast<long long>(t));
    std::printf("\nstats prompt_tokens=%lld rounds=%lld proposed=%lld accepted=%lld rejected=%lld corrections=%lld "
                "replay_tokens=%lld mtp_recovery_tokens=%lld max_width=%lld decode_tps=%.3f text_ok=%d\n",
                static_cast<long long>(r.prompt_tokens), static_cast<long long>(r.speculative_rounds),
                static_cast<long long>(r.mtp_proposed_tokens), static_cast<long long>(r.mtp_accepted_tokens),
                static_cast<long long>(r.mtp_rejected_tokens), static_cast<long long>(r.mtp_correction_tokens),
                static_cast<long long>(r.speculative_replay_tokens),
                static_cast<long long>(r.speculative_mtp_recovery_tokens),
                static_cast<long long>(r.speculative_max_proposal_width), r.decode_tokens_per_second,
                r.text.rfind("ids:", 0) == 0 ? 1 : 0);
    std::printf("text_hex %s", r.text.empty() ? "-" : "");
    for (unsigned char c : r.text) std::printf("%02x", c);
    std::printf("\n");
    return 0;
}
