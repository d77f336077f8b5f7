// tokenizer.h -- the byte-level BPE tokenizer of Qwen checkpoints, read from
// <dir>/tokenizer.json and <dir>/generation_config.json: the role of the
// reference's tokenizer::QwenTokenizer (tokenizer/qwen_tokenizer.h:15-104),
// which hybridai::Generator uses for text prompts, the chat template, the
// stop ids and the result text (generator.cc:423, 469-480, 1032, 1275).
//
// Encoding: added tokens are cut out first (leftmost, longest match), the
// rest is split by the Qwen pre-tokenizer pattern
//   (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}|
//    ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
// (matched by hand over codepoints, with the engine's own Unicode classes),
// each piece's bytes become the byte-level symbols and the merges are applied
// lowest rank first, leftmost first among equal ranks.  Host code only.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace hybridai::mi355x {

class QwenTokenizer {
public:
    QwenTokenizer() { clear(); }

    // HAI_OK, HAI_ERR_FILE_NOT_FOUND (no tokenizer.json) or
    // HAI_ERR_INVALID_MODEL (malformed files, a model type other than BPE, a
    // merge whose parts or result are not in the vocabulary, a non-integer
    // eos_token_id), with a message in *err.  A failed load leaves the
    // tokenizer empty.
    int load(const std::string& dir, std::string* err);
    bool loaded() const { return loaded_; }

    // token ids of text (add_special_tokens has no effect for these
    // checkpoints: their post-processor adds nothing)
    std::vector<int64_t> encode(const std::string& text) const;
    // bytes of the tokens; added tokens give their content unless
    // skip_special and the token is special; ids with no token are skipped
    std::string decode(const int64_t* ids, size_t n, bool skip_special) const;
    // the pre-tokenizer's pieces of a text without added tokens, as byte
    // ranges [begin, end)
    std::vector<std::pair<size_t, size_t>> pieces(const std::string& text) const;

    // "<|im_start|>role\ncontent<|im_end|>\n" per message, then the
    // assistant header and the thinking block opener
    // (qwen_tokenizer.cc build_chat_prompt)
    static std::string chat_prompt(const std::vector<std::pair<std::string, std::string>>& messages,
                                   bool add_generation_prompt, bool enable_thinking);

    const std::vector<int64_t>& eos_token_ids() const { return eos_; }
    bool is_eos_token(int64_t id) const;
    int64_t pad_token_id() const { return pad_; }
    int64_t bos_token_id() const { return bos_; }
    int64_t vocab_size() const { return static_cast<int64_t>(token_bytes_.size()); }

private:
    struct Merge {
        int32_t rank;
        int32_t merged;
    };
    struct Added {
        std::string content;
        int64_t id;
        bool special;
    };

    void clear();
    int load_files(const std::string& dir, std::string* err);
    void bpe(const std::string& text, size_t begin, size_t end, std::vector<int64_t>* out) const;

    bool loaded_ = false;
    bool ignore_merges_ = false;
    int32_t byte_symbol_[256];                      // id of the one-symbol token of each byte (-1: none)
    std::vector<std::string> token_bytes_;          // id -> the bytes its symbols stand for
    std::vector<uint8_t> has_token_;                // id -> the vocabulary holds it
    std::unordered_map<std::string, int32_t> by_bytes_;   // bytes -> id (ignore_merges lookups)
    std::unordered_map<uint64_t, Merge> merges_;    // (left id << 32 | right id) -> rank, result
    std::vector<Added> added_;
    std::vector<std::vector<uint32_t>> added_by_byte_;  // first byte -> added_ indices, longest first
    std::unordered_map<int64_t, uint32_t> added_by_id_;
    std::vector<int64_t> eos_;
    int64_t pad_ = -1, bos_ = -1;
};

}  // namespace hybridai::mi355x
