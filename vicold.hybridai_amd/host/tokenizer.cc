// tokenizer.cc -- see tokenizer.h.
#include "tokenizer.h"

#include <algorithm>
#include <array>
#include <cstdint>
#include <queue>

#include "checkpoint.h"
#include "hai_kernels.h"
#include "json.h"

namespace hybridai::mi355x {

namespace {

enum class CpClass : uint8_t { kLetter = 1, kMark = 2, kNumber = 4 };
struct CodepointRange {
    uint32_t first, last;
    CpClass cls;
};
#include "unicode_classes.inc"

constexpr uint8_t kL = 1, kM = 2, kN = 4, kS = 8;  // \p{L} \p{M} \p{N} \s
constexpr uint32_t kInvalidByte = 0xFFFFFFFFu;       // a byte that starts no valid UTF-8 sequence

uint8_t class_of_slow(uint32_t cp) {
    for (uint32_t w : kSpaceCodepoints)
        if (w == cp) return kS;
    const CodepointRange* b = std::begin(kClassRanges);
    const CodepointRange* e = std::end(kClassRanges);
    const CodepointRange* it =
        std::upper_bound(b, e, cp, [](uint32_t c, const CodepointRange& r) { return c < r.first; });
    if (it == b) return 0;
    --it;
    return cp <= it->last ? static_cast<uint8_t>(it->cls) : 0;
}

uint8_t class_of(uint32_t cp) {
    static const std::array<uint8_t, 128> ascii = [] {
        std::array<uint8_t, 128> t{};
        for (uint32_t c = 0; c < 128; ++c) t[c] = class_of_slow(c);
        return t;
    }();
    if (cp < 128) return ascii[cp];
    if (cp == kInvalidByte) return 0;
    return class_of_slow(cp);
}

// One codepoint of s at byte i: its value and length; an ill-formed sequence
// (overlong, surrogate, above U+10FFFF, truncated) yields its first byte
// alone as kInvalidByte, so that every byte of the text is kept.
uint32_t next_codepoint(const std::string& s, size_t i, size_t end, size_t* len) {
    const auto u = [&](size_t k) { return static_cast<uint8_t>(s[k]); };
    const uint8_t c = u(i);
    *len = 1;
    if (c < 0x80) return c;
    size_t n;
    uint32_t cp, min;
    if ((c & 0xE0) == 0xC0) n = 2, cp = c & 0x1F, min = 0x80;
    else if ((c & 0xF0) == 0xE0) n = 3, cp = c & 0x0F, min = 0x800;
    else if ((c & 0xF8) == 0xF0) n = 4, cp = c & 0x07, min = 0x10000;
    else return kInvalidByte;
    if (i + n > end) return kInvalidByte;
    for (size_t k = 1; k < n; ++k) {
        if ((u(i + k) & 0xC0) != 0x80) return kInvalidByte;
        cp = (cp << 6) | (u(i + k) & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return kInvalidByte;
    *len = n;
    return cp;
}

void put_utf8(uint32_t cp, std::string* out) {
    if (cp < 0x80) {
        out->push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
        out->push_back(static_cast<char>(0xC0 | (cp >> 6)));
        out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
        out->push_back(static_cast<char>(0xE0 | (cp >> 12)));
        out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
        out->push_back(static_cast<char>(0xF0 | (cp >> 18)));
        out->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
        out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
}

// The byte-level alphabet (the GPT-2 byte encoder every Qwen vocabulary is
// written in): the 188 printable bytes stand for themselves, the other 68
// bytes take the codepoints 256.. in byte order.
struct ByteAlphabet {
    std::array<uint32_t, 256> symbol{};
    std::array<int16_t, 256 + 68> byte{};  // symbol codepoint -> byte, -1 when none
    ByteAlphabet() {
        byte.fill(-1);
        uint32_t extra = 0;
        for (uint32_t b = 0; b < 256; ++b) {
            const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE);
            symbol[b] = printable ? b : 256 + extra++;
            byte[symbol[b]] = static_cast<int16_t>(b);
        }
    }
};
const ByteAlphabet& alphabet() {
    static const ByteAlphabet a;
    return a;
}

// bytes a vocabulary entry stands for; false when a character of it is not
// in the byte-level alphabet (such characters are dropped)
bool symbols_to_bytes(const std::string& key, std::string* bytes) {
    bytes->clear();
    bool pure = true;
    for (size_t i = 0; i < key.size();) {
        size_t len;
        const uint32_t cp = next_codepoint(key, i, key.size(), &len);
        i += len;
        if (cp < alphabet().byte.size() && alphabet().byte[cp] >= 0) bytes->push_back(static_cast<char>(alphabet().byte[cp]));
        else pure = false;
    }
    return pure;
}

// Lower-case the letters of the contraction alternatives the way the
// pattern's (?i:...) group compares them (U+017F folds to 's').
uint32_t fold(uint32_t c) {
    if (c >= 'A' && c <= 'Z') return c + ('a' - 'A');
    if (c == 0x17F) return 's';
    return c;
}

// End (codepoint index) of the pattern's match at codepoint i; the
// alternatives are tried in the pattern's order.  Every codepoint is a
// letter / mark, a number, whitespace or in the symbol class, so some
// alternative always matches.
size_t match_at(const std::vector<uint32_t>& cp, const std::vector<uint8_t>& cls, size_t i) {
    const size_t n = cp.size();
    const auto is_nl = [&](size_t k) { return cp[k] == '\r' || cp[k] == '\n'; };
    // (?i:'s|'t|'re|'ve|'m|'ll|'d)
    if (cp[i] == '\'' && i + 1 < n) {
        const uint32_t a = fold(cp[i + 1]);
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
        if (i + 2 < n) {
            const uint32_t b = fold(cp[i + 2]);
            if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return i + 3;
        }
    }
    // [^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+ : a mark may be the optional first
    // character or the first of the run; either way the run goes on through
    // every following letter and mark
    if (!is_nl(i) && !(cls[i] & kN) && ((cls[i] & (kL | kM)) || (i + 1 < n && (cls[i + 1] & (kL | kM))))) {
        size_t j = i + 1;
        while (j < n && (cls[j] & (kL | kM))) ++j;
        return j;
    }
    // \p{N}
    if (cls[i] & kN) return i + 1;
    // ' ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*'
    {
        const size_t j = cp[i] == ' ' ? i + 1 : i;
        if (j < n && cls[j] == 0) {
            size_t k = j;
            while (k < n && cls[k] == 0) ++k;
            while (k < n && is_nl(k)) ++k;
            return k;
        }
    }
    // \s*[\r\n]+ : through the run's last line break
    size_t j = i, last_nl = n;
    while (j < n && (cls[j] & kS)) {
        if (is_nl(j)) last_nl = j;
        ++j;
    }
    if (last_nl < n) return last_nl + 1;
    // \s+(?!\S) : a run followed by text gives back its last whitespace
    if (j - i >= 2 && j < n) return j - 1;
    // \s+
    if (j > i) return j;
    return i + 1;
}

struct Candidate {
    int32_t rank;
    uint32_t pos;
    int32_t merged;
    bool operator>(const Candidate& o) const { return rank != o.rank ? rank > o.rank : pos > o.pos; }
};

int fail(std::string* err, int code, const std::string& what) {
    if (err) *err = what;
    return code;
}

bool int_id(const Json& v, int64_t* out) { return v.is_integer() && v.to_int64(out); }

}  // namespace

void QwenTokenizer::clear() {
    loaded_ = false;
    ignore_merges_ = false;
    std::fill(std::begin(byte_symbol_), std::end(byte_symbol_), -1);
    token_bytes_.clear();
    has_token_.clear();
    by_bytes_.clear();
    merges_.clear();
    added_.clear();
    added_by_byte_.assign(256, {});
    added_by_id_.clear();
    eos_.clear();
    pad_ = bos_ = -1;
}

// QwenTokenizer::load (qwen_tokenizer.cc:59-187): tokenizer.json's BPE model
// (vocab, merges as "a b" strings or [a, b] pairs, ignore_merges), its
// added_tokens, and generation_config.json's eos / pad / bos ids.
int QwenTokenizer::load(const std::string& dir, std::string* err) {
    clear();
    const int rc = load_files(dir, err);
    if (rc != HAI_OK) clear();
    return rc;
}

int QwenTokenizer::load_files(const std::string& dir, std::string* err) {
    const std::string path = path_join(dir, "tokenizer.json");
    if (!is_regular_file(path)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "tokenizer.json not found in " + dir);
    std::string text, why;
    if (!read_whole_file(path, &text)) return fail(err, HAI_ERR_FILE_NOT_FOUND, "Failed to open tokenizer.json");
    Json root;
    if (!Json::parse(text, &root, &why)) return fail(err, HAI_ERR_INVALID_MODEL, "Invalid tokenizer.json: " + why);
    text.clear();
    const Json* model = root.find("model");
    if (model == nullptr || !model->is_object())
        return fail(err, HAI_ERR_INVALID_MODEL, "tokenizer.json missing model section");
    const Json* type = model->find("type");
    if (type == nullptr || !type->is_string() || type->as_string() != "BPE")
        return fail(err, HAI_ERR_INVALID_MODEL, "Only BPE tokenizers are supported");
    const Json* vocab = model->find("vocab");
    const Json* merges = model->find("merges");
    if (vocab == nullptr || !vocab->is_object() || (merges != nullptr && !merges->is_array()))
        return fail(err, HAI_ERR_INVALID_MODEL, "tokenizer.json model needs a vocab object and a merges array");
    if (const Json* im = model->find("ignore_merges"); im != nullptr && im->is_bool()) ignore_merges_ = im->as_bool();

    std::unordered_map<std::string, int32_t> by_key;
    by_key.reserve(vocab->members().size());
    int64_t max_id = -1;
    for (const auto& kv : vocab->members()) {
        int64_t id;
        if (!int_id(kv.second, &id) || id < 0 || id > INT32_MAX)
            return fail(err, HAI_ERR_INVALID_MODEL, "tokenizer.json vocab id of \"" + kv.first + "\" is not a valid id");
        by_key[kv.first] = static_cast<int32_t>(id);
        max_id = std::max(max_id, id);
    }
    token_bytes_.assign(static_cast<size_t>(max_id + 1), {});
    has_token_.assign(static_cast<size_t>(max_id + 1), 0);
    std::string bytes;
    for (const auto& kv : by_key) {
        const bool pure = symbols_to_bytes(kv.first, &bytes);
        token_bytes_[static_cast<size_t>(kv.second)] = bytes;
        has_token_[static_cast<size_t>(kv.second)] = 1;
        if (ignore_merges_ && pure) by_bytes_[bytes] = kv.second;
    }
    for (uint32_t b = 0; b < 256; ++b) {
        std::string key;
        put_utf8(alphabet().symbol[b], &key);
        const auto it = by_key.find(key);
        if (it != by_key.end()) byte_symbol_[b] = it->second;
    }

    if (merges != nullptr) {
        merges_.reserve(merges->items().size());
        int32_t rank = 0;
        for (const Json& m : merges->items()) {
            std::string a, b;
            if (m.is_string()) {
                const std::string& s = m.as_string();
                const size_t sp = s.find(' ');
                if (sp == std::string::npos) return fail(err, HAI_ERR_INVALID_MODEL, "merge without a space: " + s);
                a = s.substr(0, sp);
                b = s.substr(sp + 1);
            } else if (m.is_array() && m.items().size() == 2 && m.items()[0].is_string() && m.items()[1].is_string()) {
                a = m.items()[0].as_string();
                b = m.items()[1].as_string();
            } else {
                return fail(err, HAI_ERR_INVALID_MODEL, "merges hold \"a b\" strings or [a, b] pairs");
            }
            const auto ia = by_key.find(a), ib = by_key.find(b), iab = by_key.find(a + b);
            if (ia == by_key.end() || ib == by_key.end() || iab == by_key.end())
                return fail(err, HAI_ERR_INVALID_MODEL, "merge \"" + a + " " + b + "\" is not in the vocabulary");
            const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(ia->second)) << 32) |
                                 static_cast<uint32_t>(ib->second);
            merges_[key] = Merge{rank++, iab->second};
        }
    }

    if (const Json* added = root.find("added_tokens"); added != nullptr && added->is_array()) {
        for (const Json& t : added->items()) {
            const Json* content = t.find("content");
            const Json* idv = t.find("id");
            const Json* special = t.find("special");
            int64_t id = -1;
            if (content == nullptr || !content->is_string() || content->as_string().empty()) continue;
            if (idv == nullptr || !int_id(*idv, &id) || id < 0) continue;
            const bool sp = special != nullptr && special->is_bool() && special->as_bool();
            if (const auto it = added_by_id_.find(id); it != added_by_id_.end()) {
                added_[it->second] = Added{content->as_string(), id, sp};
            } else {
                added_by_id_[id] = static_cast<uint32_t>(added_.size());
                added_.push_back(Added{content->as_string(), id, sp});
            }
        }
        // the last entry of a repeated content wins, as a content -> id map
        std::unordered_map<std::string, uint32_t> by_content;
        for (uint32_t k = 0; k < added_.size(); ++k) by_content[added_[k].content] = k;
        for (const auto& kv : by_content)
            added_by_byte_[static_cast<uint8_t>(kv.first[0])].push_back(kv.second);
        for (auto& list : added_by_byte_)
            std::sort(list.begin(), list.end(), [&](uint32_t x, uint32_t y) {
                return added_[x].content.size() > added_[y].content.size();
            });
    }

    const std::string gen_path = path_join(dir, "generation_config.json");
    if (is_regular_file(gen_path)) {
        Json gen;
        std::string gtext;
        if (!read_whole_file(gen_path, &gtext) || !Json::parse(gtext, &gen, &why))
            return fail(err, HAI_ERR_INVALID_MODEL, "Invalid generation_config.json: " + why);
        if (const Json* eos = gen.find("eos_token_id")) {
            int64_t id;
            if (int_id(*eos, &id)) {
                eos_.push_back(id);
            } else if (eos->is_array()) {
                for (const Json& e : eos->items()) {
                    if (!int_id(e, &id))
                        return fail(err, HAI_ERR_INVALID_MODEL, "generation_config.json contains a non-integer EOS id");
                    eos_.push_back(id);
                }
            } else {
                return fail(err, HAI_ERR_INVALID_MODEL, "generation_config.json has invalid eos_token_id");
            }
        }
        int64_t v;
        if (const Json* p = gen.find("pad_token_id"); p != nullptr && int_id(*p, &v)) pad_ = v;
        if (const Json* b = gen.find("bos_token_id"); b != nullptr && int_id(*b, &v)) bos_ = v;
    }
    loaded_ = true;
    return HAI_OK;
}

bool QwenTokenizer::is_eos_token(int64_t id) const { return std::find(eos_.begin(), eos_.end(), id) != eos_.end(); }

std::vector<std::pair<size_t, size_t>> QwenTokenizer::pieces(const std::string& text) const {
    std::vector<uint32_t> cp;
    std::vector<uint32_t> off;
    std::vector<uint8_t> cls;
    for (size_t i = 0; i < text.size();) {
        size_t len;
        const uint32_t c = next_codepoint(text, i, text.size(), &len);
        cp.push_back(c);
        off.push_back(static_cast<uint32_t>(i));
        cls.push_back(class_of(c));
        i += len;
    }
    off.push_back(static_cast<uint32_t>(text.size()));
    std::vector<std::pair<size_t, size_t>> out;
    for (size_t i = 0; i < cp.size();) {
        const size_t j = match_at(cp, cls, i);
        out.emplace_back(off[i], off[j]);
        i = j;
    }
    return out;
}

// The merges over one piece (the heap order of the reference's repeated
// lowest-rank scan, qwen_tokenizer.cc:393-428): lowest rank first, leftmost
// among equal ranks; a queued pair is stale once its left symbol was merged
// away or the pair now at its place merges into a different token.
void QwenTokenizer::bpe(const std::string& text, size_t begin, size_t end, std::vector<int64_t>* out) const {
    if (begin == end) return;
    if (ignore_merges_) {
        const auto it = by_bytes_.find(text.substr(begin, end - begin));
        if (it != by_bytes_.end()) {
            out->push_back(it->second);
            return;
        }
    }
    std::vector<int32_t> id;
    id.reserve(end - begin);
    for (size_t i = begin; i < end; ++i) {
        const int32_t s = byte_symbol_[static_cast<uint8_t>(text[i])];
        if (s >= 0) id.push_back(s);  // a byte without a symbol token is dropped
    }
    const size_t n = id.size();
    if (n == 0) return;
    if (n == 1) {
        out->push_back(id[0]);
        return;
    }
    std::vector<int32_t> prev(n), next(n);
    std::vector<uint8_t> alive(n, 1);
    for (size_t i = 0; i < n; ++i) {
        prev[i] = static_cast<int32_t>(i) - 1;
        next[i] = i + 1 < n ? static_cast<int32_t>(i + 1) : -1;
    }
    const auto lookup = [&](int32_t l, int32_t r) -> const Merge* {
        const auto it = merges_.find((static_cast<uint64_t>(static_cast<uint32_t>(l)) << 32) | static_cast<uint32_t>(r));
        return it == merges_.end() ? nullptr : &it->second;
    };
    std::priority_queue<Candidate, std::vector<Candidate>, std::greater<Candidate>> queue;
    for (size_t i = 0; i + 1 < n; ++i)
        if (const Merge* m = lookup(id[i], id[i + 1])) queue.push({m->rank, static_cast<uint32_t>(i), m->merged});
    while (!queue.empty()) {
        const Candidate c = queue.top();
        queue.pop();
        if (!alive[c.pos] || next[c.pos] < 0) continue;
        const int32_t r = next[c.pos];
        const Merge* now = lookup(id[c.pos], id[r]);
        if (now == nullptr || now->merged != c.merged) continue;
        id[c.pos] = c.merged;
        alive[r] = 0;
        next[c.pos] = next[r];
        if (next[r] >= 0) prev[next[r]] = static_cast<int32_t>(c.pos);
        if (prev[c.pos] >= 0)
            if (const Merge* m = lookup(id[prev[c.pos]], id[c.pos]))
                queue.push({m->rank, static_cast<uint32_t>(prev[c.pos]), m->merged});
        if (next[c.pos] >= 0)
            if (const Merge* m = lookup(id[c.pos], id[next[c.pos]])) queue.push({m->rank, c.pos, m->merged});
    }
    for (int32_t i = 0; i >= 0; i = next[i]) out->push_back(id[i]);
}

// QwenTokenizer::encode (qwen_tokenizer.cc:430-457)
std::vector<int64_t> QwenTokenizer::encode(const std::string& text) const {
    std::vector<int64_t> out;
    const auto plain = [&](size_t b, size_t e) {
        if (b == e) return;
        const std::string seg = text.substr(b, e - b);
        for (const auto& p : pieces(seg)) bpe(seg, p.first, p.second, &out);
    };
    size_t seg = 0;
    for (size_t i = 0; i < text.size();) {
        const Added* hit = nullptr;
        for (uint32_t k : added_by_byte_[static_cast<uint8_t>(text[i])]) {
            if (text.compare(i, added_[k].content.size(), added_[k].content) == 0) {
                hit = &added_[k];
                break;
            }
        }
        if (hit == nullptr) {
            ++i;
            continue;
        }
        plain(seg, i);
        out.push_back(hit->id);
        i += hit->content.size();
        seg = i;
    }
    plain(seg, text.size());
    return out;
}

// QwenTokenizer::decode (qwen_tokenizer.cc:459-488)
std::string QwenTokenizer::decode(const int64_t* ids, size_t n, bool skip_special) const {
    std::string out;
    for (size_t k = 0; k < n; ++k) {
        const int64_t id = ids[k];
        if (const auto it = added_by_id_.find(id); it != added_by_id_.end()) {
            const Added& a = added_[it->second];
            if (!skip_special || !a.special) out += a.content;
            continue;
        }
        if (id >= 0 && id < static_cast<int64_t>(token_bytes_.size()) && has_token_[static_cast<size_t>(id)])
            out += token_bytes_[static_cast<size_t>(id)];
    }
    return out;
}

// QwenTokenizer::build_chat_prompt (qwen_tokenizer.cc:490-503): the ChatML
// layout of Qwen checkpoints
std::string QwenTokenizer::chat_prompt(const std::vector<std::pair<std::string, std::string>>& messages,
                                       bool add_generation_prompt, bool enable_thinking) {
    std::string p;
    for (const auto& m : messages) p += "<|im_start|>" + m.first + "\n" + m.second + "<|im_end|>\n";
    if (add_generation_prompt) {
        p += "<|im_start|>assistant\n";
        p += enable_thinking ? "<think>\n" : "<think>\n\n</think>\n\n";
    }
    return p;
}

}  // namespace hybridai::mi355x
