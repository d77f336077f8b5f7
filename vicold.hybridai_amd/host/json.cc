// json.cc -- recursive-descent JSON reader (RFC 8259 grammar; strings with
// \u escapes decoded to UTF-8, surrogate pairs joined).
#include "json.h"

#include <cerrno>
#include <cstdlib>
#include <limits>

namespace hybridai::mi355x {

bool Json::is_integer() const {
    if (type_ != Type::Number) return false;
    return text_.find_first_of(".eE") == std::string::npos;
}

bool Json::to_int64(int64_t* out) const {
    if (!is_integer()) return false;
    errno = 0;
    char* end = nullptr;
    const long long v = std::strtoll(text_.c_str(), &end, 10);
    if (errno != 0 || end == nullptr || *end != '\0') return false;
    *out = static_cast<int64_t>(v);
    return true;
}

bool Json::to_uint64(uint64_t* out) const {
    if (!is_integer() || text_[0] == '-') return false;
    errno = 0;
    char* end = nullptr;
    const unsigned long long v = std::strtoull(text_.c_str(), &end, 10);
    if (errno != 0 || end == nullptr || *end != '\0') return false;
    *out = static_cast<uint64_t>(v);
    return true;
}

double Json::to_double() const { return type_ == Type::Number ? std::strtod(text_.c_str(), nullptr) : 0.0; }

const Json* Json::find(const std::string& key) const {
    if (type_ != Type::Object) return nullptr;
    const Json* hit = nullptr;
    for (const auto& kv : object_)
        if (kv.first == key) hit = &kv.second;
    return hit;
}

class JsonParser {
public:
    explicit JsonParser(const std::string& s) : s_(s) {}

    bool run(Json* out, std::string* error) {
        skip_ws();
        if (!value(out, 0)) return fail_out(error);
        skip_ws();
        if (pos_ != s_.size()) {
            why_ = "trailing characters";
            return fail_out(error);
        }
        return true;
    }

private:
    static constexpr int kMaxDepth = 256;
    const std::string& s_;
    size_t pos_ = 0;
    std::string why_;

    bool fail_out(std::string* error) {
        if (error) *error = "JSON: " + why_ + " at byte " + std::to_string(pos_);
        return false;
    }
    bool fail(const char* why) {
        why_ = why;
        return false;
    }
    void skip_ws() {
        while (pos_ < s_.size() && (s_[pos_] == ' ' || s_[pos_] == '\t' || s_[pos_] == '\n' || s_[pos_] == '\r'))
            ++pos_;
    }
    bool literal(const char* word) {
        size_t n = 0;
        while (word[n]) ++n;
        if (s_.compare(pos_, n, word) != 0) return fail("invalid literal");
        pos_ += n;
        return true;
    }

    bool value(Json* out, int depth) {
        if (depth > kMaxDepth) return fail("nesting too deep");
        if (pos_ >= s_.size()) return fail("unexpected end");
        const char c = s_[pos_];
        if (c == '{') return object(out, depth);
        if (c == '[') return array(out, depth);
        if (c == '"') {
            out->type_ = Json::Type::String;
            return string(&out->text_);
        }
        if (c == 't') {
            out->type_ = Json::Type::Bool;
            out->bool_ = true;
            return literal("true");
        }
        if (c == 'f') {
            out->type_ = Json::Type::Bool;
            out->bool_ = false;
            return literal("false");
        }
        if (c == 'n') {
            out->type_ = Json::Type::Null;
            return literal("null");
        }
        return number(out);
    }

    bool number(Json* out) {
        const size_t start = pos_;
        auto digits = [&]() {
            const size_t d0 = pos_;
            while (pos_ < s_.size() && s_[pos_] >= '0' && s_[pos_] <= '9') ++pos_;
            return pos_ > d0;
        };
        if (pos_ < s_.size() && s_[pos_] == '-') ++pos_;
        if (pos_ < s_.size() && s_[pos_] == '0') {
            ++pos_;
        } else if (!digits()) {
            return fail("invalid value");
        }
        if (pos_ < s_.size() && s_[pos_] == '.') {
            ++pos_;
            if (!digits()) return fail("invalid fraction");
        }
        if (pos_ < s_.size() && (s_[pos_] == 'e' || s_[pos_] == 'E')) {
            ++pos_;
            if (pos_ < s_.size() && (s_[pos_] == '+' || s_[pos_] == '-')) ++pos_;
            if (!digits()) return fail("invalid exponent");
        }
        out->type_ = Json::Type::Number;
        out->text_ = s_.substr(start, pos_ - start);
        return true;
    }

    static void put_utf8(uint32_t cp, std::string* out) {
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

    bool hex4(uint32_t* v) {
        if (pos_ + 4 > s_.size()) return fail("short \\u escape");
        uint32_t r = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = s_[pos_++];
            r <<= 4;
            if (c >= '0' && c <= '9') r |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') r |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') r |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("invalid \\u escape");
        }
        *v = r;
        return true;
    }

    bool string(std::string* out) {
        ++pos_;  // opening quote
        out->clear();
        while (true) {
            if (pos_ >= s_.size()) return fail("unterminated string");
            const unsigned char c = static_cast<unsigned char>(s_[pos_++]);
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                out->push_back(static_cast<char>(c));
                continue;
            }
            if (pos_ >= s_.size()) return fail("unterminated escape");
            const char e = s_[pos_++];
            switch (e) {
                case '"': out->push_back('"'); break;
                case '\\': out->push_back('\\'); break;
                case '/': out->push_back('/'); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    uint32_t cp = 0;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo = 0;
                        if (pos_ + 2 > s_.size() || s_[pos_] != '\\' || s_[pos_ + 1] != 'u')
                            return fail("unpaired surrogate");
                        pos_ += 2;
                        if (!hex4(&lo)) return false;
                        if (lo < 0xDC00 || lo >= 0xE000) return fail("invalid surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("unpaired surrogate");
                    }
                    put_utf8(cp, out);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
    }

    bool array(Json* out, int depth) {
        ++pos_;
        out->type_ = Json::Type::Array;
        skip_ws();
        if (pos_ < s_.size() && s_[pos_] == ']') {
            ++pos_;
            return true;
        }
        while (true) {
            skip_ws();
            out->array_.emplace_back();
            if (!value(&out->array_.back(), depth + 1)) return false;
            skip_ws();
            if (pos_ >= s_.size()) return fail("unterminated array");
            if (s_[pos_] == ',') {
                ++pos_;
                continue;
            }
            if (s_[pos_] == ']') {
                ++pos_;
                return true;
            }
            return fail("expected , or ]");
        }
    }

    bool object(Json* out, int depth) {
        ++pos_;
        out->type_ = Json::Type::Object;
        skip_ws();
        if (pos_ < s_.size() && s_[pos_] == '}') {
            ++pos_;
            return true;
        }
        while (true) {
            skip_ws();
            if (pos_ >= s_.size() || s_[pos_] != '"') return fail("expected a member name");
            std::string key;
            if (!string(&key)) return false;
            skip_ws();
            if (pos_ >= s_.size() || s_[pos_] != ':') return fail("expected :");
            ++pos_;
            skip_ws();
            out->object_.emplace_back(std::move(key), Json{});
            if (!value(&out->object_.back().second, depth + 1)) return false;
            skip_ws();
            if (pos_ >= s_.size()) return fail("unterminated object");
            if (s_[pos_] == ',') {
                ++pos_;
                continue;
            }
            if (s_[pos_] == '}') {
                ++pos_;
                return true;
            }
            return fail("expected , or }");
        }
    }
};

bool Json::parse(const std::string& text, Json* out, std::string* error) {
    Json v;
    JsonParser p(text);
    if (!p.run(&v, error)) return false;
    *out = std::move(v);
    return true;
}

}  // namespace hybridai::mi355x
