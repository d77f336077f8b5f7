// json.h -- a small JSON reader for the checkpoint files the loader opens:
// safetensors headers, model.safetensors.index.json and config.json.
// Values are immutable after parsing; numbers keep their text so that
// integers up to 64 bits (tensor byte offsets) read back exactly.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace hybridai::mi355x {

class Json {
public:
    enum class Type { Null, Bool, Number, String, Array, Object };

    Type type() const { return type_; }
    bool is_null() const { return type_ == Type::Null; }
    bool is_bool() const { return type_ == Type::Bool; }
    bool is_number() const { return type_ == Type::Number; }
    bool is_string() const { return type_ == Type::String; }
    bool is_array() const { return type_ == Type::Array; }
    bool is_object() const { return type_ == Type::Object; }
    // an integer literal (no fraction or exponent)
    bool is_integer() const;

    bool as_bool() const { return bool_; }
    const std::string& as_string() const { return text_; }
    // the number's value; false when the literal does not fit
    bool to_int64(int64_t* out) const;
    bool to_uint64(uint64_t* out) const;
    double to_double() const;

    const std::vector<Json>& items() const { return array_; }
    // members in file order (duplicate keys: the last one wins in find())
    const std::vector<std::pair<std::string, Json>>& members() const { return object_; }
    // nullptr when absent or when this is not an object
    const Json* find(const std::string& key) const;

    // Parses the whole of text; on failure returns false with a message
    // naming the byte offset.
    static bool parse(const std::string& text, Json* out, std::string* error);

private:
    friend class JsonParser;
    Type type_ = Type::Null;
    bool bool_ = false;
    std::string text_;  // string value, or the number's literal
    std::vector<Json> array_;
    std::vector<std::pair<std::string, Json>> object_;
};

}  // namespace hybridai::mi355x
