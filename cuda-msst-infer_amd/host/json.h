// json.h — the JSON value the model configs use (the reference's JsonValue,
// src/weights.h:14-96): null, bool, number, string, array, object; parse()
// throws std::runtime_error on malformed input.  Objects keep their keys
// sorted (std::map); lookups of missing keys throw, get_* return defaults.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace cudasep {

class JsonValue {
public:
    enum Type { Null, Bool, Number, String, Array, Object };

    JsonValue() = default;
    static JsonValue parse(const std::string& text);

    Type type() const { return type_; }
    bool is_null() const { return type_ == Null; }
    bool is_array() const { return type_ == Array; }
    bool is_object() const { return type_ == Object; }

    bool as_bool() const;
    double as_number() const;
    int as_int() const { return (int)as_number(); }
    const std::string& as_string() const;

    size_t size() const;                                  // array / object size
    const JsonValue& operator[](size_t i) const;          // array element
    const JsonValue& operator[](const std::string& key) const;  // object member
    bool has(const std::string& key) const;

    int get_int(const std::string& key, int def) const;
    double get_number(const std::string& key, double def) const;
    bool get_bool(const std::string& key, bool def) const;
    std::string get_string(const std::string& key, const std::string& def) const;

private:
    friend class JsonReader;
    Type type_ = Null;
    bool b_ = false;
    double n_ = 0.0;
    std::string s_;
    std::vector<JsonValue> a_;
    std::shared_ptr<std::map<std::string, JsonValue>> o_;
};

}  // namespace cudasep
