// json.cpp — recursive-descent JSON reader (RFC 8259 subset the configs use:
// no surrogate-pair decoding beyond the BMP).
#include "json.h"

#include <cmath>
#include <cstdlib>
#include <stdexcept>

namespace cudasep {

class JsonReader {
public:
    explicit JsonReader(const std::string& t) : t_(t) {}

    JsonValue document() {
        JsonValue v = value();
        ws();
        if (i_ != t_.size()) fail("trailing characters");
        return v;
    }

private:
    const std::string& t_;
    size_t i_ = 0;

    [[noreturn]] void fail(const std::string& what) {
        throw std::runtime_error("JSON: " + what + " at offset " + std::to_string(i_));
    }
    void ws() {
        while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r'))
            ++i_;
    }
    char peek() {
        ws();
        if (i_ >= t_.size()) fail("unexpected end");
        return t_[i_];
    }
    void expect(char c) {
        if (peek() != c) fail(std::string("expected '") + c + "'");
        ++i_;
    }
    bool literal(const char* w) {
        size_t n = 0;
        while (w[n]) ++n;
        if (t_.compare(i_, n, w) == 0) {
            i_ += n;
            return true;
        }
        return false;
    }

    JsonValue value() {
        const char c = peek();
        JsonValue v;
        if (c == '{') return object();
        if (c == '[') return array();
        if (c == '"') {
            v.type_ = JsonValue::String;
            v.s_ = string();
            return v;
        }
        if (literal("true")) {
            v.type_ = JsonValue::Bool;
            v.b_ = true;
            return v;
        }
        if (literal("false")) {
            v.type_ = JsonValue::Bool;
            return v;
        }
        if (literal("null")) return v;
        return number();
    }

    JsonValue number() {
        const char* begin = t_.c_str() + i_;
        char* end = nullptr;
        const double d = std::strtod(begin, &end);
        if (end == begin) fail("bad value");
        i_ += (size_t)(end - begin);
        JsonValue v;
        v.type_ = JsonValue::Number;
        v.n_ = d;
        return v;
    }

    static void put_utf8(std::string& s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }

    std::string string() {
        expect('"');
        std::string s;
        while (true) {
            if (i_ >= t_.size()) fail("unterminated string");
            const char c = t_[i_++];
            if (c == '"') break;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (i_ >= t_.size()) fail("bad escape");
            const char e = t_[i_++];
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    if (i_ + 4 > t_.size()) fail("bad \\u escape");
                    put_utf8(s, (unsigned)std::strtoul(t_.substr(i_, 4).c_str(), nullptr, 16));
                    i_ += 4;
                    break;
                }
                default: fail("bad escape");
            }
        }
        return s;
    }

    JsonValue array() {
        expect('[');
        JsonValue v;
        v.type_ = JsonValue::Array;
        if (peek() == ']') {
            ++i_;
            return v;
        }
        while (true) {
            v.a_.push_back(value());
            if (peek() == ']') {
                ++i_;
                return v;
            }
            expect(',');
        }
    }

    JsonValue object() {
        expect('{');
        JsonValue v;
        v.type_ = JsonValue::Object;
        v.o_ = std::make_shared<std::map<std::string, JsonValue>>();
        if (peek() == '}') {
            ++i_;
            return v;
        }
        while (true) {
            if (peek() != '"') fail("expected a key");
            std::string k = string();
            expect(':');
            (*v.o_)[k] = value();
            if (peek() == '}') {
                ++i_;
                return v;
            }
            expect(',');
        }
    }
};

JsonValue JsonValue::parse(const std::string& text) { return JsonReader(text).document(); }

bool JsonValue::as_bool() const {
    if (type_ == Bool) return b_;
    if (type_ == Number) return n_ != 0.0;
    throw std::runtime_error("JSON: not a bool");
}

double JsonValue::as_number() const {
    if (type_ == Number) return n_;
    if (type_ == Bool) return b_ ? 1.0 : 0.0;
    throw std::runtime_error("JSON: not a number");
}

const std::string& JsonValue::as_string() const {
    if (type_ != String) throw std::runtime_error("JSON: not a string");
    return s_;
}

size_t JsonValue::size() const {
    if (type_ == Array) return a_.size();
    if (type_ == Object) return o_->size();
    throw std::runtime_error("JSON: size() of a scalar");
}

const JsonValue& JsonValue::operator[](size_t i) const {
    if (type_ != Array) throw std::runtime_error("JSON: not an array");
    if (i >= a_.size()) throw std::runtime_error("JSON: index out of range");
    return a_[i];
}

const JsonValue& JsonValue::operator[](const std::string& key) const {
    if (type_ != Object) throw std::runtime_error("JSON: not an object");
    auto it = o_->find(key);
    if (it == o_->end()) throw std::runtime_error("JSON: key not found: " + key);
    return it->second;
}

bool JsonValue::has(const std::string& key) const {
    return type_ == Object && o_->count(key) != 0;
}

int JsonValue::get_int(const std::string& key, int def) const {
    return has(key) && !(*this)[key].is_null() ? (int)std::lround((*this)[key].as_number()) : def;
}

double JsonValue::get_number(const std::string& key, double def) const {
    return has(key) && !(*this)[key].is_null() ? (*this)[key].as_number() : def;
}

bool JsonValue::get_bool(const std::string& key, bool def) const {
    return has(key) && !(*this)[key].is_null() ? (*this)[key].as_bool() : def;
}

std::string JsonValue::get_string(const std::string& key, const std::string& def) const {
    return has(key) && (*this)[key].type() == String ? (*this)[key].as_string() : def;
}

}  // namespace cudasep
