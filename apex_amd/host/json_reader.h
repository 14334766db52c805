// A small JSON reader for the packed model's manifest.json: objects, arrays, strings
// (with \" \\ \/ \b \f \n \r \t and \uXXXX escapes, BMP code points as UTF-8),
// numbers, true, false, null.  Errors throw std::runtime_error with the byte offset.
#pragma once
#include <cctype>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace apex {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    const Value &at(const std::string &key) const {
        if (kind != Object)
            throw std::runtime_error("json: not an object (looking for \"" + key + "\")");
        auto it = obj.find(key);
        if (it == obj.end())
            throw std::runtime_error("json: missing key \"" + key + "\"");
        return it->second;
    }
    const Value &at(size_t i) const {
        if (kind != Array || i >= arr.size())
            throw std::runtime_error("json: array index out of range");
        return arr[i];
    }
    bool contains(const std::string &key) const { return kind == Object && obj.count(key); }
    double number() const {
        if (kind != Number)
            throw std::runtime_error("json: not a number");
        return num;
    }
    int64_t integer() const {
        const double v = number();
        if (v != (double)(int64_t)v)
            throw std::runtime_error("json: not an integer");
        return (int64_t)v;
    }
    bool boolean() const {
        if (kind != Bool)
            throw std::runtime_error("json: not a boolean");
        return b;
    }
    const std::string &string() const {
        if (kind != String)
            throw std::runtime_error("json: not a string");
        return str;
    }
    const std::vector<Value> &array() const {
        if (kind != Array)
            throw std::runtime_error("json: not an array");
        return arr;
    }
};

class Reader {
  public:
    explicit Reader(const std::string &text) : s_(text) {}

    Value parse() {
        Value v = value();
        space();
        if (i_ != s_.size())
            error("trailing characters");
        return v;
    }

  private:
    const std::string &s_;
    size_t i_ = 0;

    [[noreturn]] void error(const std::string &what) const {
        throw std::runtime_error("json: " + what + " at byte " + std::to_string(i_));
    }
    void space() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t'))
            ++i_;
    }
    bool take(char c) {
        space();
        if (i_ < s_.size() && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!take(c))
            error(std::string("expected '") + c + "'");
    }
    bool word(const char *w) {
        const size_t n = std::char_traits<char>::length(w);
        if (s_.compare(i_, n, w) == 0) {
            i_ += n;
            return true;
        }
        return false;
    }

    Value value() {
        space();
        if (i_ >= s_.size())
            error("unexpected end");
        Value v;
        const char c = s_[i_];
        if (c == '{') {
            ++i_;
            v.kind = Value::Object;
            if (take('}'))
                return v;
            do {
                space();
                std::string key = string_body();
                expect(':');
                v.obj[key] = value();
            } while (take(','));
            expect('}');
        } else if (c == '[') {
            ++i_;
            v.kind = Value::Array;
            if (take(']'))
                return v;
            do
                v.arr.push_back(value());
            while (take(','));
            expect(']');
        } else if (c == '"') {
            v.kind = Value::String;
            v.str = string_body();
        } else if (word("true")) {
            v.kind = Value::Bool;
            v.b = true;
        } else if (word("false")) {
            v.kind = Value::Bool;
        } else if (word("null")) {
            v.kind = Value::Null;
        } else {
            v.kind = Value::Number;
            v.num = number_body();
        }
        return v;
    }

    double number_body() {
        const size_t start = i_;
        if (i_ < s_.size() && (s_[i_] == '-' || s_[i_] == '+'))
            ++i_;
        while (i_ < s_.size() && (std::isdigit((unsigned char)s_[i_]) || s_[i_] == '.' ||
                                  s_[i_] == 'e' || s_[i_] == 'E' || s_[i_] == '-' || s_[i_] == '+'))
            ++i_;
        if (i_ == start)
            error("expected a value");
        size_t used = 0;
        const std::string tok = s_.substr(start, i_ - start);
        double d = 0.0;
        try {
            d = std::stod(tok, &used);
        } catch (const std::exception &) {
            error("bad number");
        }
        if (used != tok.size())
            error("bad number");
        return d;
    }

    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }

    std::string string_body() {
        if (i_ >= s_.size() || s_[i_] != '"')
            error("expected a string");
        ++i_;
        std::string out;
        while (true) {
            if (i_ >= s_.size())
                error("unterminated string");
            const char c = s_[i_++];
            if (c == '"')
                return out;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= s_.size())
                error("unterminated escape");
            const char e = s_[i_++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                if (i_ + 4 > s_.size())
                    error("bad \\u escape");
                uint32_t cp = 0;
                for (int k = 0; k < 4; ++k) {
                    const char h = s_[i_++];
                    cp <<= 4;
                    if (h >= '0' && h <= '9')
                        cp |= (uint32_t)(h - '0');
                    else if (h >= 'a' && h <= 'f')
                        cp |= (uint32_t)(h - 'a' + 10);
                    else if (h >= 'A' && h <= 'F')
                        cp |= (uint32_t)(h - 'A' + 10);
                    else
                        error("bad \\u escape");
                }
                utf8(out, cp);
                break;
            }
            default: error("bad escape");
            }
        }
    }
};

inline Value parse(const std::string &text) { return Reader(text).parse(); }

} // namespace json
} // namespace apex
