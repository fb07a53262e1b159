// json.hpp - the JSON the engine protocol needs: a value type, a strict parser for one request line and string
// escaping for events. Missing keys and wrong types read as defaults, like the reference's accessors
// (engine/src/main.cpp:562-600 reads every field with a default).
#pragma once
#include <stdint.h>
#include <stdio.h>

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace kiln::json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double n = 0.0;
    std::string s;
    std::vector<Value> a;
    std::map<std::string, Value> o;

    bool is_null() const { return kind == Null; }
    bool has(const std::string& k) const { return kind == Object && o.count(k) != 0; }
    const Value& operator[](const std::string& k) const {
        static const Value none;
        if (kind != Object) return none;
        auto it = o.find(k);
        return it == o.end() ? none : it->second;
    }
    std::string str(const std::string& def = "") const { return kind == String ? s : def; }
    double num(double def = 0.0) const { return kind == Number ? n : def; }
    int64_t i64(int64_t def = 0) const { return kind == Number ? (int64_t)n : def; }
    bool boolean(bool def = false) const { return kind == Bool ? b : def; }
    const std::vector<Value>& items() const {
        static const std::vector<Value> empty;
        return kind == Array ? a : empty;
    }
};

class Parser {
   public:
    explicit Parser(const std::string& t) : t_(t) {}
    Value parse() {
        Value v = value(0);
        ws();
        if (i_ != t_.size()) err("trailing characters");
        return v;
    }

   private:
    const std::string& t_;
    size_t i_ = 0;

    [[noreturn]] void err(const char* what) {
        throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i_));
    }
    void ws() {
        while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r')) i_++;
    }
    bool lit(const char* w) {
        size_t n = 0;
        while (w[n]) n++;
        if (t_.compare(i_, n, w) != 0) return false;
        i_ += n;
        return true;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) out += (char)(0xC0 | cp >> 6), out += (char)(0x80 | (cp & 63));
        else if (cp < 0x10000)
            out += (char)(0xE0 | cp >> 12), out += (char)(0x80 | ((cp >> 6) & 63)), out += (char)(0x80 | (cp & 63));
        else
            out += (char)(0xF0 | cp >> 18), out += (char)(0x80 | ((cp >> 12) & 63)),
                out += (char)(0x80 | ((cp >> 6) & 63)), out += (char)(0x80 | (cp & 63));
    }
    uint32_t hex4() {
        if (i_ + 4 > t_.size()) err("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = t_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else err("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        std::string out;
        i_++;  // opening quote
        for (;;) {
            if (i_ >= t_.size()) err("unterminated string");
            const char c = t_[i_++];
            if (c == '"') return out;
            if ((unsigned char)c < 0x20) err("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= t_.size()) err("unterminated escape");
            const char e = t_[i_++];
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
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && i_ + 6 <= t_.size() && t_[i_] == '\\' && t_[i_ + 1] == 'u') {
                        i_ += 2;
                        const uint32_t lo = hex4();
                        if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: err("bad escape");
            }
        }
    }
    Value value(int depth) {
        if (depth > 64) err("nesting too deep");
        ws();
        if (i_ >= t_.size()) err("unexpected end");
        Value v;
        const char c = t_[i_];
        if (c == '{') {
            v.kind = Value::Object;
            i_++;
            ws();
            if (i_ < t_.size() && t_[i_] == '}') return i_++, v;
            for (;;) {
                ws();
                if (i_ >= t_.size() || t_[i_] != '"') err("expected a key");
                std::string k = string();
                ws();
                if (i_ >= t_.size() || t_[i_] != ':') err("expected ':'");
                i_++;
                v.o[k] = value(depth + 1);
                ws();
                if (i_ < t_.size() && t_[i_] == ',') { i_++; continue; }
                if (i_ < t_.size() && t_[i_] == '}') return i_++, v;
                err("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Value::Array;
            i_++;
            ws();
            if (i_ < t_.size() && t_[i_] == ']') return i_++, v;
            for (;;) {
                v.a.push_back(value(depth + 1));
                ws();
                if (i_ < t_.size() && t_[i_] == ',') { i_++; continue; }
                if (i_ < t_.size() && t_[i_] == ']') return i_++, v;
                err("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Value::String;
            v.s = string();
            return v;
        }
        if (lit("true")) return v.kind = Value::Bool, v.b = true, v;
        if (lit("false")) return v.kind = Value::Bool, v.b = false, v;
        if (lit("null")) return v;
        // number: -? digits (. digits)? ([eE] [+-]? digits)?
        const size_t s0 = i_;
        if (t_[i_] == '-') i_++;
        if (i_ >= t_.size() || t_[i_] < '0' || t_[i_] > '9') err("unexpected character");
        while (i_ < t_.size() && ((t_[i_] >= '0' && t_[i_] <= '9') || t_[i_] == '.' || t_[i_] == 'e' || t_[i_] == 'E' ||
                                  t_[i_] == '+' || t_[i_] == '-'))
            i_++;
        v.kind = Value::Number;
        size_t used = 0;
        const std::string num = t_.substr(s0, i_ - s0);
        try {
            v.n = std::stod(num, &used);
        } catch (...) {
            err("bad number");
        }
        if (used != num.size()) err("bad number");
        return v;
    }
};

inline Value parse(const std::string& text) { return Parser(text).parse(); }

// a JSON string literal (quotes included)
inline std::string quote(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (c < 0x20) {
                    char b[8];
                    snprintf(b, sizeof b, "\\u%04x", c);
                    o += b;
                } else {
                    o += (char)c;
                }
        }
    }
    return o + "\"";
}

}  // namespace kiln::json
