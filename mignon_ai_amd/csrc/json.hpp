// Minimal JSON reader for model-file headers: objects, arrays, numbers, strings, booleans, null.
// Numbers are kept as double (every header number is an int or a float32 scale, both exact in
// double). Errors throw std::runtime_error with the byte offset.
#pragma once

#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mgjson {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    bool is_null() const { return kind == Null; }
    const Value* get(const std::string& k) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
    double number_or(const std::string& k, double dflt) const {
        const Value* v = get(k);
        return (v && v->kind == Number) ? v->num : dflt;
    }
    bool bool_or(const std::string& k, bool dflt) const {
        const Value* v = get(k);
        return (v && v->kind == Bool) ? v->b : dflt;
    }
};

class Parser {
public:
    Parser(const char* s, size_t n) : s_(s), n_(n) {}

    Value parse() {
        Value v = value();
        ws();
        if (i_ != n_) fail("trailing characters");
        return v;
    }

private:
    const char* s_;
    size_t n_, i_ = 0;

    [[noreturn]] void fail(const char* what) {
        throw std::runtime_error(std::string("invalid JSON header: ") + what + " at byte " + std::to_string(i_));
    }
    void ws() {
        while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) i_++;
    }
    bool lit(const char* w) {
        size_t k = 0;
        while (w[k]) {
            if (i_ + k >= n_ || s_[i_ + k] != w[k]) return false;
            k++;
        }
        i_ += k;
        return true;
    }
    Value value() {
        ws();
        if (i_ >= n_) fail("unexpected end");
        char c = s_[i_];
        Value v;
        if (c == '{') {
            v.kind = Value::Object;
            i_++;
            ws();
            if (i_ < n_ && s_[i_] == '}') { i_++; return v; }
            for (;;) {
                ws();
                if (i_ >= n_ || s_[i_] != '"') fail("expected key");
                std::string k = string();
                ws();
                if (i_ >= n_ || s_[i_] != ':') fail("expected ':'");
                i_++;
                v.obj[k] = value();
                ws();
                if (i_ < n_ && s_[i_] == ',') { i_++; continue; }
                if (i_ < n_ && s_[i_] == '}') { i_++; break; }
                fail("expected ',' or '}'");
            }
        } else if (c == '[') {
            v.kind = Value::Array;
            i_++;
            ws();
            if (i_ < n_ && s_[i_] == ']') { i_++; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (i_ < n_ && s_[i_] == ',') { i_++; continue; }
                if (i_ < n_ && s_[i_] == ']') { i_++; break; }
                fail("expected ',' or ']'");
            }
        } else if (c == '"') {
            v.kind = Value::String;
            v.str = string();
        } else if (lit("true")) {
            v.kind = Value::Bool; v.b = true;
        } else if (lit("false")) {
            v.kind = Value::Bool; v.b = false;
        } else if (lit("null")) {
            v.kind = Value::Null;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Value::Number;
            size_t st = i_;
            if (s_[i_] == '-') i_++;
            while (i_ < n_ && ((s_[i_] >= '0' && s_[i_] <= '9') || s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E' ||
                               s_[i_] == '+' || s_[i_] == '-'))
                i_++;
            std::string t(s_ + st, i_ - st);
            char* end = nullptr;
            v.num = std::strtod(t.c_str(), &end);
            if (!end || *end) fail("bad number");
        } else {
            fail("unexpected character");
        }
        return v;
    }
    static void put_utf8(std::string& o, unsigned cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
        } else {
            o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F));
            o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
        }
    }
    unsigned hex4() {
        if (i_ + 4 > n_) fail("bad escape");
        unsigned v = 0;
        for (int k = 0; k < 4; k++) {
            char c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail("bad escape");
        }
        return v;
    }
    std::string string() {
        i_++;  // opening quote
        std::string o;
        while (i_ < n_ && s_[i_] != '"') {
            char c = s_[i_++];
            if (c != '\\') { o += c; continue; }
            if (i_ >= n_) fail("bad escape");
            char e = s_[i_++];
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    unsigned cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && i_ + 6 <= n_ && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
                        i_ += 2;
                        unsigned lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        if (i_ >= n_) fail("unterminated string");
        i_++;
        return o;
    }
};

inline Value parse(const char* s, size_t n) { return Parser(s, n).parse(); }

}  // namespace mgjson
