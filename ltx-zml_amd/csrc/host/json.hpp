// Minimal JSON reader for blob_manifest.json (the schema of
// ltx/loader.zig:22-43): objects, arrays, strings, numbers, literals.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace ltx {
namespace json {

struct Value {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    int64_t inum = 0;  // exact integer value when the literal is integral
    bool integral = false;
    std::string str;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;  // insertion order kept

    const Value* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    const Value& at(const std::string& k) const {
        const Value* v = get(k);
        if (!v) throw std::runtime_error("manifest: missing field '" + k + "'");
        return *v;
    }
    int64_t as_int() const {
        if (kind != Num || !integral) throw std::runtime_error("manifest: expected an integer");
        return inum;
    }
    const std::string& as_str() const {
        if (kind != Str) throw std::runtime_error("manifest: expected a string");
        return str;
    }
};

class Parser {
   public:
    explicit Parser(const char* s) : p_(s) {}
    Value parse() {
        Value v = value();
        ws();
        if (*p_) fail("trailing characters");
        return v;
    }

   private:
    const char* p_;
    [[noreturn]] void fail(const char* m) { throw std::runtime_error(std::string("manifest JSON: ") + m); }
    void ws() {
        while (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t') p_++;
    }
    Value value() {
        ws();
        Value v;
        switch (*p_) {
            case '{': {
                v.kind = Value::Obj;
                p_++;
                ws();
                if (*p_ == '}') {
                    p_++;
                    return v;
                }
                for (;;) {
                    ws();
                    if (*p_ != '"') fail("expected key");
                    std::string k = string();
                    ws();
                    if (*p_++ != ':') fail("expected ':'");
                    v.obj.emplace_back(std::move(k), value());
                    ws();
                    if (*p_ == ',') {
                        p_++;
                        continue;
                    }
                    if (*p_ == '}') {
                        p_++;
                        return v;
                    }
                    fail("expected ',' or '}'");
                }
            }
            case '[': {
                v.kind = Value::Arr;
                p_++;
                ws();
                if (*p_ == ']') {
                    p_++;
                    return v;
                }
                for (;;) {
                    v.arr.push_back(value());
                    ws();
                    if (*p_ == ',') {
                        p_++;
                        continue;
                    }
                    if (*p_ == ']') {
                        p_++;
                        return v;
                    }
                    fail("expected ',' or ']'");
                }
            }
            case '"':
                v.kind = Value::Str;
                v.str = string();
                return v;
            case 't':
                lit("true");
                v.kind = Value::Bool;
                v.b = true;
                return v;
            case 'f':
                lit("false");
                v.kind = Value::Bool;
                return v;
            case 'n':
                lit("null");
                return v;
            default:
                return number();
        }
    }
    void lit(const char* w) {
        for (const char* q = w; *q; q++)
            if (*p_++ != *q) fail("bad literal");
    }
    Value number() {
        const char* s = p_;
        bool integral = true;
        if (*p_ == '-') p_++;
        if (!(*p_ >= '0' && *p_ <= '9')) fail("bad value");
        while ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' || *p_ == '-') {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') integral = false;
            p_++;
        }
        Value v;
        v.kind = Value::Num;
        std::string t(s, p_ - s);
        v.num = std::strtod(t.c_str(), nullptr);
        v.integral = integral;
        if (integral) v.inum = std::strtoll(t.c_str(), nullptr, 10);
        return v;
    }
    std::string string() {
        p_++;  // opening quote
        std::string out;
        for (;;) {
            char ch = *p_++;
            if (ch == '\0') fail("unterminated string");
            if (ch == '"') return out;
            if (ch != '\\') {
                out.push_back(ch);
                continue;
            }
            char e = *p_++;
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    unsigned cp = 0;
                    for (int i = 0; i < 4; i++) {
                        char h = *p_++;
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= h - '0';
                        else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                        else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                        else fail("bad \\u escape");
                    }
                    if (cp < 0x80) out.push_back((char)cp);
                    else if (cp < 0x800) {
                        out.push_back((char)(0xc0 | (cp >> 6)));
                        out.push_back((char)(0x80 | (cp & 0x3f)));
                    } else {
                        out.push_back((char)(0xe0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
                        out.push_back((char)(0x80 | (cp & 0x3f)));
                    }
                    break;
                }
                default: fail("bad escape");
            }
        }
    }
};

inline Value parse(const char* s) { return Parser(s).parse(); }

}  // namespace json
}  // namespace ltx
