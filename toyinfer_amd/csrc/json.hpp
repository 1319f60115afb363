// Minimal JSON reader for the model files the loader parses: config.json,
// model.safetensors.index.json and the safetensors headers.  A recursive
// descent over RFC 8259 values; numbers are kept as double (exact for the
// integer offsets and sizes of any file under 2^53 bytes) together with
// their text.  Host code only.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace tijson {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;  // String, or the literal text of a Number
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    const Value* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    // A non-negative integer that fits in 64 bits, written without fraction or exponent.
    bool as_u64(uint64_t& out) const {
        if (kind != Number || str.empty() || str[0] == '-') return false;
        for (char c : str)
            if (c < '0' || c > '9') return false;
        if (str.size() > 19) return false;
        out = std::strtoull(str.c_str(), nullptr, 10);
        return true;
    }
};

class Parser {
   public:
    Parser(const char* p, const char* e) : p_(p), e_(e) {}

    bool parse(Value& v) {
        if (!value(v, 0)) return false;
        ws();
        return p_ == e_;
    }

   private:
    const char* p_;
    const char* e_;

    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s) {
        const char* q = p_;
        for (; *s; ++s, ++q)
            if (q >= e_ || *q != *s) return false;
        p_ = q;
        return true;
    }
    static void utf8(uint32_t c, std::string& out) {
        if (c < 0x80) {
            out.push_back((char)c);
        } else if (c < 0x800) {
            out.push_back((char)(0xC0 | c >> 6));
            out.push_back((char)(0x80 | (c & 0x3F)));
        } else if (c < 0x10000) {
            out.push_back((char)(0xE0 | c >> 12));
            out.push_back((char)(0x80 | (c >> 6 & 0x3F)));
            out.push_back((char)(0x80 | (c & 0x3F)));
        } else {
            out.push_back((char)(0xF0 | c >> 18));
            out.push_back((char)(0x80 | (c >> 12 & 0x3F)));
            out.push_back((char)(0x80 | (c >> 6 & 0x3F)));
            out.push_back((char)(0x80 | (c & 0x3F)));
        }
    }
    bool hex4(uint32_t& c) {
        if (e_ - p_ < 4) return false;
        c = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= h - '0';
            else if (h >= 'a' && h <= 'f') c |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') c |= h - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool string(std::string& out) {
        if (p_ >= e_ || *p_ != '"') return false;
        ++p_;
        while (p_ < e_ && *p_ != '"') {
            const char c = *p_++;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= e_) return false;
            const char x = *p_++;
            switch (x) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    uint32_t u;
                    if (!hex4(u)) return false;
                    if (u >= 0xD800 && u < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (u >= 0xDC00 && u < 0xE000) {
                        return false;
                    }
                    utf8(u, out);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= e_) return false;
        ++p_;
        return true;
    }
    bool number(Value& v) {
        const char* s = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return false;
        if (*p_ == '0') ++p_;
        else
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < e_ && *p_ == '.') {
            ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.kind = Value::Number;
        v.str.assign(s, p_);
        v.num = std::strtod(v.str.c_str(), nullptr);
        return true;
    }
    bool value(Value& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= e_) return false;
        switch (*p_) {
            case '{': {
                ++p_;
                v.kind = Value::Object;
                ws();
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                for (;;) {
                    ws();
                    std::pair<std::string, Value> kv;
                    if (!string(kv.first)) return false;
                    ws();
                    if (p_ >= e_ || *p_++ != ':') return false;
                    if (!value(kv.second, depth + 1)) return false;
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (p_ >= e_) return false;
                    if (*p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (*p_++ != '}') return false;
                    return true;
                }
            }
            case '[': {
                ++p_;
                v.kind = Value::Array;
                ws();
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                for (;;) {
                    v.arr.emplace_back();
                    if (!value(v.arr.back(), depth + 1)) return false;
                    ws();
                    if (p_ >= e_) return false;
                    if (*p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (*p_++ != ']') return false;
                    return true;
                }
            }
            case '"': v.kind = Value::String; return string(v.str);
            case 't': v.kind = Value::Bool; v.b = true; return lit("true");
            case 'f': v.kind = Value::Bool; v.b = false; return lit("false");
            case 'n': v.kind = Value::Null; return lit("null");
            default: return number(v);
        }
    }
};

inline bool parse(const std::string& text, Value& out) {
    Parser p(text.data(), text.data() + text.size());
    return p.parse(out);
}

}  // namespace tijson
