// A small JSON reader for the files a checkpoint directory holds: safetensors
// headers, config.json, the qpack layout.json and manifest.json.  Strict
// grammar (RFC 8259) without extensions; a malformed document returns false
// instead of throwing.  Numbers keep both their double value and, when they
// are written without fraction or exponent, their exact int64.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace swq {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    int64_t i = 0;
    bool integral = false;
    std::string s;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    const Value *get(const std::string &key) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(key);
        return it == obj.end() ? nullptr : &it->second;
    }
    bool is_int() const { return kind == Number && integral; }
};

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Value &out) {
        skip_ws();
        if (!value(out, 0)) return false;
        skip_ws();
        return p_ == end_;
    }

  private:
    static constexpr int kMaxDepth = 64;
    const char *p_, *end_;

    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const char *q = p_;
        for (; *w; ++w, ++q)
            if (q >= end_ || *q != *w) return false;
        p_ = q;
        return true;
    }

    bool value(Value &v, int depth) {
        if (p_ >= end_ || depth > kMaxDepth) return false;
        switch (*p_) {
            case '{': return object(v, depth);
            case '[': return array(v, depth);
            case '"': v.kind = Value::String; return string(v.s);
            case 't': v.kind = Value::Bool; v.b = true; return lit("true");
            case 'f': v.kind = Value::Bool; v.b = false; return lit("false");
            case 'n': v.kind = Value::Null; return lit("null");
            default: return number(v);
        }
    }

    bool object(Value &v, int depth) {
        v.kind = Value::Object;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == '}') {
            ++p_;
            return true;
        }
        for (;;) {
            skip_ws();
            std::string key;
            if (p_ >= end_ || *p_ != '"' || !string(key)) return false;
            skip_ws();
            if (p_ >= end_ || *p_ != ':') return false;
            ++p_;
            skip_ws();
            Value item;
            if (!value(item, depth + 1)) return false;
            v.obj[key] = std::move(item);
            skip_ws();
            if (p_ >= end_) return false;
            if (*p_ == ',') {
                ++p_;
                continue;
            }
            if (*p_ == '}') {
                ++p_;
                return true;
            }
            return false;
        }
    }

    bool array(Value &v, int depth) {
        v.kind = Value::Array;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == ']') {
            ++p_;
            return true;
        }
        for (;;) {
            skip_ws();
            Value item;
            if (!value(item, depth + 1)) return false;
            v.arr.push_back(std::move(item));
            skip_ws();
            if (p_ >= end_) return false;
            if (*p_ == ',') {
                ++p_;
                continue;
            }
            if (*p_ == ']') {
                ++p_;
                return true;
            }
            return false;
        }
    }

    static int hex(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    bool hex4(uint32_t &u) {
        if (end_ - p_ < 4) return false;
        u = 0;
        for (int k = 0; k < 4; ++k) {
            const int h = hex(p_[k]);
            if (h < 0) return false;
            u = u * 16 + static_cast<uint32_t>(h);
        }
        p_ += 4;
        return true;
    }
    static void utf8(std::string &s, uint32_t cp) {
        if (cp < 0x80) {
            s += static_cast<char>(cp);
        } else if (cp < 0x800) {
            s += static_cast<char>(0xC0 | (cp >> 6));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += static_cast<char>(0xE0 | (cp >> 12));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            s += static_cast<char>(0xF0 | (cp >> 18));
            s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }

    bool string(std::string &s) {
        ++p_;  // opening quote
        s.clear();
        while (p_ < end_) {
            const char c = *p_++;
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
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
                    uint32_t u;
                    if (!hex4(u)) return false;
                    if (u >= 0xD800 && u < 0xDC00) {  // a surrogate pair
                        uint32_t lo;
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return false;
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (u >= 0xDC00 && u < 0xE000) {
                        return false;
                    }
                    utf8(s, u);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }

    bool number(Value &v) {
        const char *start = p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_) return false;
        if (*p_ == '0') {
            ++p_;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        } else {
            return false;
        }
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string text(start, p_);
        v.kind = Value::Number;
        v.num = std::strtod(text.c_str(), nullptr);
        v.integral = false;
        if (integral && text.size() <= 18) {  // at most 18 digits: always within int64
            v.i = std::strtoll(text.c_str(), nullptr, 10);
            v.integral = true;
        }
        return true;
    }
};

inline bool parse(const std::string &text, Value &out) { return Parser(text.data(), text.size()).parse(out); }

}  // namespace json
}  // namespace swq
