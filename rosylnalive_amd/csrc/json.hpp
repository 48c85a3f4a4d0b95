// A strict JSON reader for the small documents the library reads (safetensors headers): RFC 8259 text in UTF-8, no
// comments or trailing commas, a nesting limit, strings decoded to UTF-8 with their escapes checked (a lone surrogate
// escape is an error), numbers kept as their text. Object members stay in document order with duplicates kept, so a
// caller decides what a repeated key means.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace lrm {
namespace json {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

enum class Kind { Null, Bool, Number, String, Array, Object };

struct Value {
    Kind kind = Kind::Null;
    bool boolean = false;
    std::string text;  // String: the decoded UTF-8; Number: the number's text as written
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;
};

// Strict UTF-8 (the Unicode standard's well-formed sequences): no overlong forms, no encoded surrogates, nothing above
// U+10FFFF, no truncated sequence.
inline bool utf8_valid(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint8_t lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) {
            len = 2;
        } else if (c >= 0xE0 && c <= 0xEF) {
            len = 3;
            if (c == 0xE0) lo = 0xA0;
            if (c == 0xED) hi = 0x9F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            len = 4;
            if (c == 0xF0) lo = 0x90;
            if (c == 0xF4) hi = 0x8F;
        } else {
            return false;
        }
        if (i + size_t(len) > n) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (int k = 2; k < len; ++k)
            if (s[i + size_t(k)] < 0x80 || s[i + size_t(k)] > 0xBF) return false;
        i += size_t(len);
    }
    return true;
}

inline void append_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out += char(cp);
    } else if (cp < 0x800) {
        out += char(0xC0 | (cp >> 6));
        out += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += char(0xE0 | (cp >> 12));
        out += char(0x80 | ((cp >> 6) & 0x3F));
        out += char(0x80 | (cp & 0x3F));
    } else {
        out += char(0xF0 | (cp >> 18));
        out += char(0x80 | ((cp >> 12) & 0x3F));
        out += char(0x80 | ((cp >> 6) & 0x3F));
        out += char(0x80 | (cp & 0x3F));
    }
}

class Parser {
  public:
    Parser(const uint8_t* s, size_t n, int max_depth) : s_(s), n_(n), max_depth_(max_depth) {}

    Value document() {
        ws();
        Value v = value(0);
        ws();
        if (i_ != n_) fail("unexpected text after the value");
        return v;
    }

  private:
    [[noreturn]] void fail(const char* what) const {
        throw Error(std::string(what) + " at byte " + std::to_string(i_));
    }
    void ws() {
        while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    bool literal(const char* w) {
        const size_t k = std::strlen(w);
        if (n_ - i_ >= k && std::memcmp(s_ + i_, w, k) == 0) {
            i_ += k;
            return true;
        }
        return false;
    }
    Value value(int depth) {
        if (i_ >= n_) fail("unexpected end of the text");
        Value v;
        const uint8_t c = s_[i_];
        if (c == '{' || c == '[') {
            if (depth + 1 > max_depth_) fail("the nesting is deeper than the limit");
            ++i_;
            ws();
            const uint8_t close = c == '{' ? '}' : ']';
            v.kind = c == '{' ? Kind::Object : Kind::Array;
            if (i_ < n_ && s_[i_] == close) {
                ++i_;
                return v;
            }
            for (;;) {
                if (v.kind == Kind::Object) {
                    if (i_ >= n_ || s_[i_] != '"') fail("expected a member name");
                    std::string key = string();
                    ws();
                    if (i_ >= n_ || s_[i_] != ':') fail("expected ':'");
                    ++i_;
                    ws();
                    v.members.emplace_back(std::move(key), value(depth + 1));
                } else {
                    v.items.push_back(value(depth + 1));
                }
                ws();
                if (i_ >= n_) fail("unexpected end of the text");
                if (s_[i_] == ',') {
                    ++i_;
                    ws();
                    continue;
                }
                if (s_[i_] == close) {
                    ++i_;
                    return v;
                }
                fail("expected ',' or the end of the container");
            }
        }
        if (c == '"') {
            v.kind = Kind::String;
            v.text = string();
            return v;
        }
        if (literal("true")) {
            v.kind = Kind::Bool;
            v.boolean = true;
            return v;
        }
        if (literal("false")) {
            v.kind = Kind::Bool;
            return v;
        }
        if (literal("null")) return v;
        if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Kind::Number;
            v.text = number();
            return v;
        }
        fail("unexpected character");
    }
    static bool digit(uint8_t c) { return c >= '0' && c <= '9'; }
    std::string number() {
        const size_t b = i_;
        if (s_[i_] == '-') ++i_;
        if (i_ >= n_ || !digit(s_[i_])) fail("a number needs digits");
        if (s_[i_] == '0') {
            ++i_;
        } else {
            while (i_ < n_ && digit(s_[i_])) ++i_;
        }
        if (i_ < n_ && s_[i_] == '.') {
            ++i_;
            if (i_ >= n_ || !digit(s_[i_])) fail("a fraction needs digits");
            while (i_ < n_ && digit(s_[i_])) ++i_;
        }
        if (i_ < n_ && (s_[i_] == 'e' || s_[i_] == 'E')) {
            ++i_;
            if (i_ < n_ && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
            if (i_ >= n_ || !digit(s_[i_])) fail("an exponent needs digits");
            while (i_ < n_ && digit(s_[i_])) ++i_;
        }
        return std::string(reinterpret_cast<const char*>(s_ + b), i_ - b);
    }
    uint32_t hex4() {
        if (n_ - i_ < 4) fail("a \\u escape needs four hex digits");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const uint8_t c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail("a \\u escape needs four hex digits");
        }
        return v;
    }
    // The input is valid UTF-8 (checked by the caller), so raw bytes copy through.
    std::string string() {
        ++i_;  // the opening quote
        std::string out;
        for (;;) {
            if (i_ >= n_) fail("unterminated string");
            const uint8_t c = s_[i_];
            if (c == '"') {
                ++i_;
                return out;
            }
            if (c < 0x20) fail("a control character in a string");
            if (c != '\\') {
                out += char(c);
                ++i_;
                continue;
            }
            ++i_;
            if (i_ >= n_) fail("unterminated escape");
            const uint8_t e = s_[i_++];
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
                    uint32_t u = hex4();
                    if (u >= 0xDC00 && u <= 0xDFFF) fail("a lone low surrogate escape (not valid Unicode)");
                    if (u >= 0xD800 && u <= 0xDBFF) {
                        if (n_ - i_ < 6 || s_[i_] != '\\' || s_[i_ + 1] != 'u')
                            fail("a high surrogate escape without its low half (not valid Unicode)");
                        i_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo > 0xDFFF)
                            fail("a high surrogate escape without its low half (not valid Unicode)");
                        u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    append_utf8(out, u);
                    break;
                }
                default: fail("an invalid escape");
            }
        }
    }

    const uint8_t* s_;
    size_t n_;
    size_t i_ = 0;
    int max_depth_;
};

// Parses a whole document; throws Error. The caller checks the bytes are valid UTF-8 first.
inline Value parse(const uint8_t* s, size_t n, int max_depth) { return Parser(s, n, max_depth).document(); }

// The value of a number written as an integer in 0 .. INT64_MAX ("-0" is 0); false for a fraction, an exponent, a
// negative value or one beyond int64.
inline bool nonnegative_int(const Value& v, int64_t* out) {
    if (v.kind != Kind::Number) return false;
    const std::string& t = v.text;
    size_t k = 0;
    const bool neg = !t.empty() && t[0] == '-';
    if (neg) k = 1;
    if (k >= t.size()) return false;
    uint64_t x = 0;
    for (; k < t.size(); ++k) {
        if (t[k] < '0' || t[k] > '9') return false;
        const uint64_t d = uint64_t(t[k] - '0');
        if (x > (uint64_t(INT64_MAX) - d) / 10) return false;
        x = x * 10 + d;
    }
    if (neg && x != 0) return false;
    *out = int64_t(x);
    return true;
}

}  // namespace json
}  // namespace lrm
