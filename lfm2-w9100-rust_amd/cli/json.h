// json.h -- JSON for the command-line drivers: compact output with keys in the
// order they are added, and a strict parser for one request line.
//
// Output follows serde_json's compact form as the reference's binaries print it
// (insertion-ordered objects, no spaces, finite f64 in the shortest round-trip
// digits laid out as the ryu crate does, non-finite as null, strings escaped
// with \" \\ \b \f \n \r \t and \u00xx for other control characters).
#pragma once

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace lfmjson {

inline std::string str(const std::string &s)
{
    static const char hex[] = "0123456789abcdef";
    std::string o;
    o.reserve(s.size() + 2);
    o += '"';
    for (unsigned char c : s) {
        switch (c) {
        case '"': o += "\\\""; break;
        case '\\': o += "\\\\"; break;
        case '\b': o += "\\b"; break;
        case '\f': o += "\\f"; break;
        case '\n': o += "\\n"; break;
        case '\r': o += "\\r"; break;
        case '\t': o += "\\t"; break;
        default:
            if (c < 0x20) {
                o += "\\u00";
                o += hex[c >> 4];
                o += hex[c & 15];
            } else {
                o += (char)c;
            }
        }
    }
    o += '"';
    return o;
}

// Shortest round-trip digits of v written as 0.D x 10^kk: plain decimal when
// -5 < kk <= 16 (an integral value gets ".0"), otherwise d.ddde<kk-1>.
inline std::string num(double v)
{
    if (!std::isfinite(v))
        return "null";
    if (v == 0)
        return std::signbit(v) ? "-0.0" : "0.0";
    char b[64];
    auto r = std::to_chars(b, b + sizeof(b) - 1, v, std::chars_format::scientific);
    *r.ptr = 0;
    std::string s(b), o;
    if (s[0] == '-') {
        o += '-';
        s.erase(0, 1);
    }
    const size_t e = s.find('e');
    std::string digits = s.substr(0, e);
    digits.erase(std::remove(digits.begin(), digits.end(), '.'), digits.end());
    const int length = (int)digits.size();
    const int kk = atoi(s.c_str() + e + 1) + 1;
    const int k = kk - length;
    if (k >= 0 && kk <= 16) {
        o += digits;
        o.append((size_t)k, '0');
        o += ".0";
    } else if (kk > 0 && kk <= 16) {
        o += digits.substr(0, (size_t)kk);
        o += '.';
        o += digits.substr((size_t)kk);
    } else if (kk > -5 && kk <= 0) {
        o += "0.";
        o.append((size_t)-kk, '0');
        o += digits;
    } else {
        o += digits[0];
        if (length > 1) {
            o += '.';
            o += digits.substr(1);
        }
        o += 'e';
        o += std::to_string(kk - 1);
    }
    return o;
}

inline std::string ids(const std::vector<uint32_t> &v)
{
    std::string o = "[";
    for (size_t i = 0; i < v.size(); ++i) {
        if (i)
            o += ',';
        o += std::to_string(v[i]);
    }
    return o + "]";
}

// An object whose keys print in the order they are added.
class Obj {
  public:
    Obj &raw(const char *key, const std::string &json)
    {
        if (!body_.empty())
            body_ += ',';
        body_ += str(key);
        body_ += ':';
        body_ += json;
        return *this;
    }
    Obj &s(const char *key, const std::string &v) { return raw(key, str(v)); }
    Obj &u(const char *key, uint64_t v) { return raw(key, std::to_string(v)); }
    Obj &f(const char *key, double v) { return raw(key, num(v)); }
    Obj &b(const char *key, bool v) { return raw(key, v ? "true" : "false"); }
    Obj &null(const char *key) { return raw(key, "null"); }
    Obj &list(const char *key, const std::vector<uint32_t> &v) { return raw(key, ids(v)); }
    std::string text() const { return "{" + body_ + "}"; }

  private:
    std::string body_;
};

// One line of output, flushed (each event is visible as soon as it happens).
inline void emit(FILE *f, const Obj &o)
{
    const std::string t = o.text();
    fwrite(t.data(), 1, t.size(), f);
    fputc('\n', f);
    fflush(f);
}

// ---------------------------------------------------------------- parser
struct Val {
    enum Kind { Null, Bool, Num, Str, Arr, Object } kind = Null;
    bool b = false;
    bool integer = false;  // Num without fraction or exponent
    std::string text;      // Num: the literal; Str: the decoded UTF-8
    std::vector<Val> arr;
    std::vector<std::pair<std::string, Val>> obj;
};

inline const char *kind_name(const Val &v)
{
    switch (v.kind) {
    case Val::Null: return "null";
    case Val::Bool: return "boolean";
    case Val::Num: return v.integer ? "integer" : "floating point";
    case Val::Str: return "string";
    case Val::Arr: return "sequence";
    default: return "map";
    }
}

// RFC 8259 JSON, one value with optional surrounding whitespace; nesting is
// limited to 128 levels, as serde_json's default recursion limit.
class Parser {
  public:
    explicit Parser(const std::string &s) : s_(s) {}

    bool parse(Val *out, std::string *err)
    {
        ws();
        if (!value(out, 0)) {
            *err = err_;
            return false;
        }
        ws();
        if (i_ != s_.size()) {
            *err = "trailing characters at column " + std::to_string(i_ + 1);
            return false;
        }
        return true;
    }

  private:
    bool bad(const char *what)
    {
        err_ = std::string(what) + " at column " + std::to_string(i_ + 1);
        return false;
    }
    void ws()
    {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r'))
            ++i_;
    }
    bool lit(const char *w)
    {
        const size_t n = strlen_(w);
        if (s_.compare(i_, n, w) != 0)
            return bad("expected value");
        i_ += n;
        return true;
    }
    static size_t strlen_(const char *w)
    {
        size_t n = 0;
        while (w[n])
            ++n;
        return n;
    }
    bool value(Val *v, int depth)
    {
        if (i_ >= s_.size())
            return bad("EOF while parsing a value");
        const char c = s_[i_];
        if (c == 'n') {
            v->kind = Val::Null;
            return lit("null");
        }
        if (c == 't') {
            v->kind = Val::Bool;
            v->b = true;
            return lit("true");
        }
        if (c == 'f') {
            v->kind = Val::Bool;
            return lit("false");
        }
        if (c == '"') {
            v->kind = Val::Str;
            return string(&v->text);
        }
        if (c == '-' || (c >= '0' && c <= '9'))
            return number(v);
        if (c == '[' || c == '{') {
            if (depth >= 128)
                return bad("recursion limit exceeded");
            ++i_;
            ws();
            const char close = c == '[' ? ']' : '}';
            v->kind = c == '[' ? Val::Arr : Val::Object;
            if (i_ < s_.size() && s_[i_] == close) {
                ++i_;
                return true;
            }
            for (;;) {
                if (c == '[') {
                    v->arr.emplace_back();
                    if (!value(&v->arr.back(), depth + 1))
                        return false;
                } else {
                    if (i_ >= s_.size() || s_[i_] != '"')
                        return bad("key must be a string");
                    std::string key;
                    if (!string(&key))
                        return false;
                    ws();
                    if (i_ >= s_.size() || s_[i_] != ':')
                        return bad("expected `:`");
                    ++i_;
                    ws();
                    v->obj.emplace_back(std::move(key), Val());
                    if (!value(&v->obj.back().second, depth + 1))
                        return false;
                }
                ws();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    ws();
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == close) {
                    ++i_;
                    return true;
                }
                return bad(c == '[' ? "expected `,` or `]`" : "expected `,` or `}`");
            }
        }
        return bad("expected value");
    }
    bool digits()
    {
        const size_t start = i_;
        while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9')
            ++i_;
        return i_ > start;
    }
    bool number(Val *v)
    {
        const size_t start = i_;
        v->kind = Val::Num;
        v->integer = true;
        if (s_[i_] == '-')
            ++i_;
        if (i_ < s_.size() && s_[i_] == '0')
            ++i_;
        else if (!digits())
            return bad("invalid number");
        if (i_ < s_.size() && s_[i_] == '.') {
            ++i_;
            v->integer = false;
            if (!digits())
                return bad("invalid number");
        }
        if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
            ++i_;
            v->integer = false;
            if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-'))
                ++i_;
            if (!digits())
                return bad("invalid number");
        }
        v->text = s_.substr(start, i_ - start);
        return true;
    }
    bool hex4(uint32_t *u)
    {
        if (s_.size() - i_ < 4)
            return bad("EOF while parsing a string");
        *u = 0;
        for (int k = 0; k < 4; ++k) {
            const char h = s_[i_++];
            *u <<= 4;
            if (h >= '0' && h <= '9')
                *u |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f')
                *u |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F')
                *u |= (uint32_t)(h - 'A' + 10);
            else
                return bad("invalid escape");
        }
        return true;
    }
    static void utf8(std::string *o, uint32_t cp)
    {
        if (cp < 0x80) {
            *o += (char)cp;
        } else if (cp < 0x800) {
            *o += (char)(0xC0 | cp >> 6);
            *o += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            *o += (char)(0xE0 | cp >> 12);
            *o += (char)(0x80 | (cp >> 6 & 0x3F));
            *o += (char)(0x80 | (cp & 0x3F));
        } else {
            *o += (char)(0xF0 | cp >> 18);
            *o += (char)(0x80 | (cp >> 12 & 0x3F));
            *o += (char)(0x80 | (cp >> 6 & 0x3F));
            *o += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool string(std::string *o)
    {
        ++i_; // opening quote
        for (;;) {
            if (i_ >= s_.size())
                return bad("EOF while parsing a string");
            const unsigned char c = (unsigned char)s_[i_++];
            if (c == '"')
                return true;
            if (c < 0x20)
                return bad("control character while parsing a string");
            if (c != '\\') {
                *o += (char)c;
                continue;
            }
            if (i_ >= s_.size())
                return bad("EOF while parsing a string");
            const char e = s_[i_++];
            switch (e) {
            case '"': *o += '"'; break;
            case '\\': *o += '\\'; break;
            case '/': *o += '/'; break;
            case 'b': *o += '\b'; break;
            case 'f': *o += '\f'; break;
            case 'n': *o += '\n'; break;
            case 'r': *o += '\r'; break;
            case 't': *o += '\t'; break;
            case 'u': {
                uint32_t u = 0;
                if (!hex4(&u))
                    return false;
                if (u >= 0xDC00 && u <= 0xDFFF)
                    return bad("lone trailing surrogate");
                if (u >= 0xD800 && u <= 0xDBFF) {
                    uint32_t lo = 0;
                    if (s_.compare(i_, 2, "\\u") != 0)
                        return bad("lone leading surrogate");
                    i_ += 2;
                    if (!hex4(&lo))
                        return false;
                    if (lo < 0xDC00 || lo > 0xDFFF)
                        return bad("lone leading surrogate");
                    u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(o, u);
                break;
            }
            default:
                return bad("invalid escape");
            }
        }
    }

    const std::string &s_;
    size_t i_ = 0;
    std::string err_;
};

// An unsigned integer literal within [0, max]; false for anything else.
inline bool to_unsigned(const Val &v, uint64_t max, uint64_t *out)
{
    if (v.kind != Val::Num || !v.integer || v.text[0] == '-')
        return false;
    uint64_t x = 0;
    auto r = std::from_chars(v.text.data(), v.text.data() + v.text.size(), x);
    if (r.ec != std::errc() || x > max)
        return false;
    *out = x;
    return true;
}

} // namespace lfmjson
