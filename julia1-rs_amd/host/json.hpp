// JSON reader (RFC 8259 grammar) for checkpoint configs, safetensors headers
// and request documents: objects keep insertion order (a repeated key keeps
// its first position and takes the last value, as Python dicts and
// serde_json's preserve_order maps do), arrays, strings (\uXXXX escapes with
// surrogate pairs), numbers (the literal text, its double value and an "is
// integer" flag), true/false/null.  Nesting is limited to 128 levels.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace jh {

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    bool integral = false;  // number written without fraction/exponent
    std::string raw;        // number: the literal text
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    bool is_uint() const { return kind == Number && integral && num >= 0; }
    // The exact value of a non-negative integer literal, from its text (the
    // double loses precision above 2^53); false if it is not one or exceeds 2^64 - 1.
    bool as_u64(uint64_t& out) const {
        if (!is_uint() || raw.empty() || raw[0] == '-') return false;
        uint64_t v = 0;
        for (char ch : raw) {
            if (ch < '0' || ch > '9') return false;
            const uint64_t d = (uint64_t)(ch - '0');
            if (v > (UINT64_MAX - d) / 10) return false;
            v = v * 10 + d;
        }
        out = v;
        return true;
    }
};

class JsonParser {
public:
    explicit JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}
    Json parse() {
        Json v = value();
        ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;

    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("invalid JSON: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s) {
        size_t n = std::char_traits<char>::length(s);
        if ((size_t)(end_ - p_) >= n && std::char_traits<char>::compare(p_, s, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    int depth_ = 0;
    struct Nest {
        int& d;
        explicit Nest(JsonParser& p) : d(p.depth_) {
            if (++d > 128) throw std::runtime_error("invalid JSON: recursion limit exceeded");
        }
        ~Nest() { --d; }
    };
    Json value() {
        ws();
        if (p_ >= end_) fail("unexpected end");
        Json v;
        char c = *p_;
        if (c == '{' || c == '[') {
            Nest n(*this);
            return container(c);
        }
        if (c == '"') {
            v.kind = Json::String;
            v.str = string();
            return v;
        }
        if (lit("true")) { v.kind = Json::Bool; v.b = true; return v; }
        if (lit("false")) { v.kind = Json::Bool; v.b = false; return v; }
        if (lit("null")) return v;
        return number();
    }
    Json container(char c) {
        Json v;
        if (c == '{') {
            ++p_;
            v.kind = Json::Object;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; return v; }
            for (;;) {
                ws();
                if (p_ >= end_ || *p_ != '"') fail("expected key");
                std::string k = string();
                ws();
                if (p_ >= end_ || *p_ != ':') fail("expected ':'");
                ++p_;
                Json item = value();
                bool seen = false;
                for (auto& kv : v.obj)
                    if (kv.first == k) { kv.second = std::move(item); seen = true; break; }
                if (!seen) v.obj.emplace_back(std::move(k), std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return v; }
                fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Json::Array;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return v; }
                fail("expected ',' or ']'");
            }
        }
        fail("bad value");
    }
    bool digit() const { return p_ < end_ && *p_ >= '0' && *p_ <= '9'; }
    // -? (0 | [1-9][0-9]*) (. [0-9]+)? ([eE] [+-]? [0-9]+)?
    Json number() {
        const char* s = p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (!digit()) fail("bad value");
        if (*p_ == '0') {
            ++p_;
            if (digit()) fail("leading zero");
        } else {
            while (digit()) ++p_;
        }
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (!digit()) fail("bad number");
            while (digit()) ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (!digit()) fail("bad number");
            while (digit()) ++p_;
        }
        Json v;
        v.kind = Json::Number;
        v.raw.assign(s, p_);
        v.num = std::strtod(v.raw.c_str(), nullptr);  // out of range -> +-inf or 0, like a parsed Python float
        v.integral = integral;
        return v;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
        } else {
            o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F));
            o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("bad \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        ++p_;  // opening quote
        std::string o;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') { o += c; continue; }
            if (p_ >= end_) fail("bad escape");
            char e = *p_++;
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
                    uint32_t cp = hex4();
                    if (cp >= 0xDC00 && cp < 0xE000) fail("lone trailing surrogate");
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') fail("lone leading surrogate");
                        p_ += 2;
                        uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) fail("lone leading surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        if (p_ >= end_) fail("unterminated string");
        ++p_;
        return o;
    }
};

inline Json parse_json(const std::string& s) { return JsonParser(s.data(), s.size()).parse(); }

}  // namespace jh
