// Text front end and callers above the engine (julia1_text.h): request rows,
// pyjson, the Encoder's marker serialization with its LRU caches, the legacy
// predict API, named typed questions and the hierarchical Router.  Each part
// restates the reference's Rust (file:line on each) in C++; the tokenizer and
// the scorer are supplied through the C-ABI.
#include <algorithm>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "../../include/julia1_engine.h"
#include "../../include/julia1_text.h"
#include "../csrc/abi_util.hpp"
#include "json.hpp"

using jh::Json;

namespace {

[[noreturn]] void invalid(const std::string& m) { throw jh_error(JH_ERR_INVALID, m); }

// ---------------------------------------------------------------- text utils

void check_utf8(const char* p, size_t n) {
    const unsigned char* s = (const unsigned char*)p;
    size_t i = 0;
    while (i < n) {
        const unsigned c = s[i];
        size_t len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!len || i + len > n) invalid("text is not valid UTF-8");
        uint32_t cp = len == 1 ? c : len == 2 ? (c & 0x1F) : len == 3 ? (c & 0x0F) : (c & 0x07);
        for (size_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) invalid("text is not valid UTF-8");
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        const uint32_t min = len == 1 ? 0 : len == 2 ? 0x80 : len == 3 ? 0x800 : 0x10000;
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) invalid("text is not valid UTF-8");
        i += len;
    }
}

Json parse(const char* p, size_t n, const std::string& what) {
    if (n && !p) invalid("null " + what);
    check_utf8(p, n);
    try {
        return jh::JsonParser(p, n).parse();
    } catch (const std::runtime_error& e) {
        invalid(what + ": " + e.what());
    }
}

std::string replace_all(const std::string& s, const std::string& from, const std::string& to) {
    if (from.empty()) return s;
    std::string out;
    size_t i = 0;
    for (;;) {
        const size_t j = s.find(from, i);
        if (j == std::string::npos) break;
        out.append(s, i, j - i);
        out += to;
        i = j + from.size();
    }
    out.append(s, i, std::string::npos);
    return out;
}

// Rust's char::is_whitespace over a UTF-8 line (str::trim().is_empty()).
bool blank(const std::string& line) {
    const unsigned char* s = (const unsigned char*)line.data();
    size_t i = 0, n = line.size();
    while (i < n) {
        const unsigned c = s[i];
        if (c == ' ' || (c >= 0x09 && c <= 0x0D)) { ++i; continue; }
        uint32_t cp;
        size_t len;
        if (c < 0x80) return false;
        if ((c >> 5) == 6) { cp = c & 0x1F; len = 2; }
        else if ((c >> 4) == 14) { cp = c & 0x0F; len = 3; }
        else { cp = c & 0x07; len = 4; }
        for (size_t k = 1; k < len && i + k < n; ++k) cp = (cp << 6) | (s[i + k] & 0x3F);
        const bool ws = cp == 0x85 || cp == 0xA0 || cp == 0x1680 || (cp >= 0x2000 && cp <= 0x200A) ||
                        cp == 0x2028 || cp == 0x2029 || cp == 0x202F || cp == 0x205F || cp == 0x3000;
        if (!ws) return false;
        i += len;
    }
    return true;
}

// Shortest decimal digits that read back to `v` (the f32 path for logits).
template <class F>
std::string shortest(F v) {
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof buf, v);
    return std::string(buf, r.ptr);
}

// JSON number for a result document: shortest round-trip digits, "x.0" for
// integral values so they read back as floats; non-finite values become null.
template <class F>
std::string json_float(F v) {
    if (!std::isfinite(v)) return "null";
    std::string s = shortest(v);
    if (s.find_first_of(".e") == std::string::npos) s += ".0";
    return s;
}

// ---------------------------------------------------------------- pyjson (src/pyjson.rs)

// float.__repr__ (src/pyjson.rs:56-99): shortest round-trip digits, fixed
// notation for decimal exponents -4 < point <= 16, else d.ddde+XX.
std::string float_repr(double v) {
    if (std::isnan(v)) return "NaN";
    if (std::isinf(v)) return v > 0 ? "Infinity" : "-Infinity";
    if (v == 0.0) return std::signbit(v) ? "-0.0" : "0.0";
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof buf, std::fabs(v), std::chars_format::scientific);
    const std::string sci(buf, r.ptr);
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = 0; i < e; ++i)
        if (sci[i] != '.') digits += sci[i];
    const int exponent = std::atoi(sci.c_str() + e + 1);
    const int point = exponent + 1;  // v = 0.DIGITS x 10^point
    const int n = (int)digits.size();
    std::string out = v < 0 ? "-" : "";
    if (-4 < point && point <= 16) {
        if (point <= 0) out += "0." + std::string(-point, '0') + digits;
        else if (point >= n) out += digits + std::string(point - n, '0') + ".0";
        else out += digits.substr(0, point) + "." + digits.substr(point);
    } else {
        out += digits.substr(0, 1);
        if (n > 1) out += "." + digits.substr(1);
        const int ee = point - 1;
        char eb[16];
        std::snprintf(eb, sizeof eb, "e%c%02d", ee < 0 ? '-' : '+', std::abs(ee));
        out += eb;
    }
    return out;
}

// json.dumps string escaping with ensure_ascii=False (src/pyjson.rs:102-118).
void write_string(std::string& out, const std::string& s) {
    out += '"';
    for (unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            case 0x08: out += "\\b"; break;
            case 0x0C: out += "\\f"; break;
            default:
                if (c < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", c);
                    out += b;
                } else {
                    out += (char)c;
                }
        }
    }
    out += '"';
}

// Python's json reads literals without '.', 'e' or 'E' as int and the rest as
// float (src/pyjson.rs:47-54).
void write_number(std::string& out, const Json& v) {
    if (v.raw.find_first_of(".eE") != std::string::npos) out += float_repr(v.num);
    else if (v.raw == "-0") out += '0';
    else out += v.raw;
}

// json.dumps separators (", " and ": "), insertion order (src/pyjson.rs:13-45).
void dumps(std::string& out, const Json& v) {
    switch (v.kind) {
        case Json::Null: out += "null"; break;
        case Json::Bool: out += v.b ? "true" : "false"; break;
        case Json::Number: write_number(out, v); break;
        case Json::String: write_string(out, v.str); break;
        case Json::Array:
            out += '[';
            for (size_t i = 0; i < v.arr.size(); ++i) {
                if (i) out += ", ";
                dumps(out, v.arr[i]);
            }
            out += ']';
            break;
        case Json::Object:
            out += '{';
            for (size_t i = 0; i < v.obj.size(); ++i) {
                if (i) out += ", ";
                write_string(out, v.obj[i].first);
                out += ": ";
                dumps(out, v.obj[i].second);
            }
            out += '}';
            break;
    }
}

std::string dumps(const Json& v) {
    std::string out;
    dumps(out, v);
    return out;
}

// ---------------------------------------------------------------- requests (src/request.rs)

enum QType { kChoice = 0, kScore = 1, kNoul = 2 };
const char* const kQNames[3] = {"choice", "score", "noul"};

int qtype_parse(const std::string& s) {
    for (int i = 0; i < 3; ++i)
        if (s == kQNames[i]) return i;
    return -1;
}

struct Request {
    bool text = true;  // State::Text, else State::Json
    std::string state_text;
    Json state_json;
    std::string question;
    std::vector<std::string> options;
    int qtype = kChoice;

    // State::render (src/request.rs:51-56)
    std::string render() const { return text ? state_text : dumps(state_json); }
    // State::to_value (src/request.rs:58-63)
    Json state_value() const {
        if (!text) return state_json;
        Json j;
        j.kind = Json::String;
        j.str = state_text;
        return j;
    }
};

// State::from_value (src/request.rs:41-47)
bool state_from_value(const Json& v, Request& r) {
    if (v.kind == Json::String) {
        r.text = true;
        r.state_text = v.str;
        return true;
    }
    if (v.kind == Json::Object || v.kind == Json::Array) {
        r.text = false;
        r.state_json = v;
        return true;
    }
    return false;
}

// serde_json's Number::as_u64 with arbitrary_precision: the literal parses as u64.
bool as_u64(const Json& v, uint64_t& out) {
    if (v.kind != Json::Number || v.raw.empty() || v.raw.find_first_not_of("0123456789") != std::string::npos)
        return false;
    errno = 0;
    char* end = nullptr;
    const unsigned long long x = std::strtoull(v.raw.c_str(), &end, 10);
    if (errno == ERANGE || *end) return false;
    out = x;
    return true;
}

// Request::from_value (src/request.rs:90-130): one legacy request object.
Request request_from_value(const Json& row, size_t line) {
    const std::string prefix = "JSONL line " + std::to_string(line) + ": ";
    if (row.kind != Json::Object) invalid(prefix + "request must be a JSON object");
    Request r;
    const Json* st = row.get("state");
    const Json* q = row.get("question");
    if (!st || !state_from_value(*st, r) || !q || q->kind != Json::String)
        invalid(prefix + "state must be text/JSON and question must be text");
    r.question = q->str;
    const Json* opts = row.get("options");
    bool ok = opts && opts->kind == Json::Array;
    if (ok)
        for (const Json& x : opts->arr) {
            if (x.kind != Json::String || x.str.empty()) { ok = false; break; }
            r.options.push_back(x.str);
        }
    if (!ok || r.options.size() < 2 || r.options.size() > 20)
        invalid(prefix + "options must contain 2–20 nonempty rendered descriptions");
    if (const Json* t = row.get("type")) {
        const int k = t->kind == Json::String ? qtype_parse(t->str) : -1;
        if (k < 0) invalid(prefix + "type must be choice, score, or noul");
        r.qtype = k;
    }
    if (r.qtype == kNoul && r.options.size() != 2) invalid(prefix + "noul options must be ordered [false, true]");
    if (const Json* target = row.get("target")) {
        uint64_t t = 0;
        if (!as_u64(*target, t) || t >= r.options.size())
            invalid(prefix + "target must index the supplied option list");
    }
    const Json* teacher = row.get("teacher_logits");
    if (teacher && teacher->kind != Json::Null) {
        bool good = teacher->kind == Json::Array && teacher->arr.size() == r.options.size();
        if (good)
            for (const Json& x : teacher->arr)
                if (x.kind != Json::Number || !std::isfinite(x.num)) { good = false; break; }
        if (!good) invalid(prefix + "teacher logits must be finite and match option count/order");
    }
    return r;
}

// Request::validate (src/request.rs:132-146): rows built in code.
void request_validate(const Request& r, size_t line) {
    const std::string prefix = "JSONL line " + std::to_string(line) + ": ";
    bool empty = false;
    for (const auto& o : r.options) empty |= o.empty();
    if (r.options.size() < 2 || r.options.size() > 20 || empty)
        invalid(prefix + "options must contain 2–20 nonempty rendered descriptions");
    if (!r.text && r.state_json.kind != Json::Object && r.state_json.kind != Json::Array)
        invalid(prefix + "state must be text/JSON and question must be text");
    if (r.qtype == kNoul && r.options.size() != 2) invalid(prefix + "noul options must be ordered [false, true]");
}

// Rows as the router receives them (`Request::new`, src/request.rs:80-84):
// state text/JSON, question text, options strings, optional type; the
// router applies its own option checks.
Request request_new_from_value(const Json& row, size_t line) {
    const std::string prefix = "JSONL line " + std::to_string(line) + ": ";
    if (row.kind != Json::Object) invalid(prefix + "request must be a JSON object");
    Request r;
    const Json* st = row.get("state");
    const Json* q = row.get("question");
    if (!st || !state_from_value(*st, r) || !q || q->kind != Json::String)
        invalid(prefix + "state must be text/JSON and question must be text");
    r.question = q->str;
    const Json* opts = row.get("options");
    if (!opts || opts->kind != Json::Array) invalid(prefix + "options must be an array of strings");
    for (const Json& x : opts->arr) {
        if (x.kind != Json::String) invalid(prefix + "options must be an array of strings");
        r.options.push_back(x.str);
    }
    if (const Json* t = row.get("type")) {
        const int k = t->kind == Json::String ? qtype_parse(t->str) : -1;
        if (k < 0) invalid(prefix + "type must be choice, score, or noul");
        r.qtype = k;
    }
    return r;
}

Json request_to_json(const Request& r) {
    Json o;
    o.kind = Json::Object;
    o.obj.emplace_back("state", r.state_value());
    Json q;
    q.kind = Json::String;
    q.str = r.question;
    o.obj.emplace_back("question", q);
    Json opts;
    opts.kind = Json::Array;
    for (const auto& s : r.options) {
        Json x;
        x.kind = Json::String;
        x.str = s;
        opts.arr.push_back(x);
    }
    o.obj.emplace_back("options", opts);
    Json t;
    t.kind = Json::String;
    t.str = kQNames[r.qtype];
    o.obj.emplace_back("type", t);
    return o;
}

// Lines of a JSONL document (str::lines: split at '\n', drop one trailing '\r').
template <class F>
void for_each_line(const char* p, size_t n, F&& f) {
    size_t i = 0, line = 0;
    while (i < n) {
        size_t j = i;
        while (j < n && p[j] != '\n') ++j;
        size_t e = j;
        if (e > i && p[e - 1] == '\r') --e;
        f(++line, std::string(p + i, e - i));
        i = j + 1;
    }
}

// parse_rows (src/engine.rs:298-307)
std::vector<Request> parse_rows(const char* p, size_t n, bool router_rows = false) {
    if (n && !p) invalid("null rows");
    check_utf8(p, n);
    std::vector<Request> rows;
    for_each_line(p, n, [&](size_t line, const std::string& l) {
        if (blank(l)) return;
        Json v;
        try {
            v = jh::JsonParser(l.data(), l.size()).parse();
        } catch (const std::runtime_error&) {
            invalid("line " + std::to_string(line) + ": invalid JSON");
        }
        rows.push_back(router_rows ? request_new_from_value(v, line) : request_from_value(v, line));
    });
    return rows;
}

// argmax (src/request.rs:164-172): first index of the maximum.
template <class T>
size_t argmax(const std::vector<T>& v) {
    size_t best = 0;
    for (size_t i = 0; i < v.size(); ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

// display_probabilities (src/request.rs:150-161)
std::vector<double> display_probabilities(const std::vector<double>& v) {
    if (v.empty()) return {};
    const size_t w = argmax(v);
    bool decisive = v[w] > 0.95;
    for (size_t i = 0; i < v.size() && decisive; ++i)
        if (i != w && !(v[i] < 0.045)) decisive = false;
    std::vector<double> out(v.size(), 0.0);
    if (decisive) {
        out[w] = 1.0;
        return out;
    }
    double total = 0.0;
    for (size_t i = 0; i < v.size(); ++i) {
        out[i] = v[i] >= 0.01 ? v[i] : 0.0;
        total += out[i];
    }
    for (double& x : out) x /= total;
    return out;
}

// softmax_f32 (src/request.rs:175-180): f32 throughout, like torch.softmax.
std::vector<float> softmax_f32(const std::vector<float>& v) {
    float mx = -INFINITY;
    for (float x : v) mx = std::fmax(mx, x);
    std::vector<float> e(v.size());
    float total = 0.0f;
    for (size_t i = 0; i < v.size(); ++i) {
        e[i] = std::exp(v[i] - mx);
        total += e[i];
    }
    for (float& x : e) x /= total;
    return e;
}

// ---------------------------------------------------------------- LRU cache

template <class V>
class Lru {
public:
    explicit Lru(size_t cap) : cap_(cap) {}
    bool enabled() const { return cap_ > 0; }
    bool get(const std::string& k, V& out) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = map_.find(k);
        if (it == map_.end()) return false;
        order_.splice(order_.begin(), order_, it->second);
        out = it->second->second;
        return true;
    }
    void put(const std::string& k, const V& v) {
        if (!cap_) return;
        std::lock_guard<std::mutex> g(mu_);
        auto it = map_.find(k);
        if (it != map_.end()) {
            it->second->second = v;
            order_.splice(order_.begin(), order_, it->second);
            return;
        }
        order_.emplace_front(k, v);
        map_[k] = order_.begin();
        if (map_.size() > cap_) {
            map_.erase(order_.back().first);
            order_.pop_back();
        }
    }
    void clear() {
        std::lock_guard<std::mutex> g(mu_);
        map_.clear();
        order_.clear();
    }

private:
    size_t cap_;
    std::mutex mu_;
    std::list<std::pair<std::string, V>> order_;
    std::unordered_map<std::string, typename std::list<std::pair<std::string, V>>::iterator> map_;
};

// ---------------------------------------------------------------- encoder (src/encode.rs)

constexpr size_t kOptionTokens = 48;  // src/encode.rs:12

struct Encoded {
    std::vector<uint32_t> ids;
    std::vector<uint32_t> markers;  // positions of the mask marker before each option
    int qtype = kChoice;
    bool truncated = false;
    std::vector<size_t> option_tokens;  // strict mode only
};

using Ids = std::shared_ptr<const std::vector<uint32_t>>;

}  // namespace

struct jt_encoder {
    jt_tokenizer tok{};
    std::string mask_token;
    uint32_t mask_id = 0, cls_id = 0, sep_id = 0, pad_id = 0;
    size_t max_length = 0, head_length = 0;
    bool strict = false;
    Lru<Ids> tokens{0};
    Lru<std::shared_ptr<const Encoded>> encodings{0};

    jt_encoder(size_t tc, size_t ec) : tokens(tc), encodings(ec) {}

    // Token ids already produced for this call by a batch tokenization (encode_many).
    using Pre = std::unordered_map<std::string, Ids>;

    // Encoder::tokenize (src/encode.rs:104-116)
    Ids tokenize(const std::string& text, const Pre* pre = nullptr) {
        if (pre) {
            auto it = pre->find(text);
            if (it != pre->end()) return it->second;
        }
        Ids hit;
        if (tokens.get(text, hit)) return hit;
        std::vector<uint32_t> ids(std::max<size_t>(64, text.size() + 8));
        size_t count = 0;
        if (tok.encode(tok.ctx, text.data(), text.size(), ids.data(), ids.size(), &count) != 0)
            invalid("tokenizer failed");
        if (count > ids.size()) {
            ids.resize(count);
            size_t again = 0;
            if (tok.encode(tok.ctx, text.data(), text.size(), ids.data(), ids.size(), &again) != 0 || again != count)
                invalid("tokenizer failed");
        }
        ids.resize(count);
        auto out = std::make_shared<const std::vector<uint32_t>>(std::move(ids));
        tokens.put(text, out);
        return out;
    }

    // Encoder::encode (src/encode.rs:118-135): the cache key covers the
    // rendered state, question, options, qtype and whether the state is text.
    static std::string cache_key(const Request& row, const std::string& state) {
        std::string key;
        auto field = [&](const std::string& s) {
            key += std::to_string(s.size());
            key += ':';
            key += s;
        };
        field(state);
        field(row.question);
        key += std::to_string(row.options.size());
        key += '|';
        for (const auto& o : row.options) field(o);
        key += kQNames[row.qtype];
        key += row.text ? 't' : 'j';
        return key;
    }

    std::shared_ptr<const Encoded> encode(const Request& row) {
        const std::string state = row.render();
        std::string key;
        if (encodings.enabled()) {
            key = cache_key(row, state);
            std::shared_ptr<const Encoded> hit;
            if (encodings.get(key, hit)) return hit;
        }
        auto e = std::make_shared<const Encoded>(sequence(state, row));
        if (encodings.enabled()) encodings.put(key, e);
        return e;
    }

    // Engine::encode's row encoding (src/engine.rs:183-188): the reference
    // encodes rows in parallel with Tokenizer::encode_fast.  Here, with a
    // batch tokenizer and more than one row, every distinct segment the
    // uncached rows need that the token cache lacks is tokenized in one call
    // (the tokenizer may run it in parallel), then each row is assembled as
    // encode() would; the results are the same ids.  A single row keeps the
    // per-text calls: its few segments do not repay a parallel dispatch.
    std::vector<std::shared_ptr<const Encoded>> encode_many(const std::vector<Request>& rows) {
        std::vector<std::shared_ptr<const Encoded>> out(rows.size());
        if (!tok.encode_batch || rows.size() < 2) {
            for (size_t i = 0; i < rows.size(); ++i) out[i] = encode(rows[i]);
            return out;
        }
        std::vector<std::string> states(rows.size()), keys(rows.size());
        std::vector<size_t> miss;
        for (size_t i = 0; i < rows.size(); ++i) {
            states[i] = rows[i].render();
            if (encodings.enabled()) {
                keys[i] = cache_key(rows[i], states[i]);
                if (encodings.get(keys[i], out[i])) continue;
            }
            miss.push_back(i);
        }
        std::vector<std::string> texts;
        std::unordered_set<std::string> seen;
        for (size_t i : miss)
            for (std::string& t : segments(rows[i], states[i])) {
                Ids hit;
                if (seen.count(t) || tokens.get(t, hit)) continue;
                seen.insert(t);
                texts.push_back(std::move(t));
            }
        const Pre pre = tokenize_batch(texts);
        for (size_t i : miss) {
            out[i] = std::make_shared<const Encoded>(sequence(states[i], rows[i], &pre));
            if (encodings.enabled()) encodings.put(keys[i], out[i]);
        }
        return out;
    }

    // One encode_batch call for `texts`; the results also enter the token cache.
    Pre tokenize_batch(const std::vector<std::string>& texts) {
        Pre pre;
        if (texts.empty()) return pre;
        std::vector<const char*> ptrs;
        std::vector<size_t> lens, counts(texts.size(), 0);
        for (const auto& t : texts) {
            ptrs.push_back(t.data());
            lens.push_back(t.size());
        }
        const uint32_t* ids = nullptr;
        if (tok.encode_batch(tok.ctx, texts.size(), ptrs.data(), lens.data(), counts.data(), &ids) != 0)
            invalid("tokenizer failed");
        size_t total = 0;
        for (size_t c : counts) total += c;
        if (total && !ids) invalid("tokenizer failed");
        size_t off = 0;
        for (size_t i = 0; i < texts.size(); ++i) {
            auto v = std::make_shared<const std::vector<uint32_t>>(ids + off, ids + off + counts[i]);
            off += counts[i];
            tokens.put(texts[i], v);
            pre.emplace(texts[i], std::move(v));
        }
        return pre;
    }

    // The texts Encoder::sequence tokenizes for a row: the question head,
    // each option (with its leading space) and the state, marker text blanked.
    std::string clean(const std::string& t) const { return replace_all(t, mask_token, " "); }
    std::string head_text(const Request& row) const {
        return std::string(kQNames[row.qtype]) + " question: " + clean(row.question);
    }
    std::string option_text(const std::string& o) const { return " " + clean(o); }
    std::vector<std::string> segments(const Request& row, const std::string& state) const {
        std::vector<std::string> out{head_text(row)};
        for (const auto& o : row.options) out.push_back(option_text(o));
        out.push_back(clean(state));
        return out;
    }

    // Encoder::sequence (src/encode.rs:137-195): [CLS] head [SEP] (<mask>
    // option)* [SEP] state [SEP], with the head/option budget and the state
    // truncated to max_length.
    Encoded sequence(const std::string& state, const Request& row, const Pre* pre = nullptr) {
        const std::string& mask = mask_token;
        if (strict) {
            bool found = state.find(mask) != std::string::npos || row.question.find(mask) != std::string::npos;
            for (const auto& o : row.options) found |= o.find(mask) != std::string::npos;
            if (found) invalid("Reserved model marker in request");
        }
        const Ids head = tokenize(head_text(row), pre);
        std::vector<Ids> option_ids;
        for (const auto& o : row.options) option_ids.push_back(tokenize(option_text(o), pre));
        if (strict)
            for (const auto& x : option_ids)
                if (x->size() > kOptionTokens) invalid("Option exceeds 48-token model contract");
        std::vector<std::vector<uint32_t>> options;
        for (const auto& x : option_ids) {
            std::vector<uint32_t> o{mask_id};
            o.insert(o.end(), x->begin(), x->begin() + std::min(x->size(), kOptionTokens));
            options.push_back(std::move(o));
        }
        const int64_t hl = (int64_t)head_length;
        auto total = [&] {
            int64_t s = 0;
            for (const auto& o : options) s += (int64_t)o.size();
            return s;
        };
        int64_t budget = hl - total();
        if (budget < 16) {
            // (head_length - 16).div_euclid(options) clamped below at 4
            const int64_t n = (int64_t)options.size();
            int64_t q = (hl - 16) / n;
            if ((hl - 16) % n < 0) --q;
            const size_t per_option = (size_t)std::max<int64_t>(q, 4);
            for (auto& o : options)
                if (o.size() > per_option) o.resize(per_option);
            budget = hl - total();
        }
        if (strict) {
            bool lossy = (int64_t)head->size() > budget;
            for (size_t i = 0; i < options.size(); ++i) lossy |= options[i].size() != option_ids[i]->size() + 1;
            if (lossy) invalid("Question/options exceed lossless head budget");
        }
        Encoded e;
        e.ids.reserve(std::min<size_t>(max_length, 4096));
        e.ids.push_back(cls_id);
        const size_t keep = std::min(head->size(), (size_t)std::max<int64_t>(budget, 8));
        e.ids.insert(e.ids.end(), head->begin(), head->begin() + keep);
        e.ids.push_back(sep_id);
        for (const auto& o : options) {
            e.markers.push_back((uint32_t)e.ids.size());
            e.ids.insert(e.ids.end(), o.begin(), o.end());
        }
        e.ids.push_back(sep_id);
        const Ids state_ids = tokenize(clean(state), pre);
        const int64_t room = (int64_t)max_length - (int64_t)e.ids.size() - 1;
        if (room < 1) invalid("Question/options exceed sequence budget; shorten descriptions");
        if (strict && (int64_t)state_ids->size() > room) invalid("Game state exceeds lossless context budget");
        e.ids.insert(e.ids.end(), state_ids->begin(), state_ids->begin() + std::min<size_t>(state_ids->size(), room));
        e.ids.push_back(sep_id);
        e.qtype = row.qtype;
        e.truncated = (int64_t)state_ids->size() > room;
        if (strict)
            for (const auto& x : option_ids) e.option_tokens.push_back(x->size());
        return e;
    }
};

struct jt_rows {
    std::vector<std::vector<float>> rows;
};

struct jt_scorer {
    // engine scorer
    je_engine* engine = nullptr;
    jt_encoder* encoder = nullptr;
    // callback scorer
    jt_logits_fn fn = nullptr;
    void* ctx = nullptr;

    // Logits::logits (src/engine.rs:238-244, 287-295)
    std::vector<std::vector<float>> logits(const std::vector<Request>& rows) {
        if (rows.empty()) return {};
        if (fn) {
            Json arr;
            arr.kind = Json::Array;
            for (const auto& r : rows) arr.arr.push_back(request_to_json(r));
            const std::string text = dumps(arr);
            jt_rows out;
            if (fn(ctx, text.data(), text.size(), &out) != 0) invalid("scorer callback failed");
            return std::move(out.rows);
        }
        // Engine::encode: validate every row, then encode every row, before inference.
        for (size_t i = 0; i < rows.size(); ++i) request_validate(rows[i], i + 1);
        const std::vector<std::shared_ptr<const Encoded>> enc = encoder->encode_many(rows);
        std::vector<uint32_t> ids, markers;
        std::vector<size_t> id_off{0}, mk_off{0};
        std::vector<uint8_t> qt;
        for (const auto& e : enc) {
            ids.insert(ids.end(), e->ids.begin(), e->ids.end());
            markers.insert(markers.end(), e->markers.begin(), e->markers.end());
            id_off.push_back(ids.size());
            mk_off.push_back(markers.size());
            qt.push_back((uint8_t)e->qtype);
        }
        std::vector<float> flat(markers.size());
        const int rc = je_logits_encoded(engine, enc.size(), ids.data(), id_off.data(), markers.data(), mk_off.data(),
                                         qt.data(), flat.data());
        if (rc != JH_OK) throw jh_error(rc, jh_last_error());
        std::vector<std::vector<float>> out(enc.size());
        for (size_t i = 0; i < enc.size(); ++i) out[i].assign(flat.begin() + mk_off[i], flat.begin() + mk_off[i + 1]);
        return out;
    }
};

namespace {

// ---------------------------------------------------------------- typed questions (src/typed.rs)

struct QuestionMeta {
    std::string id;
    int qtype;
    std::vector<std::string> keys;
};

struct Answer {
    int qtype;
    std::vector<std::string> keys;
    std::vector<double> p;
};

Json jstr(const std::string& s) {
    Json j;
    j.kind = Json::String;
    j.str = s;
    return j;
}

// typed_rows (src/typed.rs:65-112): every row validated before inference.
void typed_rows(const Request& state, const Json& questions, std::vector<Request>& rows,
                std::vector<QuestionMeta>& meta) {
    if (questions.kind != Json::Object || questions.obj.empty()) invalid("questions must be a nonempty mapping");
    for (const auto& [qid, q] : questions.obj) {
        if (q.kind != Json::Object || qid.empty()) invalid("Questions require nonempty string IDs and question objects");
        const Json* t = q.get("type");
        const int kind = t && t->kind == Json::String ? qtype_parse(t->str) : -1;
        const Json* criteria = q.get("criteria");
        if (criteria && criteria->kind == Json::Null) criteria = nullptr;
        std::vector<std::string> keys;
        Json labels;
        labels.kind = Json::Array;
        if (kind == kChoice) {
            bool ok = criteria && criteria->kind == Json::Object;
            if (ok)
                for (const auto& kv : criteria->obj) ok &= !kv.first.empty();
            if (!ok) invalid("Choice criteria must map nonempty IDs to descriptions");
            for (const auto& kv : criteria->obj) {
                keys.push_back(kv.first);
                labels.arr.push_back(kv.second);
            }
        } else if (kind == kScore) {
            if (!criteria || criteria->kind != Json::Array) invalid("Score requires an ordered rubric");
            for (size_t i = 0; i < criteria->arr.size(); ++i) keys.push_back(std::to_string(i));
            labels.arr = criteria->arr;
        } else if (kind == kNoul) {
            keys = {"false", "true"};
            if (!criteria) {
                labels.arr = {jstr("false"), jstr("true")};
            } else {
                const bool ok = criteria->kind == Json::Object && criteria->obj.size() == 2 && criteria->get("false") &&
                                criteria->get("true");
                if (!ok) invalid("Noul criteria must map false and true to descriptions");
                labels.arr = {*criteria->get("false"), *criteria->get("true")};
            }
        } else {
            invalid("Unsupported question type");
        }
        Json row;
        row.kind = Json::Object;
        row.obj.emplace_back("state", state.state_value());
        const Json* instr = q.get("instructions");
        row.obj.emplace_back("question", instr ? *instr : Json());
        row.obj.emplace_back("type", jstr(kQNames[kind]));
        row.obj.emplace_back("options", labels);
        rows.push_back(request_from_value(row, rows.size() + 1));
        meta.push_back({qid, kind, keys});
    }
}

// answers_from_logits (src/typed.rs:115-131): float64 softmax per question.
std::vector<Answer> answers_from_logits(const std::vector<QuestionMeta>& meta,
                                        const std::vector<std::vector<float>>& scores) {
    if (scores.size() != meta.size()) invalid("Model returned an incorrect answer count");
    std::vector<Answer> out;
    for (size_t i = 0; i < meta.size(); ++i) {
        const auto& z = scores[i];
        bool bad = z.size() != meta[i].keys.size();
        for (float v : z) bad |= !std::isfinite(v);
        if (bad) invalid("Invalid model scores");
        float mx = -INFINITY;
        for (float v : z) mx = std::fmax(mx, v);
        std::vector<double> e(z.size());
        double total = 0.0;
        for (size_t k = 0; k < z.size(); ++k) {
            e[k] = std::exp((double)z[k] - (double)mx);
            total += e[k];
        }
        for (double& x : e) x /= total;
        out.push_back({meta[i].qtype, meta[i].keys, std::move(e)});
    }
    return out;
}

// Answer::to_json + answers_to_json (src/typed.rs:37-62)
std::string answers_to_json(const std::vector<QuestionMeta>& meta, const std::vector<Answer>& answers) {
    std::string o = "{\"answers\": {";
    for (size_t i = 0; i < answers.size(); ++i) {
        const Answer& a = answers[i];
        if (i) o += ", ";
        write_string(o, meta[i].id);
        o += ": {\"type\": ";
        write_string(o, kQNames[a.qtype]);
        o += ", \"probabilities\": {";
        for (size_t k = 0; k < a.keys.size(); ++k) {
            if (k) o += ", ";
            write_string(o, a.keys[k]);
            o += ": " + json_float(a.p[k]);
        }
        o += "}";
        if (a.qtype == kChoice) {
            o += ", \"choice\": ";
            write_string(o, a.keys[argmax(a.p)]);
        } else if (a.qtype == kScore) {
            double s = 0.0;
            for (size_t k = 0; k < a.p.size(); ++k) s += (double)k * a.p[k];
            o += ", \"score\": " + json_float(s);
        } else {
            o += ", \"noul\": " + json_float(a.p[1]);
        }
        if (a.qtype != kNoul) {
            double m = -INFINITY;
            for (double x : a.p) m = std::fmax(m, x);
            o += ", \"max_probability\": " + json_float(m);
        }
        o += "}";
    }
    o += "}}";
    return o;
}

std::string float_list(const std::vector<float>& v) {
    std::string o = "[";
    for (size_t i = 0; i < v.size(); ++i) {
        if (i) o += ", ";
        o += json_float(v[i]);
    }
    return o + "]";
}

std::string double_list(const std::vector<double>& v) {
    std::string o = "[";
    for (size_t i = 0; i < v.size(); ++i) {
        if (i) o += ", ";
        o += json_float(v[i]);
    }
    return o + "]";
}

template <class T>
std::string int_list(const std::vector<T>& v) {
    std::string o = "[";
    for (size_t i = 0; i < v.size(); ++i) {
        if (i) o += ", ";
        o += std::to_string(v[i]);
    }
    return o + "]";
}

char* give(const std::string& s) {
    char* p = (char*)std::malloc(s.size() + 1);
    if (!p) throw std::bad_alloc();
    std::memcpy(p, s.data(), s.size());
    p[s.size()] = '\0';
    return p;
}

// Router::confident_winner (src/router.rs:132-142)
bool confident_winner(const std::vector<float>& scores, size_t best) {
    std::vector<double> s(scores.begin(), scores.end());
    double runner_up = -INFINITY;
    for (size_t i = 0; i < s.size(); ++i)
        if (i != best) runner_up = std::fmax(runner_up, s[i]);
    if (runner_up - s[best] >= std::log(0.045 / 0.95)) return false;
    double total = 0.0;
    for (double v : s) total += std::exp(v - s[best]);
    return 1.0 / total > 0.95 && std::exp(runner_up - s[best]) / total < 0.045;
}

}  // namespace

// ---------------------------------------------------------------- router (src/router.rs)

struct jt_router {
    jt_scorer* engine;
    size_t width, survivors, batch_size, max_options;
    Lru<std::vector<float>> cache;
    std::mutex lock;

    jt_router(jt_scorer* e, size_t w, size_t s, size_t b, size_t c, size_t m)
        : engine(e), width(w), survivors(s), batch_size(b), max_options(m), cache(c) {}

    // Router::validate (src/router.rs:65-80)
    void validate(const Request& row) const {
        if (row.options.size() < 2 || row.options.size() > max_options)
            invalid("Expected 2–" + std::to_string(max_options) + " options");
        for (const auto& o : row.options)
            if (o.empty()) invalid("Options must be nonempty strings");
        if (row.qtype == kNoul && row.options.size() != 2) invalid("noul requires [false, true]");
        if (row.qtype != kChoice && row.options.size() > width)
            invalid("Hierarchical routing supports choice decisions only");
    }

    // Router::key (src/router.rs:84-86)
    static std::string key(const Request& row) {
        std::string k = dumps(row.state_value());
        k += '\0';
        k += row.question;
        k += '\0';
        k += kQNames[row.qtype];
        k += '\0';
        for (size_t i = 0; i < row.options.size(); ++i) {
            if (i) k += '\0';
            k += row.options[i];
        }
        return k;
    }

    // Router::score (src/router.rs:88-129): cache, in-call dedup, chunks of batch_size.
    std::vector<std::vector<float>> score(const std::vector<Request>& jobs, size_t& used, size_t& hits) {
        std::vector<std::vector<float>> values(jobs.size());
        std::vector<bool> have(jobs.size(), false);
        std::vector<std::pair<std::string, std::vector<size_t>>> missing;
        std::unordered_map<std::string, size_t> index;
        hits = 0;
        for (size_t i = 0; i < jobs.size(); ++i) {
            std::string k = key(jobs[i]);
            if (cache.enabled() && cache.get(k, values[i])) {
                have[i] = true;
                ++hits;
                continue;
            }
            auto it = index.find(k);
            if (it != index.end()) {
                missing[it->second].second.push_back(i);
                ++hits;
            } else {
                index.emplace(k, missing.size());
                missing.push_back({std::move(k), {i}});
            }
        }
        for (size_t c = 0; c < missing.size(); c += batch_size) {
            const size_t end = std::min(missing.size(), c + batch_size);
            std::vector<Request> rows;
            for (size_t j = c; j < end; ++j) rows.push_back(jobs[missing[j].second[0]]);
            auto output = engine->logits(rows);
            if (output.size() != rows.size()) invalid("Engine returned the wrong number of rows");
            for (size_t j = c; j < end; ++j) {
                auto& scores = output[j - c];
                bool bad = scores.size() != jobs[missing[j].second[0]].options.size();
                for (float v : scores) bad |= !std::isfinite(v);
                if (bad) invalid("Engine logits must be finite and match option count");
                for (size_t i : missing[j].second) {
                    values[i] = scores;
                    have[i] = true;
                }
                cache.put(missing[j].first, scores);
            }
        }
        used = missing.size();
        return values;
    }

    struct Result {
        size_t index = 0;
        std::vector<size_t> candidates;
        std::vector<double> probabilities;
        size_t rounds = 0;
        bool hierarchical = false;
    };

    // Router::route_many (src/router.rs:147-210)
    std::string route_many(const std::vector<Request>& rows) {
        std::lock_guard<std::mutex> g(lock);
        for (const auto& r : rows) validate(r);
        std::vector<std::vector<size_t>> candidates(rows.size());
        for (size_t i = 0; i < rows.size(); ++i)
            for (size_t k = 0; k < rows[i].options.size(); ++k) candidates[i].push_back(k);
        std::vector<Result> results(rows.size());
        std::vector<bool> done(rows.size(), false);
        size_t model_rows = 0, hits = 0, remaining = rows.size();
        while (remaining) {
            std::vector<Request> jobs;
            struct Slot {
                size_t row;
                std::vector<size_t> group;
                bool last;
            };
            std::vector<Slot> layout;
            for (size_t i = 0; i < rows.size(); ++i) {
                if (done[i]) continue;
                results[i].rounds += 1;
                std::vector<size_t> current = std::move(candidates[i]);
                candidates[i].clear();
                const bool last = current.size() <= width;
                for (size_t c = 0; c < current.size(); c += width) {
                    std::vector<size_t> group(current.begin() + c, current.begin() + std::min(current.size(), c + width));
                    if (group.size() == 1) {
                        candidates[i].push_back(group[0]);
                        continue;
                    }
                    Request job = rows[i];
                    job.options.clear();
                    for (size_t k : group) job.options.push_back(rows[i].options[k]);
                    jobs.push_back(std::move(job));
                    layout.push_back({i, std::move(group), last});
                }
            }
            if (jobs.empty()) invalid("routing made no progress");
            size_t used = 0, cached = 0;
            auto scored = score(jobs, used, cached);
            model_rows += used;
            hits += cached;
            for (size_t j = 0; j < layout.size(); ++j) {
                const Slot& s = layout[j];
                const auto& scores = scored[j];
                const size_t best = argmax(scores);
                if (s.last) {
                    float mxf = -INFINITY;
                    for (float x : scores) mxf = std::fmax(mxf, x);
                    const double mx = mxf;
                    std::vector<double> w(scores.size());
                    double total = 0.0;
                    for (size_t k = 0; k < scores.size(); ++k) {
                        w[k] = std::exp((double)scores[k] - mx);
                        total += w[k];
                    }
                    for (double& x : w) x /= total;
                    Result& r = results[s.row];
                    r.index = s.group[best];
                    r.probabilities = display_probabilities(w);
                    r.candidates = s.group;
                    r.hierarchical = rows[s.row].options.size() > width;
                    done[s.row] = true;
                    --remaining;
                } else if (confident_winner(scores, best)) {
                    candidates[s.row].push_back(s.group[best]);
                } else {
                    std::vector<size_t> rem(s.group.size());
                    for (size_t k = 0; k < rem.size(); ++k) rem[k] = k;
                    std::vector<size_t> chosen;
                    for (size_t t = 0; t < std::min(survivors, s.group.size()); ++t) {
                        std::vector<float> local;
                        for (size_t k : rem) local.push_back(scores[k]);
                        const size_t a = argmax(local);
                        chosen.push_back(s.group[rem[a]]);
                        rem.erase(rem.begin() + a);
                    }
                    std::sort(chosen.begin(), chosen.end());
                    candidates[s.row].insert(candidates[s.row].end(), chosen.begin(), chosen.end());
                }
            }
        }
        std::string o = "[";
        for (size_t i = 0; i < results.size(); ++i) {
            const Result& r = results[i];
            if (i) o += ", ";
            o += "{\"index\": " + std::to_string(r.index) + ", \"candidates\": " + int_list(r.candidates) +
                 ", \"probabilities\": " + double_list(r.probabilities) + ", \"rounds\": " + std::to_string(r.rounds) +
                 ", \"model_rows\": " + std::to_string(model_rows) + ", \"cache_hits\": " + std::to_string(hits) +
                 ", \"hierarchical\": " + (r.hierarchical ? "true" : "false") + ", \"probability_scope\": \"" +
                 (r.hierarchical ? "final_candidates" : "all_options") + "\"}";
        }
        return o + "]";
    }
};

// ---------------------------------------------------------------- C-ABI

extern "C" {

void jt_free(void* p) { std::free(p); }

int jt_pyjson_dumps(const char* json, size_t len, char** out) {
    return jh_guarded([&] {
        if (!out) invalid("null output");
        *out = nullptr;
        *out = give(dumps(parse(json, len, "invalid JSON")));
    });
}

int jt_float_repr(double value, char** out) {
    return jh_guarded([&] {
        if (!out) invalid("null output");
        *out = give(float_repr(value));
    });
}

void jt_default_encoder_options(jt_encoder_options* o) {
    if (!o) return;
    *o = jt_encoder_options{0, 256, 0, 8192, 2048};
}

int jt_encoder_create(const jt_tokenizer* tok, const char* cfg, size_t len, const jt_encoder_options* opt,
                      jt_encoder** out) {
    return jh_guarded([&] {
        if (!out || !tok || !tok->encode || !tok->token_to_id || !opt) invalid("null argument");
        *out = nullptr;
        // Encoder::from_parts (src/encode.rs:58-93)
        if ((size_t)opt->head_length + 4 >= (size_t)opt->max_length)
            invalid("max_length must leave room beyond the question head");
        const Json config = parse(cfg, len, "tokenizer_config.json");
        auto e = std::make_unique<jt_encoder>(opt->token_cache, opt->encoding_cache);
        e->tok = *tok;
        auto token = [&](const char* key, std::string* name_out) {
            const Json* v = config.get(key);
            if (!v || v->kind != Json::String) invalid(std::string("tokenizer lacks ") + key);
            uint32_t id = 0;
            if (tok->token_to_id(tok->ctx, v->str.c_str(), &id) != 0)
                invalid(std::string("unknown ") + key + " " + v->str);
            if (name_out) *name_out = v->str;
            return id;
        };
        e->mask_id = token("mask_token", &e->mask_token);
        e->cls_id = token("cls_token", nullptr);
        e->sep_id = token("sep_token", nullptr);
        e->pad_id = token("pad_token", nullptr);
        e->max_length = opt->max_length;
        e->head_length = opt->head_length;
        e->strict = opt->strict != 0;
        *out = e.release();
    });
}

void jt_encoder_destroy(jt_encoder* e) { delete e; }

void jt_encoder_clear_cache(jt_encoder* e) {
    if (!e) return;
    e->tokens.clear();
    e->encodings.clear();
}

int jt_encoder_special_ids(jt_encoder* e, uint32_t out[4]) {
    return jh_guarded([&] {
        if (!e || !out) invalid("null argument");
        out[0] = e->mask_id;
        out[1] = e->cls_id;
        out[2] = e->sep_id;
        out[3] = e->pad_id;
    });
}

int jt_encode(jt_encoder* e, const char* row_json, size_t len, size_t line, char** out) {
    return jh_guarded([&] {
        if (!e || !out) invalid("null argument");
        *out = nullptr;
        const Request r = request_from_value(parse(row_json, len, "invalid JSON"), line);
        const auto enc = e->encode(r);
        std::string o = "{\"ids\": " + int_list(enc->ids) + ", \"markers\": " + int_list(enc->markers) +
                        ", \"qtype\": \"" + kQNames[enc->qtype] + "\", \"truncated\": " +
                        (enc->truncated ? "true" : "false") + ", \"option_tokens\": " + int_list(enc->option_tokens) +
                        "}";
        *out = give(o);
    });
}

int jt_encoding_info(jt_encoder* e, const char* jsonl, size_t len, char** out) {
    return jh_guarded([&] {
        if (!e || !out) invalid("null argument");
        *out = nullptr;
        // Engine::encoding_info (src/engine.rs:261-280)
        if (!e->strict) invalid("Lossless encoding audit requires strict_encoding=True");
        const auto rows = parse_rows(jsonl, len);
        for (size_t i = 0; i < rows.size(); ++i) request_validate(rows[i], i + 1);
        const std::vector<std::shared_ptr<const Encoded>> enc = e->encode_many(rows);
        std::string o = "[";
        for (size_t i = 0; i < enc.size(); ++i) {
            if (i) o += ", ";
            o += "{\"tokens\": " + std::to_string(enc[i]->ids.size()) + ", \"optionTokens\": " +
                 int_list(enc[i]->option_tokens) + ", \"headLength\": " + std::to_string(e->head_length) +
                 ", \"stateTruncated\": false, \"optionsTruncated\": false}";
        }
        *out = give(o + "]");
    });
}

int jt_rows_push(jt_rows* rows, const float* logits, size_t count) {
    return jh_guarded([&] {
        if (!rows || (count && !logits)) invalid("null argument");
        rows->rows.emplace_back(logits, logits + count);
    });
}

int jt_scorer_callback(jt_logits_fn fn, void* ctx, jt_scorer** out) {
    return jh_guarded([&] {
        if (!fn || !out) invalid("null argument");
        auto s = std::make_unique<jt_scorer>();
        s->fn = fn;
        s->ctx = ctx;
        *out = s.release();
    });
}

int jt_scorer_engine(je_engine* engine, jt_encoder* encoder, jt_scorer** out) {
    return jh_guarded([&] {
        if (!engine || !encoder || !out) invalid("null argument");
        auto s = std::make_unique<jt_scorer>();
        s->engine = engine;
        s->encoder = encoder;
        *out = s.release();
    });
}

void jt_scorer_destroy(jt_scorer* s) { delete s; }

int jt_logits(jt_scorer* s, const char* jsonl, size_t len, char** out) {
    return jh_guarded([&] {
        if (!s || !out) invalid("null argument");
        *out = nullptr;
        const auto rows = parse_rows(jsonl, len);
        const auto z = s->logits(rows);
        if (z.size() != rows.size()) invalid("Engine returned the wrong number of rows");
        std::string o = "[";
        for (size_t i = 0; i < z.size(); ++i) {
            if (i) o += ", ";
            o += float_list(z[i]);
        }
        *out = give(o + "]");
    });
}

int jt_predict(jt_scorer* s, const char* jsonl, size_t len, int probabilities, char** out) {
    return jh_guarded([&] {
        if (!s || !out) invalid("null argument");
        *out = nullptr;
        // Engine::predict (src/engine.rs:247-258)
        const auto rows = parse_rows(jsonl, len);
        const auto z = s->logits(rows);
        if (z.size() != rows.size()) invalid("Engine returned the wrong number of rows");
        std::string o = "[";
        for (size_t i = 0; i < z.size(); ++i) {
            if (i) o += ", ";
            o += "{\"index\": " + std::to_string(argmax(z[i]));
            if (probabilities) {
                const auto sm = softmax_f32(z[i]);
                o += ", \"probabilities\": " + double_list(display_probabilities(std::vector<double>(sm.begin(), sm.end())));
            }
            o += "}";
        }
        *out = give(o + "]");
    });
}

int jt_predict_typed(jt_scorer* s, const char* state_json, size_t state_len, const char* questions_json,
                     size_t questions_len, char** out) {
    return jh_guarded([&] {
        if (!s || !out) invalid("null argument");
        *out = nullptr;
        Request state;
        if (!state_from_value(parse(state_json, state_len, "state"), state))
            invalid("state must be text/JSON and question must be text");
        const Json questions = parse(questions_json, questions_len, "questions");
        std::vector<Request> rows;
        std::vector<QuestionMeta> meta;
        typed_rows(state, questions, rows, meta);
        const auto answers = answers_from_logits(meta, s->logits(rows));
        *out = give(answers_to_json(meta, answers));
    });
}

int jt_router_create(jt_scorer* s, uint32_t width, uint32_t survivors, uint32_t batch_size, uint32_t cache_size,
                     uint32_t max_options, jt_router** out) {
    return jh_guarded([&] {
        if (!s || !out) invalid("null argument");
        *out = nullptr;
        // Router::new (src/router.rs:39-55)
        if (width < 2 || width > 20 || survivors < 1 || survivors >= width)
            invalid("Require 2 <= width <= 20 and 1 <= survivors < width");
        if (batch_size < 1 || max_options < width) invalid("Invalid batch/cache/capacity limit");
        *out = new jt_router(s, width, survivors, batch_size, cache_size, max_options);
    });
}

int jt_router_route_many(jt_router* r, const char* jsonl, size_t len, char** out) {
    return jh_guarded([&] {
        if (!r || !out) invalid("null argument");
        *out = nullptr;
        *out = give(r->route_many(parse_rows(jsonl, len, true)));
    });
}

void jt_router_clear_cache(jt_router* r) {
    if (r) r->cache.clear();
}

void jt_router_destroy(jt_router* r) { delete r; }

int jt_display_probabilities(const double* values, size_t n, double* out) {
    return jh_guarded([&] {
        if (n && (!values || !out)) invalid("null argument");
        const auto r = display_probabilities(std::vector<double>(values, values + n));
        std::copy(r.begin(), r.end(), out);
    });
}

int jt_confident_winner(const float* scores, size_t n, size_t best, int* out) {
    return jh_guarded([&] {
        if (!scores || !out || best >= n) invalid("bad argument");
        *out = confident_winner(std::vector<float>(scores, scores + n), best) ? 1 : 0;
    });
}

}  // extern "C"
