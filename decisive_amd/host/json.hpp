// json.hpp -- a small JSON value for the host layer (requests, parameters,
// responses). The reference passes serde_json::Value through its inference
// API (src/inference/mod.rs:18-42); this is the C++ stand-in: null, bool,
// number (double, remembering whether it was written as an integer, as
// serde_json's Number does), string, array and object (members kept in
// insertion order: the reference builds serde_json with `preserve_order`,
// Cargo.toml:50), with a strict parser and a compact writer whose number
// text is serde_json's (shortest round-trip digits, `1.0` for integral
// floats).
#pragma once

#include <cctype>
#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace decisive {

// Object members in insertion order (serde_json's Map under preserve_order).
// Lookup is a linear scan: requests and responses hold a handful of keys.
// Assigning to an existing key keeps its position; two maps are equal when
// they hold the same keys with equal values, in any order.
template <class V>
class OrderedMap {
public:
    using value_type = std::pair<std::string, V>;
    using iterator = typename std::vector<value_type>::iterator;
    using const_iterator = typename std::vector<value_type>::const_iterator;

    iterator begin() { return items_.begin(); }
    iterator end() { return items_.end(); }
    const_iterator begin() const { return items_.begin(); }
    const_iterator end() const { return items_.end(); }
    size_t size() const { return items_.size(); }
    bool empty() const { return items_.empty(); }

    iterator find(const std::string &key) {
        for (auto it = items_.begin(); it != items_.end(); ++it)
            if (it->first == key) return it;
        return items_.end();
    }
    const_iterator find(const std::string &key) const {
        for (auto it = items_.begin(); it != items_.end(); ++it)
            if (it->first == key) return it;
        return items_.end();
    }
    size_t count(const std::string &key) const { return find(key) == end() ? 0 : 1; }
    V &operator[](const std::string &key) {
        auto it = find(key);
        if (it != end()) return it->second;
        items_.emplace_back(key, V());
        return items_.back().second;
    }
    bool operator==(const OrderedMap &o) const {
        if (size() != o.size()) return false;
        for (const auto &kv : items_) {
            auto it = o.find(kv.first);
            if (it == o.end() || !(it->second == kv.second)) return false;
        }
        return true;
    }

private:
    std::vector<value_type> items_;
};

class Json {
public:
    enum class Kind { Null, Bool, Number, String, Array, Object };
    using Array = std::vector<Json>;
    using Object = OrderedMap<Json>;

    Json() = default;
    Json(std::nullptr_t) {}
    Json(bool b) : kind_(Kind::Bool), b_(b) {}
    Json(int v) : kind_(Kind::Number), integer_(true), n_(v) {}
    Json(int64_t v) : kind_(Kind::Number), integer_(true), n_((double)v) {}
    Json(uint64_t v) : kind_(Kind::Number), integer_(true), n_((double)v) {}
    Json(double v) : kind_(Kind::Number), n_(v) {}
    Json(const char *s) : kind_(Kind::String), s_(s) {}
    Json(std::string s) : kind_(Kind::String), s_(std::move(s)) {}
    Json(Array a) : kind_(Kind::Array), a_(std::make_shared<Array>(std::move(a))) {}
    Json(Object o) : kind_(Kind::Object), o_(std::make_shared<Object>(std::move(o))) {}

    static Json array() { return Json(Array{}); }
    static Json object() { return Json(Object{}); }

    Kind kind() const { return kind_; }
    bool is_null() const { return kind_ == Kind::Null; }
    bool is_bool() const { return kind_ == Kind::Bool; }
    bool is_number() const { return kind_ == Kind::Number; }
    // a number written or built as an integer (serde_json's is_u64/is_i64)
    bool is_integer() const { return kind_ == Kind::Number && integer_; }
    bool is_string() const { return kind_ == Kind::String; }
    bool is_array() const { return kind_ == Kind::Array; }
    bool is_object() const { return kind_ == Kind::Object; }

    bool as_bool() const { return b_; }
    double as_number() const { return n_; }
    const std::string &as_string() const { return s_; }
    const Array &as_array() const { return elements(); }
    Array &as_array() { elements(); own(); return *a_; }
    const Object &as_object() const { return members(); }
    Object &as_object() { members(); own(); return *o_; }

    // Object member access; a missing key of a const object reads as null.
    const Json &operator[](const std::string &key) const {
        static const Json null;
        if (kind_ != Kind::Object) return null;
        auto it = o_->find(key);
        return it == o_->end() ? null : it->second;
    }
    Json &operator[](const std::string &key) {
        if (kind_ == Kind::Null) *this = object();
        if (kind_ != Kind::Object) throw std::runtime_error("not a JSON object");
        own();
        return (*o_)[key];
    }
    const Json &operator[](const char *key) const { return (*this)[std::string(key)]; }
    Json &operator[](const char *key) { return (*this)[std::string(key)]; }
    // Array element access (bounds checked).
    const Json &operator[](size_t i) const { return elements().at(i); }
    const Json &operator[](int i) const { return elements().at((size_t)i); }
    Json &operator[](size_t i) { elements(); own(); return a_->at(i); }
    Json &operator[](int i) { elements(); own(); return a_->at((size_t)i); }
    void push_back(Json v) {
        if (kind_ == Kind::Null) *this = array();
        own();
        a_->push_back(std::move(v));
    }
    size_t size() const {
        return kind_ == Kind::Array ? a_->size() : kind_ == Kind::Object ? o_->size() : 0;
    }

    bool operator==(const Json &o) const {
        if (kind_ != o.kind_) return false;
        switch (kind_) {
            case Kind::Null: return true;
            case Kind::Bool: return b_ == o.b_;
            case Kind::Number: return n_ == o.n_;
            case Kind::String: return s_ == o.s_;
            case Kind::Array: return *a_ == *o.a_;
            case Kind::Object: return *o_ == *o.o_;
        }
        return false;
    }
    bool operator!=(const Json &o) const { return !(*this == o); }

    // The shortest decimal digits that read back as x, and the exponent e
    // of the first digit (x = d1.d2d3... * 10^e). x finite.
    static void shortest_digits(double x, std::string &digits, int &exponent, bool &negative) {
        char buf[64];
        auto r = std::to_chars(buf, buf + sizeof buf, x, std::chars_format::scientific);
        std::string t(buf, r.ptr);
        negative = t[0] == '-';
        if (negative) t.erase(0, 1);
        size_t e = t.find('e');
        exponent = std::stoi(t.substr(e + 1));
        digits.clear();
        for (size_t i = 0; i < e; i++)
            if (t[i] != '.') digits += t[i];
    }

    // serde_json's float text (ryu's format: plain decimal with a ".0" for
    // integral values while the decimal point stays within 21 digits, down
    // to 1e-6, and d.ddde[-]x otherwise).
    static std::string float_text(double x) {
        std::string digits;
        int e;
        bool neg;
        shortest_digits(x, digits, e, neg);
        std::string out = neg ? "-" : "";
        const int n = (int)digits.size();
        const int kk = e + 1;  // digits before the decimal point
        if (x == 0) {
            out += "0.0";
        } else if (n <= kk && kk <= 21) {
            out += digits + std::string((size_t)(kk - n), '0') + ".0";
        } else if (0 < kk && kk <= 21) {
            out += digits.substr(0, (size_t)kk) + "." + digits.substr((size_t)kk);
        } else if (-6 < kk && kk <= 0) {
            out += "0." + std::string((size_t)(-kk), '0') + digits;
        } else {
            out += digits.substr(0, 1);
            if (n > 1) out += "." + digits.substr(1);
            out += "e" + std::to_string(e);
        }
        return out;
    }

    std::string dump() const {
        std::string out;
        write(out);
        return out;
    }

    // Strict RFC 8259 parse of the whole text; throws std::runtime_error.
    static Json parse(const std::string &text) {
        size_t at = 0;
        Json v = parse_value(text, at, 0);
        skip_ws(text, at);
        if (at != text.size()) throw std::runtime_error("trailing characters after JSON value");
        return v;
    }

private:
    Kind kind_ = Kind::Null;
    bool b_ = false;
    bool integer_ = false;
    double n_ = 0.0;
    std::string s_;
    std::shared_ptr<Array> a_;
    std::shared_ptr<Object> o_;

    const Array &elements() const {
        if (kind_ != Kind::Array) throw std::runtime_error("not a JSON array");
        return *a_;
    }
    const Object &members() const {
        if (kind_ != Kind::Object) throw std::runtime_error("not a JSON object");
        return *o_;
    }

    // copy on write: values share containers until one is modified
    void own() {
        if (kind_ == Kind::Array && a_.use_count() > 1) a_ = std::make_shared<Array>(*a_);
        if (kind_ == Kind::Object && o_.use_count() > 1) o_ = std::make_shared<Object>(*o_);
    }

    static void write_string(std::string &out, const std::string &s) {
        out += '"';
        for (unsigned char c : s) {
            switch (c) {
                case '"': out += "\\\""; break;
                case '\\': out += "\\\\"; break;
                case '\n': out += "\\n"; break;
                case '\r': out += "\\r"; break;
                case '\t': out += "\\t"; break;
                case '\b': out += "\\b"; break;
                case '\f': out += "\\f"; break;
                default:
                    if (c < 0x20) {
                        char buf[8];
                        snprintf(buf, sizeof buf, "\\u%04x", c);
                        out += buf;
                    } else {
                        out += (char)c;
                    }
            }
        }
        out += '"';
    }

    void write(std::string &out) const {
        switch (kind_) {
            case Kind::Null: out += "null"; break;
            case Kind::Bool: out += b_ ? "true" : "false"; break;
            case Kind::Number: {
                if (!std::isfinite(n_)) {
                    out += "null";  // serde_json writes non-finite floats as null
                } else if (integer_) {
                    char buf[32];
                    if (n_ < 0) snprintf(buf, sizeof buf, "%lld", (long long)n_);
                    else snprintf(buf, sizeof buf, "%llu", (unsigned long long)n_);
                    out += buf;
                } else {
                    out += float_text(n_);
                }
                break;
            }
            case Kind::String: write_string(out, s_); break;
            case Kind::Array: {
                out += '[';
                for (size_t i = 0; i < a_->size(); i++) {
                    if (i) out += ',';
                    (*a_)[i].write(out);
                }
                out += ']';
                break;
            }
            case Kind::Object: {
                out += '{';
                bool first = true;
                for (const auto &kv : *o_) {
                    if (!first) out += ',';
                    first = false;
                    write_string(out, kv.first);
                    out += ':';
                    kv.second.write(out);
                }
                out += '}';
                break;
            }
        }
    }

    static void skip_ws(const std::string &t, size_t &at) {
        while (at < t.size() && (t[at] == ' ' || t[at] == '\n' || t[at] == '\r' || t[at] == '\t')) at++;
    }

    static void expect(const std::string &t, size_t &at, const char *word) {
        for (const char *p = word; *p; p++, at++)
            if (at >= t.size() || t[at] != *p) throw std::runtime_error("invalid JSON literal");
    }

    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }

    static uint32_t hex4(const std::string &t, size_t &at) {
        if (at + 4 > t.size()) throw std::runtime_error("truncated JSON escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            char c = t[at++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else throw std::runtime_error("invalid JSON escape");
        }
        return v;
    }

    static std::string parse_string(const std::string &t, size_t &at) {
        if (t[at] != '"') throw std::runtime_error("expected JSON string");
        at++;
        std::string out;
        while (true) {
            if (at >= t.size()) throw std::runtime_error("unterminated JSON string");
            unsigned char c = (unsigned char)t[at++];
            if (c == '"') break;
            if (c < 0x20) throw std::runtime_error("control character in JSON string");
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (at >= t.size()) throw std::runtime_error("unterminated JSON escape");
            char e = t[at++];
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
                    uint32_t cp = hex4(t, at);
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        if (at + 2 > t.size() || t[at] != '\\' || t[at + 1] != 'u')
                            throw std::runtime_error("unpaired JSON surrogate");
                        at += 2;
                        uint32_t lo = hex4(t, at);
                        if (lo < 0xDC00 || lo >= 0xE000) throw std::runtime_error("invalid JSON surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        throw std::runtime_error("unpaired JSON surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: throw std::runtime_error("invalid JSON escape");
            }
        }
        return out;
    }

    static Json parse_number(const std::string &t, size_t &at) {
        size_t start = at;
        if (t[at] == '-') at++;
        if (at >= t.size()) throw std::runtime_error("invalid JSON number");
        if (t[at] == '0') {
            at++;
        } else if (t[at] >= '1' && t[at] <= '9') {
            while (at < t.size() && isdigit((unsigned char)t[at])) at++;
        } else {
            throw std::runtime_error("invalid JSON number");
        }
        if (at < t.size() && t[at] == '.') {
            at++;
            if (at >= t.size() || !isdigit((unsigned char)t[at])) throw std::runtime_error("invalid JSON number");
            while (at < t.size() && isdigit((unsigned char)t[at])) at++;
        }
        if (at < t.size() && (t[at] == 'e' || t[at] == 'E')) {
            at++;
            if (at < t.size() && (t[at] == '+' || t[at] == '-')) at++;
            if (at >= t.size() || !isdigit((unsigned char)t[at])) throw std::runtime_error("invalid JSON number");
            while (at < t.size() && isdigit((unsigned char)t[at])) at++;
        }
        std::string text = t.substr(start, at - start);
        Json v(std::stod(text));
        // serde_json keeps integer literals within u64/i64 as integers
        bool plain = text.find_first_of(".eE") == std::string::npos;
        if (plain && v.n_ >= -9.223372036854775808e18 && v.n_ < 1.8446744073709551616e19) v.integer_ = true;
        return v;
    }

    static Json parse_value(const std::string &t, size_t &at, int depth) {
        if (depth > 128) throw std::runtime_error("JSON nested too deeply");
        skip_ws(t, at);
        if (at >= t.size()) throw std::runtime_error("unexpected end of JSON");
        char c = t[at];
        if (c == 'n') { expect(t, at, "null"); return Json(); }
        if (c == 't') { expect(t, at, "true"); return Json(true); }
        if (c == 'f') { expect(t, at, "false"); return Json(false); }
        if (c == '"') return Json(parse_string(t, at));
        if (c == '[') {
            at++;
            Json arr = array();
            skip_ws(t, at);
            if (at < t.size() && t[at] == ']') { at++; return arr; }
            while (true) {
                arr.push_back(parse_value(t, at, depth + 1));
                skip_ws(t, at);
                if (at >= t.size()) throw std::runtime_error("unterminated JSON array");
                if (t[at] == ',') { at++; continue; }
                if (t[at] == ']') { at++; return arr; }
                throw std::runtime_error("expected , or ] in JSON array");
            }
        }
        if (c == '{') {
            at++;
            Json obj = object();
            skip_ws(t, at);
            if (at < t.size() && t[at] == '}') { at++; return obj; }
            while (true) {
                skip_ws(t, at);
                if (at >= t.size() || t[at] != '"') throw std::runtime_error("expected JSON object key");
                std::string key = parse_string(t, at);
                skip_ws(t, at);
                if (at >= t.size() || t[at] != ':') throw std::runtime_error("expected : in JSON object");
                at++;
                obj[key] = parse_value(t, at, depth + 1);
                skip_ws(t, at);
                if (at >= t.size()) throw std::runtime_error("unterminated JSON object");
                if (t[at] == ',') { at++; continue; }
                if (t[at] == '}') { at++; return obj; }
                throw std::runtime_error("expected , or } in JSON object");
            }
        }
        if (c == '-' || (c >= '0' && c <= '9')) return parse_number(t, at);
        throw std::runtime_error("unexpected character in JSON");
    }
};

}  // namespace decisive
