// Minimal JSON value, parser and writer for the kernel-registry boundary.
//
// The reference exchanges KernelCandidateDescriptor / KernelRequest /
// TargetProfile / SelectionReport through serde (crates/dyninfer-kernel-registry
// /src/lib.rs:18-223); this reader accepts that JSON (RFC 8259: objects keep
// member order, numbers keep their text, strings are UTF-8 with \u escapes).
#pragma once
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace dmx {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    std::string str;  // String payload, or the number's literal text
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    static Value null() { return Value(); }
    static Value boolean(bool v) { Value x; x.kind = Bool; x.b = v; return x; }
    static Value string(std::string s) { Value x; x.kind = String; x.str = std::move(s); return x; }
    static Value integer(long long v) { Value x; x.kind = Number; x.str = std::to_string(v); return x; }
    static Value array() { Value x; x.kind = Array; return x; }
    static Value object() { Value x; x.kind = Object; return x; }

    bool is_null() const { return kind == Null; }
    const Value* get(const std::string& k) const {
        if (kind != Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    Value& set(const std::string& k, Value v) {
        for (auto& kv : obj)
            if (kv.first == k) { kv.second = std::move(v); return kv.second; }
        obj.emplace_back(k, std::move(v));
        return obj.back().second;
    }
    void push(Value v) { arr.push_back(std::move(v)); }
    long long as_int() const {
        if (kind != Number) throw std::runtime_error("expected a number");
        size_t pos = 0;
        long long v = std::stoll(str, &pos);
        if (pos != str.size()) throw std::runtime_error("expected an integer, got " + str);
        return v;
    }
    unsigned long long as_u64() const {
        if (kind != Number || str.empty() || str[0] == '-') throw std::runtime_error("expected an unsigned integer");
        size_t pos = 0;
        unsigned long long v = std::stoull(str, &pos);
        if (pos != str.size()) throw std::runtime_error("expected an integer, got " + str);
        return v;
    }
    const std::string& as_str() const {
        if (kind != String) throw std::runtime_error("expected a string");
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
    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("invalid JSON: ") + what); }
    void ws() { while (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r') p_++; }
    bool lit(const char* w) {
        size_t n = std::char_traits<char>::length(w);
        if (std::char_traits<char>::compare(p_, w, n) == 0) { p_ += n; return true; }
        return false;
    }
    Value value() {
        ws();
        switch (*p_) {
        case '{': return object();
        case '[': return array();
        case '"': return Value::string(string());
        case 't': if (lit("true")) return Value::boolean(true); break;
        case 'f': if (lit("false")) return Value::boolean(false); break;
        case 'n': if (lit("null")) return Value::null(); break;
        default:
            if (*p_ == '-' || (*p_ >= '0' && *p_ <= '9')) return number();
        }
        fail("unexpected token");
    }
    Value number() {
        const char* s = p_;
        if (*p_ == '-') p_++;
        if (!(*p_ >= '0' && *p_ <= '9')) fail("bad number");
        while ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' || *p_ == '-') p_++;
        Value v;
        v.kind = Value::Number;
        v.str.assign(s, p_);
        return v;
    }
    static void utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
        else { o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
    }
    uint32_t hex4() {
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        std::string o;
        p_++;  // opening quote
        while (*p_ != '"') {
            if (!*p_) fail("unterminated string");
            if (*p_ == '\\') {
                p_++;
                switch (*p_++) {
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
                    if (cp >= 0xD800 && cp < 0xDC00 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(o, cp);
                    break;
                }
                default: fail("bad escape");
                }
            } else {
                o += *p_++;
            }
        }
        p_++;
        return o;
    }
    Value array() {
        Value v = Value::array();
        p_++;
        ws();
        if (*p_ == ']') { p_++; return v; }
        for (;;) {
            v.push(value());
            ws();
            if (*p_ == ',') { p_++; continue; }
            if (*p_ == ']') { p_++; return v; }
            fail("expected , or ]");
        }
    }
    Value object() {
        Value v = Value::object();
        p_++;
        ws();
        if (*p_ == '}') { p_++; return v; }
        for (;;) {
            ws();
            if (*p_ != '"') fail("expected a key");
            std::string k = string();
            ws();
            if (*p_++ != ':') fail("expected :");
            v.obj.emplace_back(std::move(k), value());
            ws();
            if (*p_ == ',') { p_++; continue; }
            if (*p_ == '}') { p_++; return v; }
            fail("expected , or }");
        }
    }
};

inline void write_string(std::string& o, const std::string& s) {
    o += '"';
    for (unsigned char c : s) {
        switch (c) {
        case '"': o += "\\\""; break;
        case '\\': o += "\\\\"; break;
        case '\n': o += "\\n"; break;
        case '\r': o += "\\r"; break;
        case '\t': o += "\\t"; break;
        default:
            if (c < 0x20) {
                char buf[8];
                static const char* hx = "0123456789abcdef";
                buf[0] = '\\'; buf[1] = 'u'; buf[2] = '0'; buf[3] = '0'; buf[4] = hx[c >> 4]; buf[5] = hx[c & 15]; buf[6] = 0;
                o += buf;
            } else {
                o += (char)c;
            }
        }
    }
    o += '"';
}

inline void write(std::string& o, const Value& v) {
    switch (v.kind) {
    case Value::Null: o += "null"; break;
    case Value::Bool: o += v.b ? "true" : "false"; break;
    case Value::Number: o += v.str; break;
    case Value::String: write_string(o, v.str); break;
    case Value::Array:
        o += '[';
        for (size_t i = 0; i < v.arr.size(); i++) { if (i) o += ','; write(o, v.arr[i]); }
        o += ']';
        break;
    case Value::Object:
        o += '{';
        for (size_t i = 0; i < v.obj.size(); i++) {
            if (i) o += ',';
            write_string(o, v.obj[i].first);
            o += ':';
            write(o, v.obj[i].second);
        }
        o += '}';
        break;
    }
}

inline std::string dump(const Value& v) {
    std::string o;
    write(o, v);
    return o;
}

}  // namespace json
}  // namespace dmx
