// GGUF container indexing, restating container.rs:179-340 of
// crates/dyninfer-checkpoint-gguf: magic "GGUF", version 2 or 3, counts,
// metadata key/values (value types 0..12, arrays), tensor directory (name,
// rank, dims reversed to row-major, type, relative offset), data section at
// the header end rounded up to general.alignment (default 32, container.rs:16),
// every tensor's exact byte range checked against the file length.
#include "gguf.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "json.hpp"

namespace dmx {

// Well-formed UTF-8 (RFC 3629: no overlong forms, no surrogates, at most
// U+10FFFF), the check Rust's String::from_utf8 makes (container.rs:62-81).
bool valid_utf8(const uint8_t* s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) { i++; continue; }
        uint32_t len, cp;
        if (c >= 0xC2 && c <= 0xDF) { len = 2; cp = c & 0x1Fu; }
        else if (c >= 0xE0 && c <= 0xEF) { len = 3; cp = c & 0x0Fu; }
        else if (c >= 0xF0 && c <= 0xF4) { len = 4; cp = c & 0x07u; }
        else return false;
        if (n - i < len) return false;
        for (uint32_t k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0u) != 0x80u) return false;
            cp = (cp << 6) | (s[i + k] & 0x3Fu);
        }
        if ((len == 3 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)))
            return false;
        i += len;
    }
    return true;
}

namespace {

// InspectionLimits::default() (crates/dyninfer-checkpoint/src/limits.rs)
constexpr uint64_t kMaxHeaderBytes = 64ull << 20, kMaxTensors = 1000000, kMaxEntries = 1000000;
constexpr uint64_t kMaxKeyLen = 16 * 1024, kMaxRank = 16, kMaxDim = 1ull << 40;


struct Cursor {
    const uint8_t* p;
    uint64_t len, pos = 0;
    std::string err;
    bool need(uint64_t n) {
        if (!err.empty()) return false;
        if (n > len - pos) { err = "GGUF header truncated"; return false; }
        return true;
    }
    template <class T> T get() {
        T v{};
        if (!need(sizeof(T))) return v;
        std::memcpy(&v, p + pos, sizeof(T));  // the file is little-endian, as is the host
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!err.empty()) return {};
        if (n > kMaxKeyLen) { err = "GGUF string length " + std::to_string(n) + " exceeds limit"; return {}; }
        if (!need(n)) return {};
        if (!valid_utf8(p + pos, n)) { err = "GGUF string is not UTF-8"; return {}; }
        std::string s(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += n;
        return s;
    }
};

json::Value number_f64(double v) {
    if (!std::isfinite(v)) return json::Value::null();  // serde_json: non-finite -> null
    json::Value x = json::Value::integer(0);
    char buf[40];
    std::snprintf(buf, sizeof buf, "%.17g", v);
    x.str = buf;
    return x;
}

json::Value number_u64(uint64_t v) {
    json::Value x = json::Value::integer(0);
    x.str = std::to_string(v);
    return x;
}

json::Value read_value(Cursor& c, uint32_t type, int depth) {
    switch (type) {
    case 0: return json::Value::integer(c.get<uint8_t>());
    case 1: return json::Value::integer(c.get<int8_t>());
    case 2: return json::Value::integer(c.get<uint16_t>());
    case 3: return json::Value::integer(c.get<int16_t>());
    case 4: return json::Value::integer(c.get<uint32_t>());
    case 5: return json::Value::integer(c.get<int32_t>());
    case 6: return number_f64(c.get<float>());
    case 7: return json::Value::boolean(c.get<uint8_t>() != 0);
    case 8: return json::Value::string(c.str());
    case 9: {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (!c.err.empty()) return {};
        if (n > kMaxEntries) { c.err = "GGUF array length " + std::to_string(n) + " exceeds limit"; return {}; }
        if (depth > 8) { c.err = "GGUF arrays nested too deeply"; return {}; }
        json::Value a = json::Value::array();
        for (uint64_t i = 0; i < n && c.err.empty(); i++) a.push(read_value(c, et, depth + 1));
        return a;
    }
    case 10: return number_u64(c.get<uint64_t>());
    case 11: return json::Value::integer(c.get<int64_t>());
    case 12: return number_f64(c.get<double>());
    default:
        if (c.err.empty()) c.err = "unsupported GGUF metadata value type " + std::to_string(type);
        return {};
    }
}

}  // namespace

bool gguf_type_geometry(uint32_t code, uint64_t* block, uint64_t* bytes) {
    struct T { uint32_t code; uint64_t block, bytes; };
    static const T table[] = {  // types.rs:10-45, 137-201
        {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},    {7, 32, 24},   {8, 32, 34},
        {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292},
        {16, 256, 66}, {17, 256, 74}, {18, 256, 98}, {19, 256, 50},  {20, 32, 18},  {21, 256, 110}, {22, 256, 82},
        {23, 256, 136}, {24, 1, 1},   {25, 1, 2},    {26, 1, 4},    {27, 1, 8},     {28, 1, 8},    {29, 256, 56},
        {30, 1, 2},    {34, 256, 54}, {35, 256, 66}, {39, 32, 17},
    };
    for (const T& t : table)
        if (t.code == code) {
            *block = t.block;
            *bytes = t.bytes;
            return true;
        }
    return false;
}

std::string gguf_index(const uint8_t* base, uint64_t len, GgufIndex& idx) {
    Cursor c{base, len < kMaxHeaderBytes ? len : kMaxHeaderBytes};
    if (len < 4 || std::memcmp(base, "GGUF", 4) != 0) return "not a GGUF file (bad magic)";
    c.pos = 4;
    const uint32_t version = c.get<uint32_t>();
    if (c.err.empty() && (version < 2 || version > 3))
        return "unsupported GGUF version " + std::to_string(version) + " (supported: 2, 3)";
    const uint64_t ntensor = c.get<uint64_t>(), nkv = c.get<uint64_t>();
    if (!c.err.empty()) return c.err;
    if (ntensor > kMaxTensors || nkv > kMaxEntries)
        return "GGUF counts exceed limits: tensors=" + std::to_string(ntensor) + " kv=" + std::to_string(nkv);
    json::Value meta = json::Value::object();
    std::vector<std::pair<std::string, json::Value>> kvs;
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        std::string key = c.str();
        const uint32_t type = c.get<uint32_t>();
        json::Value v = read_value(c, type, 0);
        if (!c.err.empty()) return c.err;
        // general.alignment read as any unsigned integer (as_u64 in the reference)
        if (key == "general.alignment" && (type == 0 || type == 2 || type == 4 || type == 10)) alignment = std::stoull(v.str);
        if (key == "general.alignment" && (type == 1 || type == 3 || type == 5 || type == 11) && v.str[0] != '-')
            alignment = std::stoull(v.str);
        kvs.emplace_back(std::move(key), std::move(v));
    }
    std::stable_sort(kvs.begin(), kvs.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
    for (auto& kv : kvs) meta.set(kv.first, kv.second);  // later duplicates replace earlier ones
    struct Dir { std::string name; std::vector<uint64_t> shape; uint32_t type; uint64_t off; };
    std::vector<Dir> dirs;
    dirs.reserve((size_t)ntensor);
    for (uint64_t i = 0; i < ntensor; i++) {
        Dir d;
        d.name = c.str();
        const uint32_t rank = c.get<uint32_t>();
        if (!c.err.empty()) return c.err;
        if (rank > kMaxRank) return "GGUF tensor rank " + std::to_string(rank) + " exceeds limit (" + d.name + ")";
        for (uint32_t r = 0; r < rank; r++) d.shape.push_back(c.get<uint64_t>());
        std::reverse(d.shape.begin(), d.shape.end());
        d.type = c.get<uint32_t>();
        d.off = c.get<uint64_t>();
        if (!c.err.empty()) return c.err;
        for (uint64_t dim : d.shape)
            if (dim > kMaxDim) return "dimension " + std::to_string(dim) + " exceeds limit (" + d.name + ")";
        dirs.push_back(std::move(d));
    }
    // align_up as the reference computes it (div_ceil, then the multiple):
    // the quotient is at least 1, so the multiple overflows only for an
    // alignment beyond any file length, which is then reported as such
    uint64_t data = c.pos;
    if (alignment) {
        const uint64_t q = c.pos / alignment + (c.pos % alignment ? 1u : 0u);
        if (q > UINT64_MAX / alignment) return "GGUF data section offset overflows (general.alignment " + std::to_string(alignment) + ")";
        data = q * alignment;
    }
    idx.tensors.clear();
    for (Dir& d : dirs) {
        uint64_t block = 0, bytes = 0, numel = 1;
        if (!gguf_type_geometry(d.type, &block, &bytes)) return "unknown GGUF tensor type " + std::to_string(d.type) + " (" + d.name + ")";
        for (uint64_t dim : d.shape) {
            if (dim && numel > UINT64_MAX / dim) return "shape numel overflow (" + d.name + ")";
            numel *= dim;
        }
        if (numel % block) return "GGUF numel " + std::to_string(numel) + " not divisible by block " + std::to_string(block) + " (" + d.name + ")";
        const uint64_t nbytes = numel / block * bytes;
        if (d.off > UINT64_MAX - data) return "tensor absolute offset overflow (" + d.name + ")";
        const uint64_t abs = data + d.off;
        if (abs > len || nbytes > len - abs) return "tensor data extends past end of file (" + d.name + ")";
        idx.tensors.push_back({std::move(d.name), d.type, std::move(d.shape), abs, nbytes});
    }
    std::sort(idx.tensors.begin(), idx.tensors.end(), [](const GgufTensor& a, const GgufTensor& b) { return a.name < b.name; });
    for (size_t i = 1; i < idx.tensors.size(); i++)
        if (idx.tensors[i].name == idx.tensors[i - 1].name) return "duplicate GGUF tensor name " + idx.tensors[i].name;
    idx.base = base;
    idx.len = len;
    idx.version = version;
    idx.alignment = alignment;
    idx.metadata_json = json::dump(meta);
    return {};
}

}  // namespace dmx
