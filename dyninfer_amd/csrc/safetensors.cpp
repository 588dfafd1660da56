// SafeTensors indexing (crates/dyninfer-checkpoint-safetensors/src/container.rs):
// 8-byte little-endian header length (1 .. 64 MiB), a UTF-8 JSON object header
// ("__metadata__" plus one {dtype, shape, data_offsets} entry per tensor, offsets
// relative to the end of the header), each tensor's byte length equal to
// numel x element size, inside the file, no two ranges overlapping; entries
// sorted by name.  And the MLX affine convention's weight (mlx.rs:17-261).
#include "safetensors.hpp"

#include <algorithm>
#include <cstring>

#include "gguf.hpp"
#include "json.hpp"

namespace dmx {

namespace {

// InspectionLimits::default() (crates/dyninfer-checkpoint/src/limits.rs)
constexpr uint64_t kMaxHeaderBytes = 64ull << 20, kMaxTensors = 1000000;
constexpr uint64_t kMaxKeyLen = 16 * 1024, kMaxRank = 16, kMaxDim = 1ull << 40, kMaxTotalBytes = 1ull << 50;

// parse_dtype (container.rs:24-46) and ScalarType::size_bytes
uint32_t dtype_size(const std::string& d) {
    static const std::pair<const char*, uint32_t> table[] = {
        {"F32", 4}, {"F16", 2}, {"BF16", 2}, {"F64", 8}, {"I8", 1},  {"I16", 2}, {"I32", 4},
        {"I64", 8}, {"U8", 1},  {"U16", 2},  {"U32", 4}, {"U64", 8}, {"BOOL", 1},
    };
    for (const auto& e : table)
        if (d == e.first) return e.second;
    return 0;
}

bool mul_ovf(uint64_t a, uint64_t b, uint64_t* r) { return __builtin_mul_overflow(a, b, r); }

// A JSON value as serde_json's Value::as_u64 reads it: a non-negative integer
// literal (no fraction or exponent), else "absent".
bool json_u64(const json::Value* v, uint64_t* out) {
    if (!v || v->kind != json::Value::Number) return false;
    try {
        *out = v->as_u64();
        return true;
    } catch (...) {
        return false;
    }
}

void note_quant(StIndex& idx, const std::string& key, const json::Value& v) {
    uint64_t u = 0;
    if (key == "mlx.quantization.bits" && !idx.has_bits && json_u64(&v, &u)) idx.has_bits = true, idx.bits = u;
    if (key == "mlx.quantization.group_size" && !idx.has_group && json_u64(&v, &u)) idx.has_group = true, idx.group = u;
    if (key == "format" && v.kind == json::Value::String) {
        std::string f = v.str;
        for (char& c : f) c = (char)std::tolower((unsigned char)c);
        idx.format_mlx = f == "mlx";
    }
}

void rebuild_metadata_json(StIndex& idx, std::vector<std::pair<std::string, json::Value>> meta) {
    std::sort(meta.begin(), meta.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
    json::Value o = json::Value::object();
    for (auto& kv : meta) o.obj.emplace_back(kv.first, std::move(kv.second));
    idx.metadata_json = json::dump(o);
}

}  // namespace

const StTensor* st_find(const StIndex& idx, const std::string& name) {
    auto it = std::lower_bound(idx.tensors.begin(), idx.tensors.end(), name,
                               [](const StTensor& t, const std::string& n) { return t.name < n; });
    return it != idx.tensors.end() && it->name == name ? &*it : nullptr;
}

std::string st_index(const uint8_t* base, uint64_t len, StIndex& idx) {
    idx.base = base;
    idx.len = len;
    if (len < 8) return "SafeTensors file shorter than its 8-byte header length";
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | base[i];
    if (hlen == 0 || hlen > kMaxHeaderBytes) return "invalid SafeTensors header length: " + std::to_string(hlen);
    if (len - 8 < hlen) return "SafeTensors header extends past end of file";
    const uint8_t* h = base + 8;
    if (!valid_utf8(h, hlen) || std::memchr(h, 0, (size_t)hlen))
        return "SafeTensors header JSON invalid: not UTF-8 text";
    json::Value root;
    try {
        root = json::Parser(std::string(reinterpret_cast<const char*>(h), (size_t)hlen).c_str()).parse();
    } catch (const std::exception& e) {
        return std::string("SafeTensors header JSON invalid: ") + e.what();
    }
    if (root.kind != json::Value::Object) return "SafeTensors header must be a JSON object";
    idx.data_base = 8 + hlen;
    std::vector<std::pair<std::string, json::Value>> meta;
    uint64_t total = 0;
    for (const auto& kv : root.obj) {
        const std::string& key = kv.first;
        if (key == "__metadata__") {
            if (kv.second.kind == json::Value::Object)
                for (const auto& m : kv.second.obj) meta.emplace_back(m.first, m.second);
            continue;
        }
        if (key.size() > kMaxKeyLen) return "key length " + std::to_string(key.size()) + " exceeds limit " + std::to_string(kMaxKeyLen);
        const json::Value& info = kv.second;
        const json::Value* dt = info.get("dtype");
        const json::Value* sh = info.get("shape");
        const json::Value* off = info.get("data_offsets");
        if (info.kind != json::Value::Object || !dt || dt->kind != json::Value::String || !sh ||
            sh->kind != json::Value::Array || !off || off->kind != json::Value::Array || off->arr.size() != 2)
            return "invalid tensor info: " + key;
        StTensor t;
        t.name = key;
        t.dtype = dt->str;
        for (const auto& d : sh->arr) {
            uint64_t u = 0;
            if (!json_u64(&d, &u)) return "invalid tensor info: " + key;
            t.shape.push_back(u);
        }
        uint64_t o0 = 0, o1 = 0;
        if (!json_u64(&off->arr[0], &o0) || !json_u64(&off->arr[1], &o1)) return "invalid tensor info: " + key;
        if (t.shape.size() > kMaxRank) return "rank " + std::to_string(t.shape.size()) + " exceeds limit " + std::to_string(kMaxRank);
        for (uint64_t d : t.shape)
            if (d > kMaxDim) return "dimension " + std::to_string(d) + " exceeds limit " + std::to_string(kMaxDim);
        if (o1 < o0) return "data_offsets end < start: " + key;
        const uint64_t length = o1 - o0;
        t.elem = dtype_size(t.dtype);
        if (!t.elem) return "unsupported SafeTensors dtype: " + t.dtype;
        uint64_t numel = 1, expect = 0;
        for (uint64_t d : t.shape)
            if (mul_ovf(numel, d, &numel)) return "shape numel overflow: " + key;
        if (mul_ovf(numel, t.elem, &expect)) return "declared tensor byte length overflow: " + key;
        if (length != expect)
            return "tensor byte length " + std::to_string(length) + " != numel " + std::to_string(numel) + " * elem " +
                   std::to_string(t.elem) + " (= " + std::to_string(expect) + "): " + key;
        if (o0 > UINT64_MAX - idx.data_base) return "tensor offset overflow: " + key;
        t.offset = idx.data_base + o0;
        t.nbytes = length;
        if (t.offset > len || len - t.offset < length) return "tensor data range extends past end of file: " + key;
        total = total + length < total ? UINT64_MAX : total + length;
        idx.tensors.push_back(std::move(t));
    }
    if (idx.tensors.size() > kMaxTensors)
        return "tensor count " + std::to_string(idx.tensors.size()) + " exceeds limit " + std::to_string(kMaxTensors);
    std::vector<const StTensor*> by_start;
    for (const auto& t : idx.tensors) by_start.push_back(&t);
    std::stable_sort(by_start.begin(), by_start.end(), [](const StTensor* a, const StTensor* b) { return a->offset < b->offset; });
    for (size_t i = 1; i < by_start.size(); i++)
        if (by_start[i]->offset < by_start[i - 1]->offset + by_start[i - 1]->nbytes)
            return "overlapping tensor byte ranges between `" + by_start[i - 1]->name + "` and `" + by_start[i]->name + "`";
    if (total > kMaxTotalBytes)
        return "total declared tensor bytes " + std::to_string(total) + " exceeds limit " + std::to_string(kMaxTotalBytes);
    std::sort(idx.tensors.begin(), idx.tensors.end(), [](const StTensor& a, const StTensor& b) { return a.name < b.name; });
    // A repeated name would give one key two byte ranges; the reference's JSON
    // map keeps only the last, which silently drops a range: rejected here.
    for (size_t i = 1; i < idx.tensors.size(); i++)
        if (idx.tensors[i].name == idx.tensors[i - 1].name) return "duplicate tensor name `" + idx.tensors[i].name + "`";
    for (const auto& m : meta) note_quant(idx, m.first, m.second);
    rebuild_metadata_json(idx, std::move(meta));
    return "";
}

void st_merge_config(StIndex& idx, const std::string& config_text) {
    json::Value cfg;
    try {
        cfg = json::Parser(config_text.c_str()).parse();
    } catch (...) {
        return;
    }
    if (cfg.kind != json::Value::Object) return;
    const json::Value* q = cfg.get("quantization_config");
    if (!q || q->kind != json::Value::Object) q = cfg.get("quantization");
    if (!q || q->kind != json::Value::Object) return;
    // entry(key).or_insert(value): header metadata wins
    json::Value meta;
    try {
        meta = json::Parser(idx.metadata_json.c_str()).parse();
    } catch (...) {
        return;
    }
    std::vector<std::pair<std::string, json::Value>> kv(meta.obj.begin(), meta.obj.end());
    auto add = [&](const char* from, const char* key) {
        const json::Value* v = q->get(from);
        uint64_t u = 0;
        if (!json_u64(v, &u)) return;
        for (const auto& e : kv)
            if (e.first == key) return;
        kv.emplace_back(key, *v);
        note_quant(idx, key, *v);
    };
    add("bits", "mlx.quantization.bits");
    add("group_size", "mlx.quantization.group_size");
    rebuild_metadata_json(idx, std::move(kv));
}

std::string st_mlx_weight(const StIndex& idx, const std::string& weight_key, const StTensor** packed,
                          const StTensor** scales, const StTensor** biases, uint64_t* n, uint64_t* k, uint64_t* group) {
    // the convention (match_score, mlx.rs:23-51; decode :53-136)
    if (!idx.format_mlx) return "not an MLX SafeTensors checkpoint (metadata `format` is not \"mlx\")";
    if (!idx.has_bits) return "missing required MLX metadata `mlx.quantization.bits`";
    if (!idx.has_group) return "missing required MLX metadata `mlx.quantization.group_size`";
    const uint64_t bits = idx.bits, g = idx.group;
    if (bits > UINT32_MAX || g > UINT32_MAX || !(bits == 2 || bits == 3 || bits == 4 || bits == 6 || bits == 8) || g == 0)
        return "unsupported MLX affine configuration bits=" + std::to_string(bits) + ", group_size=" + std::to_string(g);
    const size_t sfx = weight_key.size() >= 7 ? weight_key.size() - 7 : std::string::npos;
    if (sfx == std::string::npos || weight_key.compare(sfx, 7, ".weight") != 0)
        return "MLX quantized weight must be a `.weight` tensor: " + weight_key;
    const std::string stem = weight_key.substr(0, sfx);
    const StTensor* w = st_find(idx, weight_key);
    if (!w) return "no tensor named " + weight_key;
    const StTensor* s = st_find(idx, stem + ".scales");
    const StTensor* b = st_find(idx, stem + ".biases");
    if (!s || !b)
        return "MLX quantized weight must have both .scales and .biases components: " + weight_key + " (scales=" +
               (s ? "true" : "false") + ", biases=" + (b ? "true" : "false") + ")";
    // decode_affine_weight (mlx.rs:152-261)
    if (w->shape.empty()) return "MLX packed weight must have rank >= 1: " + weight_key;
    if (w->dtype != "U32") return "MLX packed weight storage must be u32: " + weight_key + " is " + w->dtype;
    auto float_type = [](const std::string& d) { return d == "F16" || d == "BF16" || d == "F32"; };
    if (s->dtype != b->dtype || !float_type(s->dtype))
        return "MLX scales and biases must use the same floating-point type: " + weight_key + " (scales=" + s->dtype +
               ", biases=" + b->dtype + ")";
    uint64_t num = 0;
    if (mul_ovf(w->shape.back(), 32, &num)) return "MLX logical shape overflow";
    if (num % bits) return "MLX packed axis cannot be expanded exactly: " + weight_key;
    const uint64_t logical_last = num / bits;
    if (logical_last % g) return "MLX logical quantization axis is not group divisible: " + weight_key;
    std::vector<uint64_t> gshape = w->shape;
    gshape.back() = logical_last / g;
    if (s->shape != gshape || b->shape != gshape) return "MLX scales/biases shape does not match logical groups: " + weight_key;
    // this library's kernels: 4-bit codes, rank-2 weights
    if (bits != 4) return "this library runs mlx.affine.u4 only; " + weight_key + " has " + std::to_string(bits) + "-bit codes";
    if (w->shape.size() != 2) return "tensor " + weight_key + " is not rank 2";
    *packed = w;
    *scales = s;
    *biases = b;
    *n = w->shape[0];
    *k = logical_last;
    *group = g;
    return "";
}

}  // namespace dmx
