// Kernel-registry side of the drop-in: the gfx950 candidates this library
// qualifies, and a C++ restatement of the reference's selection so the
// candidates can be checked against the reference's rules without Rust.
//
//   candidates        <- QuantizationDefinition::kernel_candidates
//                        (gguf_codegen.rs:50-113, mlx_affine.rs:157-238)
//   registry_select   <- KernelRegistry::select (crates/dyninfer-kernel-registry/src/lib.rs:302-348)
//   rejection_reasons <- rejection_reasons (lib.rs:499-584)
//   score             <- DeterministicCostModel::score (lib.rs:249-268)
//   require error     <- KernelRegistry::require's E_KERNEL_COVERAGE (lib.rs:350-399)
//   precision_check   <- the compiler's precision gate (crates/dyninfer-compiler/src/lib.rs:289-306),
//                        relaxed for bf16-activation candidates of this library
#include <algorithm>
#include <cctype>
#include <string>
#include <vector>

#include "json.hpp"
#include "registry.hpp"

namespace dmx {

using json::Value;

namespace {

Value strings(std::initializer_list<const char*> xs) {
    Value a = Value::array();
    for (const char* x : xs) a.push(Value::string(x));
    return a;
}

// One serde KernelCandidateDescriptor (lib.rs:132-149) for a gfx950 kernel;
// `act` is its activation type (input and output), accumulation is f32.
Value candidate(const std::string& codec, const char* op_kind, const char* op_suffix, long long block,
                const std::string& notes, const char* act = "f32") {
    Value c = Value::object();
    const std::string id = codec + "." + op_suffix + ".mi355x_hip";
    c.set("id", Value::string(id));
    c.set("operation", Value::string(op_kind));
    Value enc = Value::object();
    enc.set("id", Value::string(codec));
    enc.set("version", Value::integer(1));
    c.set("encoding", enc);
    c.set("input_types", strings({act}));
    c.set("output_types", strings({act}));
    c.set("accumulator_types", strings({"f32"}));
    Value shape = Value::object();
    shape.set("logical_rank", Value::integer(2));
    Value am = Value::array();
    Value m = Value::object();
    m.set("axis", Value::integer(1));
    m.set("multiple_of", Value::integer(block));
    am.push(m);
    shape.set("axis_multiples", am);
    c.set("shape", shape);
    c.set("orientations", strings({"native"}));
    Value target = Value::object();
    target.set("backends", strings({"hip", "rocm"}));
    target.set("exact_architectures", strings({"gfx950"}));
    c.set("target", target);
    c.set("modes", strings({"prefill", "decode"}));
    c.set("lowering", Value::string(id));
    // 400 > the IREE HIP entries' 300: both earn the +1000 exact-backend bonus
    // on driver "hip", so this entry wins on gfx950 and is rejected elsewhere.
    // The bf16-activation entries score 390: a request that names no activation
    // type (every request the reference makes) keeps selecting the f32 entry.
    c.set("deterministic_score", Value::integer(std::string(act) == "f32" ? 400 : 390));
    c.set("readiness", Value::string("production"));
    c.set("notes", Value::string(notes));
    return c;
}

}  // namespace

const std::string& candidates_json() {
    static const std::string s = [] {
        Value all = Value::array();
        // gguf.q4_k, gguf.q5_k and gguf.iq4_xs are schema-only encodings in the reference
        // (gguf_block.rs:183-316): these entries give them their first kernels, decoding
        // GGML's block_q4_K / block_q5_K / block_iq4_xs.
        struct G { const char* codec; long long block; bool gemm; };  // gemm: a prefill GEMM exists
        const G gguf[] = {{"gguf.q4_0", 32, true}, {"gguf.q4_1", 32, true}, {"gguf.q8_0", 32, true},
                          {"gguf.q6_k", 256, true}, {"gguf.q4_k", 256, true}, {"gguf.q5_k", 256, true},
                          {"gguf.iq4_xs", 256, true}};
        for (const G& g : gguf) {
            const bool gemm = g.gemm;
            const std::string n = std::string("Consumes official GGML ") + g.codec +
                                  " interleaved blocks in place on gfx950: wave64 GEMV for 1-16 rows "
                                  "(in-register dequantisation, f32 accumulation)" +
                                  (gemm ? "; prefill GEMM decodes the blocks in registers straight into f16 MFMA "
                                          "operands"
                                        : "") +
                                  "; activations rounded to f16 after a power-of-two scaling";
            all.push(candidate(g.codec, "embedding", "gather", g.block,
                               std::string("Gathers rows of official GGML ") + g.codec +
                                   " blocks in place on gfx950 and dequantises them to f32 (bit-exact)"));
            all.push(candidate(g.codec, "linear", "matmul", g.block, n + "; f32 in/out"));
            all.push(candidate(g.codec, "output_projection", "output", g.block, n + "; f32 in/out"));
            all.push(candidate(g.codec, "linear", "matmul_bf16", g.block, n + "; bf16 in/out", "bf16"));
            all.push(candidate(g.codec, "output_projection", "output_bf16", g.block, n + "; bf16 in/out", "bf16"));
        }
        const std::string mlx = "Direct MLX U4 words with groupwise scale/bias on gfx950 (group size a multiple "
                                "of 32), dequantised in registers next to the contraction";
        all.push(candidate("mlx.affine.u4", "embedding", "embedding", 32,
                           "Gathers rows of MLX U4 words with groupwise scale/bias on gfx950 and dequantises them "
                           "to f32 (bit-exact)"));
        all.push(candidate("mlx.affine.u4", "linear", "matmul", 32, mlx + "; f32 in/out"));
        all.push(candidate("mlx.affine.u4", "output_projection", "output", 32, mlx + "; f32 in/out"));
        all.push(candidate("mlx.affine.u4", "linear", "matmul_bf16", 32, mlx + "; bf16 in/out", "bf16"));
        all.push(candidate("mlx.affine.u4", "output_projection", "output_bf16", 32, mlx + "; bf16 in/out", "bf16"));
        return json::dump(all);
    }();
    return s;
}

namespace {

const Value& need(const Value& o, const char* k, const char* what) {
    const Value* v = o.get(k);
    if (!v) throw std::runtime_error(std::string(what) + " is missing field `" + k + "`");
    return *v;
}

const Value* opt(const Value& o, const char* k) {
    const Value* v = o.get(k);
    return (v && !v->is_null()) ? v : nullptr;
}

bool contains(const Value* arr, const std::string& s) {
    if (!arr || arr->kind != Value::Array) return false;
    for (const Value& v : arr->arr)
        if (v.kind == Value::String && v.str == s) return true;
    return false;
}

bool encoding_eq(const Value* a, const Value* b) {
    if (!a || !b) return !a && !b;
    return need(*a, "id", "encoding").as_str() == need(*b, "id", "encoding").as_str() &&
           need(*a, "version", "encoding").as_u64() == need(*b, "version", "encoding").as_u64();
}

// KernelOperationKind::is_precision_sensitive (lib.rs:61-66).
bool precision_sensitive(const std::string& op) {
    return op == "rms_norm" || op == "per_head_rms_norm" || op == "rope" || op == "attention";
}

Value reason(const char* name) {
    Value r = Value::object();
    r.set("reason", Value::string(name));
    return r;
}

std::string sensitive_type(const Value& request) {
    const Value* pp = opt(request, "precision_policy");
    if (pp) {
        const Value* t = opt(*pp, "sensitive_internal_type");
        if (t) return t->as_str();
    }
    return "f32";  // PrecisionPolicy::default (crates/dyninfer-core/src/ir.rs:214-227)
}

Value rejection_reasons(const Value& c, const Value& request, const Value& target) {
    Value reasons = Value::array();
    if (!encoding_eq(opt(c, "encoding"), opt(request, "encoding"))) reasons.push(reason("encoding_mismatch"));
    if (need(c, "readiness", "candidate").as_str() != "production") reasons.push(reason("not_production_ready"));
    if (!contains(&need(c, "modes", "candidate"), need(request, "mode", "request").as_str()))
        reasons.push(reason("mode_mismatch"));
    const Value& tc = need(c, "target", "candidate");
    const std::string driver = need(target, "driver", "target").as_str();
    bool backend_ok = false;
    for (const Value& b : need(tc, "backends", "target constraint").arr)
        if (b.as_str() == "any" || b.as_str() == driver) backend_ok = true;
    if (!backend_ok) {
        Value r = reason("backend_mismatch");
        r.set("selected", Value::string(driver));
        reasons.push(r);
    }
    const Value* exact = opt(tc, "exact_architectures");
    const Value* arch = opt(target, "architecture");
    if (exact && !exact->arr.empty() && !(arch && contains(exact, arch->as_str()))) {
        Value r = reason("architecture_mismatch");
        r.set("selected", arch ? *arch : Value::null());
        reasons.push(r);
    }
    const Value* req_features = opt(tc, "required_features");
    const Value* features = opt(target, "features");
    if (req_features)
        for (const Value& f : req_features->arr)
            if (!contains(features, f.as_str())) {
                Value r = reason("missing_target_feature");
                r.set("feature", f);
                reasons.push(r);
            }
    const Value* shape = opt(request, "logical_shape");
    const Value* cshape = opt(c, "shape");
    if (shape && cshape) {
        const Value* rank = opt(*cshape, "logical_rank");
        if (rank && (unsigned long long)shape->arr.size() != rank->as_u64()) {
            Value r = reason("rank_mismatch");
            r.set("expected", *rank);
            r.set("actual", Value::integer((long long)shape->arr.size()));
            reasons.push(r);
        }
    }
    if (shape && cshape) {
        const Value* ams = opt(*cshape, "axis_multiples");
        if (ams)
            for (const Value& am : ams->arr) {
                const unsigned long long axis = need(am, "axis", "axis multiple").as_u64();
                const unsigned long long mult = need(am, "multiple_of", "axis multiple").as_u64();
                if (axis < shape->arr.size()) {
                    const unsigned long long dim = shape->arr[axis].as_u64();
                    if (mult == 0 || dim % mult != 0) {
                        Value r = reason("axis_not_divisible");
                        r.set("axis", Value::integer((long long)axis));
                        r.set("dimension", shape->arr[axis]);
                        r.set("multiple_of", Value::integer((long long)mult));
                        reasons.push(r);
                    }
                }
            }
    }
    const Value* ors = opt(c, "orientations");
    if (ors && !ors->arr.empty() && !contains(ors, need(request, "orientation", "request").as_str()))
        reasons.push(reason("orientation_mismatch"));
    const Value& it = need(c, "input_types", "candidate");
    const Value& ot = need(c, "output_types", "candidate");
    const Value& at = need(c, "accumulator_types", "candidate");
    const std::string op = need(request, "operation", "request").as_str();
    // Extension (no reference counterpart): a request may name the model's
    // activation type; a linear or output candidate must then take it.
    const Value* act = opt(request, "activation_type");
    if (act && (op == "linear" || op == "output_projection") && !it.arr.empty() &&
        it.arr[0].as_str() != act->as_str()) {
        Value r = reason("activation_type_mismatch");
        r.set("required", *act);
        r.set("supported", it);
        reasons.push(r);
    }
    if (it.arr.empty() || ot.arr.empty() || at.arr.empty()) {
        reasons.push(reason("missing_type_choice"));
    } else if (precision_sensitive(op) && !contains(&at, sensitive_type(request))) {
        Value r = reason("precision_floor");
        r.set("required", Value::string(sensitive_type(request)));
        r.set("supported", at);
        reasons.push(r);
    }
    return reasons;
}

long long score(const Value& c, const Value& target) {
    const std::string driver = need(target, "driver", "target").as_str();
    long long bonus = 0;
    for (const Value& b : need(need(c, "target", "candidate"), "backends", "target constraint").arr)
        if (b.as_str() == driver) bonus = 1000;
    return need(c, "deterministic_score", "candidate").as_int() + bonus;
}

}  // namespace

int registry_select(const char* candidates, const char* request_json, const char* target_json, bool require,
                    std::string& out, std::string& err) {
    try {
        const Value cands = json::Parser(candidates ? candidates : candidates_json().c_str()).parse();
        const Value request = json::Parser(request_json).parse();
        const Value target = json::Parser(target_json).parse();
        if (cands.kind != Value::Array) throw std::runtime_error("candidates must be a JSON array");
        // KernelRegistry::register rejects duplicate ids (lib.rs:283-296).
        std::vector<std::string> seen;
        for (const Value& c : cands.arr) {
            const std::string id = need(c, "id", "candidate").as_str();
            if (std::find(seen.begin(), seen.end(), id) != seen.end()) {
                err = "duplicate kernel candidate `" + id + "`";
                return 1;
            }
            seen.push_back(id);
        }
        const std::string op = need(request, "operation", "request").as_str();
        struct Accepted { Value sel; long long score; std::string id; };
        std::vector<Accepted> accepted;
        Value rejected = Value::array();
        for (const Value& c : cands.arr) {
            if (need(c, "operation", "candidate").as_str() != op) continue;
            Value reasons = rejection_reasons(c, request, target);
            const std::string id = need(c, "id", "candidate").as_str();
            if (reasons.arr.empty()) {
                Value sel = Value::object();
                sel.set("descriptor", c);
                const Value& it = need(c, "input_types", "candidate").arr[0];
                sel.set("input_type", it);
                sel.set("output_type", need(c, "output_types", "candidate").arr[0]);
                sel.set("activation_type", it);
                sel.set("accumulator_type", precision_sensitive(op)
                                                ? Value::string(sensitive_type(request))
                                                : need(c, "accumulator_types", "candidate").arr[0]);
                const long long sc = score(c, target);
                sel.set("score", Value::integer(sc));
                accepted.push_back({sel, sc, id});
            } else {
                Value r = Value::object();
                r.set("candidate_id", Value::string(id));
                r.set("reasons", reasons);
                rejected.push(r);
            }
        }
        // best score first, ties by ascending id (lib.rs:338-343)
        std::stable_sort(accepted.begin(), accepted.end(), [](const Accepted& a, const Accepted& b) {
            if (a.score != b.score) return a.score > b.score;
            return a.id < b.id;
        });
        if (require) {
            if (accepted.empty()) {
                const Value* enc = opt(request, "encoding");
                const std::string encs = enc ? need(*enc, "id", "encoding").as_str() + "@" +
                                                   std::to_string(need(*enc, "version", "encoding").as_u64())
                                             : "none";
                std::string rej;
                for (const Value& r : rejected.arr) {
                    if (!rej.empty()) rej += "; ";
                    rej += r.get("candidate_id")->str + ": " + json::dump(*r.get("reasons"));
                }
                const Value* oid = opt(request, "operation_id");
                err = "E_KERNEL_COVERAGE: no production kernel for " + op + " with encoding " + encs + " in " +
                      need(request, "mode", "request").as_str() + " mode (operation " +
                      (oid ? oid->as_str() : std::string("?")) + "); rejected candidates: " +
                      (rej.empty() ? std::string("none registered") : rej);
                return 2;
            }
            out = json::dump(accepted[0].sel);
            return 0;
        }
        Value report = Value::object();
        if (!accepted.empty()) report.set("selected", accepted[0].sel);
        report.set("rejected", rejected);
        out = json::dump(report);
        return 0;
    } catch (const std::exception& e) {
        err = e.what();
        return 1;
    }
}

namespace {

// Rust Debug spelling of a serde ScalarType (crates/dyninfer-core/src/scalar.rs:9-23).
std::string scalar_debug(const std::string& t) {
    if (t == "bf16") return "Bf16";
    if (t == "bool") return "Bool";
    std::string d = t;
    if (!d.empty()) d[0] = (char)std::toupper((unsigned char)d[0]);
    return d;
}

}  // namespace

int precision_check(const char* selected_json, const char* activation_type, std::string& err) {
    try {
        const Value sel = json::Parser(selected_json).parse();
        const std::string in = need(sel, "input_type", "selected kernel").as_str();
        const std::string out = need(sel, "output_type", "selected kernel").as_str();
        const std::string act = need(sel, "activation_type", "selected kernel").as_str();
        const std::string acc = need(sel, "accumulator_type", "selected kernel").as_str();
        const Value& desc = need(sel, "descriptor", "selected kernel");
        const std::string id = need(desc, "id", "descriptor").as_str();
        const std::string lowering = need(desc, "lowering", "descriptor").as_str();
        const std::string model_act = activation_type ? activation_type : "f32";
        // lib.rs:289-306: an i64 input (token ids) or f32 throughout
        if (in == "i64" || (in == "f32" && out == "f32" && act == "f32" && acc == "f32")) return 0;
        // relaxed: bf16 activations in and out with f32 accumulation, for a model whose
        // activations are bf16 and a lowering of this library (qualified for them)
        const std::string suffix = ".mi355x_hip";
        const bool ours = lowering.size() > suffix.size() &&
                          lowering.compare(lowering.size() - suffix.size(), suffix.size(), suffix) == 0;
        if (model_act == "bf16" && ours && in == "bf16" && out == "bf16" && act == "bf16" && acc == "f32") return 0;
        err = "selected kernel `" + id + "` requires " + scalar_debug(in) + "/" + scalar_debug(out) + "/" +
              scalar_debug(act) + "/" + scalar_debug(acc) +
              (model_act == "bf16"
                   ? ", but the shared lowering is qualified only for f32 compute, or bf16 activations with f32 "
                     "accumulation on a .mi355x_hip lowering"
                   : ", but the current shared lowering is qualified only for f32 compute") +
              " (lower.precision)";
        return 2;
    } catch (const std::exception& e) {
        err = e.what();
        return 1;
    }
}

}  // namespace dmx
