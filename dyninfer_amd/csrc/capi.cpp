// C ABI of the MI355X quantized weight-matmul library (include/dyninfer_mi355x.h).
//
// Host-side validation mirrors the reference's encoding checks
// (q4_0.rs:40-113, gguf_block.rs:66-156, mlx_affine.rs:55-155): unsupported
// encodings and shapes are rejected with DYNINFER_MI355X_ERR_UNSUPPORTED, never
// routed to a fallback (README.md:83-84 "never falls back to CPU").
#include "../../include/dyninfer_mi355x.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "safetensors.hpp"
#include "kernels.hpp"
#include "registry.hpp"

// Prefill staging workspace of the no-allocation entry point: one array per
// device, allocated when the code object loads and held until the process
// ends.  In host code `scratch` only names the symbol; the device address is
// taken once per context with hipGetSymbolAddress (ctx->scratch).
constexpr size_t kScratchBytes = DYNINFER_MI355X_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// A context: the device it was opened on and that device's copy of `scratch`.
// Immutable after dyninfer_mi355x_open, so calls from any number of threads
// share it without locks; each call's temporary lives in the caller's
// workspace (or, for the no-allocation entry point, in `scratch`).
struct dyninfer_mi355x_ctx {
    int device;
    uint8_t* scratch;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(DYNINFER_MI355X_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + ": " + hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Makes ctx->device current for the duration of a call, restoring the caller's.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

uint32_t block_weights(uint32_t enc) {
    switch (enc) {
    case DYNINFER_ENC_GGUF_Q4_0:
    case DYNINFER_ENC_GGUF_Q4_1:
    case DYNINFER_ENC_GGUF_Q8_0: return 32;
    case DYNINFER_ENC_GGUF_Q6_K:
    case DYNINFER_ENC_GGUF_Q4_K:
    case DYNINFER_ENC_GGUF_Q5_K:
    case DYNINFER_ENC_GGUF_IQ4_XS: return 256;
    default: return 0;
    }
}

uint64_t block_bytes(uint32_t enc) {
    switch (enc) {
    case DYNINFER_ENC_GGUF_Q4_0: return 18;
    case DYNINFER_ENC_GGUF_Q4_1: return 20;
    case DYNINFER_ENC_GGUF_Q8_0: return 34;
    case DYNINFER_ENC_GGUF_Q6_K: return 210;
    case DYNINFER_ENC_GGUF_Q4_K: return 144;
    case DYNINFER_ENC_GGUF_Q5_K: return 176;
    case DYNINFER_ENC_GGUF_IQ4_XS: return 136;
    default: return 0;
    }
}

const char* enc_name(uint32_t enc) {
    switch (enc) {
    case DYNINFER_ENC_GGUF_Q4_0: return "gguf.q4_0";
    case DYNINFER_ENC_GGUF_Q4_1: return "gguf.q4_1";
    case DYNINFER_ENC_GGUF_Q8_0: return "gguf.q8_0";
    case DYNINFER_ENC_GGUF_Q6_K: return "gguf.q6_k";
    case DYNINFER_ENC_GGUF_Q4_K: return "gguf.q4_k";
    case DYNINFER_ENC_GGUF_Q5_K: return "gguf.q5_k";
    case DYNINFER_ENC_GGUF_IQ4_XS: return "gguf.iq4_xs";
    case DYNINFER_ENC_MLX_AFFINE_U4: return "mlx.affine.u4";
    default: return "unknown";
    }
}

// Validates a weight descriptor.  Returns 0 or an error code (message set).
int check_weight(const dyninfer_qweight_t* w) {
    if (!w) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "weight descriptor is NULL");
    if (w->rows == 0 || w->cols == 0)
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "weight has an empty dimension");
    if (w->rows > 0xFFFFFFFFull || w->cols > 0x7FFFFFFFull)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "weight dimensions exceed the 32-bit kernel indexing");
    if (!w->data) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "weight data pointer is NULL");
    const uint32_t bw = block_weights(w->encoding);
    if (bw) {
        if (w->cols % bw)
            return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                        std::string(enc_name(w->encoding)) + ": logical axis 1 (" + std::to_string(w->cols) +
                            ") is not a multiple of the block size " + std::to_string(bw));
        // 2-byte aligned blocks for Q4_0, Q8_0 and Q6_K (18, 34 and 210 bytes), 4-byte for the rest
        const uintptr_t need = w->encoding == DYNINFER_ENC_GGUF_Q4_0 || w->encoding == DYNINFER_ENC_GGUF_Q8_0 ||
                                       w->encoding == DYNINFER_ENC_GGUF_Q6_K
                                   ? 2
                                   : 4;
        if (!aligned(w->data, need))
            return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string(enc_name(w->encoding)) +
                                                                  ": block data must be " + std::to_string(need) +
                                                                  "-byte aligned");
        const uint64_t expect = w->rows * (w->cols / bw) * block_bytes(w->encoding);
        if (w->data_bytes != expect)
            return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                        std::string(enc_name(w->encoding)) + " requires one interleaved data component of " +
                            std::to_string(expect) + " bytes, got " + std::to_string(w->data_bytes) + " bytes");
        if (expect > 0xFFFFFFF0ull)
            return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, std::string(enc_name(w->encoding)) +
                                                             ": one weight tensor is limited to 4 GiB (32-bit offsets)");
        if (!dmx::gemv_k_supported(w->encoding, (uint32_t)w->cols))
            return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                        std::string(enc_name(w->encoding)) + ": logical axis 1 (" + std::to_string(w->cols) +
                            ") is too long for one workgroup's activation tile in LDS");
        return 0;
    }
    if (w->encoding != DYNINFER_ENC_MLX_AFFINE_U4)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "unsupported encoding " + std::to_string(w->encoding));
    if (w->group_size == 0 || w->group_size % 32 || w->cols % w->group_size)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                    "mlx.affine.u4: group size must be a positive multiple of 32 dividing the logical axis");
    if (!w->scales || !w->biases)
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "mlx.affine.u4: scales and biases are required");
    uintptr_t es;
    switch (w->scale_dtype) {
    case DYNINFER_DTYPE_F32: es = 4; break;
    case DYNINFER_DTYPE_F16:
    case DYNINFER_DTYPE_BF16: es = 2; break;
    default: return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "mlx.affine.u4: scale dtype must be f32, f16 or bf16");
    }
    if (!aligned(w->data, 4) || !aligned(w->scales, es) || !aligned(w->biases, es))
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "mlx.affine.u4: component pointers are misaligned");
    const uint64_t packed = w->rows * w->cols / 2, grouped = w->rows * (w->cols / w->group_size) * es;
    if (w->data_bytes != packed || w->scales_bytes != grouped || w->biases_bytes != grouped)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                    "mlx.affine.u4: MLX component byte length is invalid (packed " + std::to_string(packed) +
                        ", scales/biases " + std::to_string(grouped) + " bytes expected; got " +
                        std::to_string(w->data_bytes) + ", " + std::to_string(w->scales_bytes) + ", " +
                        std::to_string(w->biases_bytes) + ")");
    if (packed > 0xFFFFFFF0ull || grouped > 0xFFFFFFF0ull)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "mlx.affine.u4: one weight tensor is limited to 4 GiB (32-bit offsets)");
    if (!dmx::gemv_k_supported(w->encoding, (uint32_t)w->cols))
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "mlx.affine.u4: logical axis 1 (" + std::to_string(w->cols) +
                                                        ") is too long for one workgroup's activation tile in LDS");
    return 0;
}

// Activation/output dtype rules: f32 (the reference's all-f32 contract for
// quantized linears, crates/dyninfer-compiler/src/lib.rs:289-306) or bf16
// activations for every encoding, f32 or bf16 outputs.
int check_io(uint32_t x_dtype, uint32_t y_dtype, uint32_t rows) {
    if (rows == 0) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "rows must be >= 1");
    if (x_dtype != DYNINFER_DTYPE_F32 && x_dtype != DYNINFER_DTYPE_BF16)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "activations must be f32 or bf16");
    if (y_dtype != DYNINFER_DTYPE_F32 && y_dtype != DYNINFER_DTYPE_BF16)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "outputs must be f32 or bf16");
    return 0;
}

int check_ctx(dyninfer_mi355x_ctx_t* ctx) {
    if (!ctx) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "context is NULL");
    return 0;
}

dmx::GemvProblem problem_of(const dyninfer_qweight_t* w, void* y) {
    dmx::GemvProblem p;
    p.w = static_cast<const uint8_t*>(w->data);
    p.sc = static_cast<const uint8_t*>(w->scales);
    p.bi = static_cast<const uint8_t*>(w->biases);
    p.y = y;
    p.n = (uint32_t)w->rows;
    return p;
}

size_t esize(uint32_t dt) { return dt == DYNINFER_DTYPE_F32 ? 4 : 2; }

// Whether `rows` activation rows run the prefill GEMM (else the GEMV kernels
// over 16-row chunks).  Q4_1, Q8_0 and MLX U4 take the GEMM from 17 rows (MLX
// 4096x1024: 13.4 against 17.0 us at 17 rows, 19.8 against 380 us at 512).
// The 16-row GEMV of Q4_0, Q6_K and Q4_K runs on MFMA, and two of its chunks
// (17..32 rows) mostly take less time than staging plus a GEMM with so few
// workgroups (Q4_0 4096x4096 at 24 rows: 21.5 against 23.8 us; Q6_K 1024x4096
// 23.2 against 35.6 us), three never do (40 rows: Q4_0 4096x4096 32.2 against
// 24.6 us, 12288x4096 52.4 against 28.2 us); with K above 8192 the MFMA GEMV
// splits K over launches and the GEMM wins from 17 rows (Q4_0 4096x12288:
// 60.9 against 73.2 us, Q4_K 66.9 against 81.8 us).  Except Q6_K with f32
// outputs: at K above 8192 its GEMM has few row tiles, each decoding long
// Q6_K slices, and the 16-row MFMA GEMV chunks win up to 32 rows (4096x12288:
// 46 against 102 us at 17 rows, 71 against 103 at 32; 107 against 106 at 48).
// With bf16 outputs the MFMA GEMV does not split K, so the GEMM stays.
bool has_prefill_gemm(uint32_t enc, uint32_t N, uint32_t K, uint32_t rows, bool y_bf16) {
    const bool mfma_gemv = enc == DYNINFER_ENC_GGUF_Q4_0 || enc == DYNINFER_ENC_GGUF_Q6_K ||
                           enc == DYNINFER_ENC_GGUF_Q4_K || enc == DYNINFER_ENC_GGUF_Q5_K ||
                           enc == DYNINFER_ENC_GGUF_IQ4_XS;
    const bool two_chunks = mfma_gemv && (K <= 8192u || (enc == DYNINFER_ENC_GGUF_Q6_K && !y_bf16));
    const uint32_t min_rows = two_chunks ? 2u * (uint32_t)dmx::kMaxGemvBatch + 1u : (uint32_t)dmx::kMaxGemvBatch + 1u;
    return rows >= min_rows && dmx::gemm_supported(enc, N, K, rows);
}

// The prefill path: x staged once (xprep), then one GEMM per weight.
hipError_t prefill(const dyninfer_qweight_t* ws, uint32_t count, const void* x, uint32_t x_dtype, uint32_t rows,
                   void* const* ys, uint32_t y_dtype, uint8_t* work, hipStream_t st) {
    const uint32_t K = (uint32_t)ws[0].cols;
    uint16_t* xh = reinterpret_cast<uint16_t*>(work);
    float* rs = reinterpret_cast<float*>(work + dmx::prefill_xh_bytes(rows, K));
    const uint32_t enc = ws[0].encoding;
    hipError_t e = dmx::xprep_launch(x, x_dtype == DYNINFER_DTYPE_BF16, rows, K, dmx::gemm_layout(enc), xh, rs, st);
    for (uint32_t i = 0; i < count && e == hipSuccess; i++) {
        const dmx::GemmWeight wt{enc, static_cast<const uint8_t*>(ws[i].data), static_cast<const uint8_t*>(ws[i].scales),
                                 static_cast<const uint8_t*>(ws[i].biases), ws[i].group_size, ws[i].scale_dtype};
        e = dmx::gemm_launch(wt, (uint32_t)ws[i].rows, K, xh, rs, rows, ys[i], y_dtype == DYNINFER_DTYPE_BF16, st);
    }
    return e;
}

// Runs rows > 16 through the GEMV kernels 16 activation rows at a time (the
// chunks one after another on the stream, each free to use the workspace).
hipError_t gemv_rows(const dyninfer_qweight_t* ws, uint32_t count, const void* x, uint32_t x_dtype, uint32_t rows,
                     void* const* ys, uint32_t y_dtype, uint8_t* work, uint64_t work_bytes, hipStream_t st) {
    const uint32_t K = (uint32_t)ws[0].cols;
    for (uint32_t r0 = 0; r0 < rows; r0 += dmx::kMaxGemvBatch) {
        const uint32_t nb = rows - r0 < (uint32_t)dmx::kMaxGemvBatch ? rows - r0 : (uint32_t)dmx::kMaxGemvBatch;
        dmx::GemvProblem probs[dmx::kMaxProblems];
        for (uint32_t i = 0; i < count; i++)
            probs[i] = problem_of(&ws[i], static_cast<uint8_t*>(ys[i]) + (size_t)r0 * ws[i].rows * esize(y_dtype));
        const void* xr = static_cast<const uint8_t*>(x) + (size_t)r0 * K * esize(x_dtype);
        hipError_t e = dmx::gemv_launch(ws[0].encoding, probs, (int)count, K, xr, x_dtype == DYNINFER_DTYPE_BF16, nb,
                                        y_dtype == DYNINFER_DTYPE_BF16, ws[0].group_size, ws[0].scale_dtype, work,
                                        work_bytes, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// The optional workspace of the GEMV chunks of a call (the largest any chunk
// of 16 rows, or the last, smaller one, would use).
uint64_t gemv_rows_workspace(const dyninfer_qweight_t* ws, uint32_t count, uint32_t rows, uint32_t y_dtype) {
    dmx::GemvProblem probs[dmx::kMaxProblems];
    for (uint32_t i = 0; i < count; i++) probs[i] = problem_of(&ws[i], nullptr);
    auto need = [&](uint32_t nb) {
        return dmx::gemv_workspace_bytes(ws[0].encoding, probs, (int)count, nb, (uint32_t)ws[0].cols,
                                         y_dtype == DYNINFER_DTYPE_BF16, ws[0].group_size);
    };
    const uint64_t last = need(rows % (uint32_t)dmx::kMaxGemvBatch ? rows % (uint32_t)dmx::kMaxGemvBatch
                                                                    : (uint32_t)dmx::kMaxGemvBatch);
    const uint64_t full = rows > (uint32_t)dmx::kMaxGemvBatch ? need((uint32_t)dmx::kMaxGemvBatch) : 0;
    return last > full ? last : full;
}

}  // namespace

extern "C" {

const char* dyninfer_mi355x_last_error(void) { return g_last_error.c_str(); }

const char* dyninfer_mi355x_version(void) { return "dyninfer-mi355x 0.1.0 (gfx950); kernel-registry 6"; }

int dyninfer_mi355x_open(int device, dyninfer_mi355x_ctx_t** out_ctx) {
    if (!out_ctx) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "out_ctx is NULL");
    *out_ctx = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT,
                    "device " + std::to_string(device) + " out of range (" + std::to_string(count) + " devices)");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(DYNINFER_MI355X_ERR_DEVICE,
                    std::string("device is ") + prop.gcnArchName + "; this library's kernels are built for gfx950 only");
    // the device's copy of the no-allocation scratch array, with that device current
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    void* sp = nullptr;
    e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress (no-allocation scratch)");
    auto* c = new dyninfer_mi355x_ctx();
    c->device = device;
    c->scratch = static_cast<uint8_t*>(sp);
    *out_ctx = c;
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_close(dyninfer_mi355x_ctx_t* ctx) {
    delete ctx;  // the context holds no device memory (the scratch array belongs to the code object)
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_supports(const dyninfer_qweight_t* w, uint32_t rows, uint32_t x_dtype, uint32_t y_dtype) {
    if (check_weight(w) || check_io(x_dtype, y_dtype, rows)) return 0;
    return 1;
}

// Validation and routing of a qlinear_multi call, shared by the call and the
// workspace query: whether it runs the prefill GEMM, and its workspace, which
// the prefill GEMM needs and the GEMV kernels may use (the MFMA GEMV stages
// the activations once per call in it instead of once per workgroup).
static int plan_multi(const dyninfer_qweight_t* ws, uint32_t count, uint32_t x_dtype, uint32_t rows,
                      uint32_t y_dtype, bool& gemm, uint64_t& need) {
    if (!ws || count == 0 || count > (uint32_t)dmx::kMaxProblems)
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "count must be 1..4 with a weight array");
    for (uint32_t i = 0; i < count; i++) {
        if (int rc = check_weight(&ws[i])) return rc;
        if (ws[i].encoding != ws[0].encoding || ws[i].cols != ws[0].cols ||
            (ws[0].encoding == DYNINFER_ENC_MLX_AFFINE_U4 &&
             (ws[i].group_size != ws[0].group_size || ws[i].scale_dtype != ws[0].scale_dtype)))
            return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT,
                        "grouped weights must share encoding, K, group size and scale dtype");
    }
    if (int rc = check_io(x_dtype, y_dtype, rows)) return rc;
    gemm = true;
    for (uint32_t i = 0; i < count && gemm; i++)
        gemm = has_prefill_gemm(ws[i].encoding, (uint32_t)ws[i].rows, (uint32_t)ws[i].cols, rows,
                                y_dtype == DYNINFER_DTYPE_BF16);
    if (gemm && (uint64_t)rows * ws[0].cols >= (1ull << 31))
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "prefill: rows * K must stay below 2^31 (32-bit activation offsets)");
    need = gemm ? dmx::prefill_workspace_bytes(rows, (uint32_t)ws[0].cols) : gemv_rows_workspace(ws, count, rows, y_dtype);
    return 0;
}

// qlinear_multi with the caller's workspace, or (noalloc) with the device's
// static scratch array.
static int qlinear_multi_impl(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* ws, uint32_t count, const void* x,
                              uint32_t x_dtype, uint32_t rows, void* const* ys, uint32_t y_dtype, void* workspace,
                              uint64_t workspace_bytes, void* stream, bool noalloc) {
    if (int rc = check_ctx(ctx)) return rc;
    bool gemm = false;
    uint64_t need = 0;
    if (int rc = plan_multi(ws, count, x_dtype, rows, y_dtype, gemm, need)) return rc;
    if (!x || !ys) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "x / y pointers are NULL");
    for (uint32_t i = 0; i < count; i++) {
        if (!ys[i]) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "output pointer is NULL");
        if (!aligned(ys[i], esize(y_dtype))) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "output is misaligned");
    }
    if (!aligned(x, 16)) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "activations must be 16-byte aligned");
    uint8_t* work = nullptr;
    uint64_t work_bytes = 0;
    if (noalloc) {
        if (gemm && need > kScratchBytes)
            return fail(DYNINFER_MI355X_ERR_UNSUPPORTED,
                        "qlinear_multi_noalloc: the prefill staging of " + std::to_string(rows) + " rows x K " +
                            std::to_string(ws[0].cols) + " needs " + std::to_string(need) +
                            " bytes, more than the static scratch of " + std::to_string(kScratchBytes) +
                            " bytes; split the rows or call dyninfer_mi355x_qlinear_multi");
        work = ctx->scratch;
        work_bytes = kScratchBytes;
    } else if (need && (gemm || workspace)) {  // required for prefill; optional (NULL accepted) for the GEMV
        const char* what = gemm ? "prefill" : "decode";
        if (!workspace || workspace_bytes < need)
            return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT,
                        std::string(what) + " of " + std::to_string(rows) + " rows x K " + std::to_string(ws[0].cols) +
                            (gemm ? " needs a device workspace of " : " takes a device workspace (or NULL) of ") +
                            std::to_string(need) + " bytes (got " +
                            (workspace ? std::to_string(workspace_bytes) + " bytes" : std::string("NULL")) +
                            "); size it with dyninfer_mi355x_prefill_workspace_bytes");
        if (!aligned(workspace, 256))
            return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("the ") + what +
                                                                  " workspace must be 256-byte aligned");
        work = static_cast<uint8_t*>(workspace);
        work_bytes = workspace_bytes;
    }
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = gemm ? prefill(ws, count, x, x_dtype, rows, ys, y_dtype, work, st)
                              : gemv_rows(ws, count, x, x_dtype, rows, ys, y_dtype, work, work_bytes, st);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_prefill_workspace_bytes(const dyninfer_qweight_t* ws, uint32_t count, uint32_t rows,
                                            uint32_t x_dtype, uint32_t y_dtype, uint64_t* out_bytes) {
    if (!out_bytes) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "out_bytes is NULL");
    *out_bytes = 0;
    bool gemm = false;
    uint64_t need = 0;
    if (int rc = plan_multi(ws, count, x_dtype, rows, y_dtype, gemm, need)) return rc;
    *out_bytes = need;
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_qlinear_multi(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* ws, uint32_t count,
                                  const void* x, uint32_t x_dtype, uint32_t rows, void* const* ys, uint32_t y_dtype,
                                  void* workspace, uint64_t workspace_bytes, void* stream) {
    return qlinear_multi_impl(ctx, ws, count, x, x_dtype, rows, ys, y_dtype, workspace, workspace_bytes, stream,
                              false);
}

int dyninfer_mi355x_qlinear_multi_noalloc(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* ws, uint32_t count,
                                          const void* x, uint32_t x_dtype, uint32_t rows, void* const* ys,
                                          uint32_t y_dtype, void* stream) {
    return qlinear_multi_impl(ctx, ws, count, x, x_dtype, rows, ys, y_dtype, nullptr, 0, stream, true);
}

int dyninfer_mi355x_qlinear(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w, const void* x, uint32_t x_dtype,
                            uint32_t rows, void* y, uint32_t y_dtype, void* workspace, uint64_t workspace_bytes,
                            void* stream) {
    void* ys[1] = {y};
    return dyninfer_mi355x_qlinear_multi(ctx, w, 1, x, x_dtype, rows, ys, y_dtype, workspace, workspace_bytes,
                                         stream);
}

int dyninfer_mi355x_dequant(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w, float* out, void* stream) {
    if (int rc = check_ctx(ctx)) return rc;
    if (int rc = check_weight(w)) return rc;
    if (!out || !aligned(out, 4)) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "output is NULL or misaligned");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipError_t e = dmx::dequant_launch(w->encoding, static_cast<const uint8_t*>(w->data),
                                       static_cast<const uint8_t*>(w->scales), static_cast<const uint8_t*>(w->biases),
                                       (uint32_t)w->rows, (uint32_t)w->cols, w->group_size, w->scale_dtype, out,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_embedding(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w, const int64_t* ids,
                              uint32_t n_ids, float* out, void* stream) {
    if (int rc = check_ctx(ctx)) return rc;
    if (int rc = check_weight(w)) return rc;
    if (n_ids == 0) return DYNINFER_MI355X_OK;  // an empty batch gathers nothing
    if (!ids || !aligned(ids, 8)) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "ids is NULL or not 8-byte aligned");
    if (!out || !aligned(out, 16))
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "output is NULL or not 16-byte aligned");
    const uint64_t per_row = (w->cols / 4 + 255) / 256;
    if ((uint64_t)n_ids * per_row > 0x7FFFFFFFull)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "n_ids * ceil(K / 1024) must stay below 2^31");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipError_t e = dmx::gather_launch(w->encoding, static_cast<const uint8_t*>(w->data),
                                      static_cast<const uint8_t*>(w->scales), static_cast<const uint8_t*>(w->biases),
                                      (uint32_t)w->rows, (uint32_t)w->cols, w->group_size, w->scale_dtype, ids, n_ids,
                                      out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "embedding launch");
    return DYNINFER_MI355X_OK;
}

struct dyninfer_gguf {
    dmx::GgufIndex idx;
};

static int gguf_finish(const uint8_t* base, uint64_t len, void* map, dyninfer_gguf_t** out) {
    auto* g = new dyninfer_gguf();
    g->idx.map = map;
    g->idx.len = len;  // the mapping's length, so a failed index still unmaps it
    const std::string err = dmx::gguf_index(base, len, g->idx);
    if (!err.empty()) {
        dyninfer_mi355x_gguf_close(g);
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "invalid GGUF: " + err);
    }
    *out = g;
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_gguf_open(const char* path, dyninfer_gguf_t** out) {
    if (!path || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "path / out is NULL");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, std::string("invalid GGUF: empty or unreadable file ") + path);
    }
    void* m = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("mmap failed: ") + std::strerror(errno));
    return gguf_finish(static_cast<const uint8_t*>(m), (uint64_t)st.st_size, m, out);
}

int dyninfer_mi355x_gguf_open_memory(const void* data, uint64_t len, dyninfer_gguf_t** out) {
    if (!data || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "data / out is NULL");
    *out = nullptr;
    return gguf_finish(static_cast<const uint8_t*>(data), len, nullptr, out);
}

int dyninfer_mi355x_gguf_close(dyninfer_gguf_t* g) {
    if (!g) return DYNINFER_MI355X_OK;
    if (g->idx.map) ::munmap(g->idx.map, (size_t)g->idx.len);
    delete g;
    return DYNINFER_MI355X_OK;
}

uint64_t dyninfer_mi355x_gguf_tensor_count(const dyninfer_gguf_t* g) { return g ? g->idx.tensors.size() : 0; }

const char* dyninfer_mi355x_gguf_metadata_json(const dyninfer_gguf_t* g) { return g ? g->idx.metadata_json.c_str() : "{}"; }

static void gguf_fill(const dmx::GgufTensor& t, dyninfer_gguf_tensor_t* out) {
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->type_code = t.type_code;
    out->n_dims = (uint32_t)t.shape.size();
    for (size_t i = 0; i < t.shape.size(); i++) out->dims[i] = t.shape[i];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
}

static const dmx::GgufTensor* gguf_lookup(const dyninfer_gguf_t* g, const char* name) {
    auto it = std::lower_bound(g->idx.tensors.begin(), g->idx.tensors.end(), name,
                               [](const dmx::GgufTensor& t, const char* n) { return t.name < n; });
    return it != g->idx.tensors.end() && it->name == name ? &*it : nullptr;
}

int dyninfer_mi355x_gguf_tensor(const dyninfer_gguf_t* g, uint64_t index, dyninfer_gguf_tensor_t* out) {
    if (!g || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / out is NULL");
    if (index >= g->idx.tensors.size()) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "tensor index out of range");
    gguf_fill(g->idx.tensors[index], out);
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_gguf_find(const dyninfer_gguf_t* g, const char* name, dyninfer_gguf_tensor_t* out) {
    if (!g || !name || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / out is NULL");
    const dmx::GgufTensor* t = gguf_lookup(g, name);
    if (!t) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    gguf_fill(*t, out);
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_gguf_upload(const dyninfer_gguf_t* g, const char* name, void* dst, uint64_t dst_bytes, void* stream) {
    if (!g || !name || !dst) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / dst is NULL");
    const dmx::GgufTensor* t = gguf_lookup(g, name);
    if (!t) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    if (dst_bytes < t->nbytes)
        return fail(DYNINFER_MI355X_ERR_BUFFER_TOO_SMALL, "destination needs " + std::to_string(t->nbytes) + " bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst, g->idx.base + t->offset, (size_t)t->nbytes, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
    e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_gguf_qweight(const dyninfer_gguf_t* g, const char* name, const void* device_data,
                                 dyninfer_qweight_t* out) {
    if (!g || !name || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / out is NULL");
    const dmx::GgufTensor* t = gguf_lookup(g, name);
    if (!t) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    if (t->shape.size() != 2) return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "tensor " + t->name + " is not rank 2");
    if (t->type_code != dmx::ENC_Q4_0 && t->type_code != dmx::ENC_Q4_1 && t->type_code != dmx::ENC_Q8_0 &&
        t->type_code != dmx::ENC_Q6_K && t->type_code != dmx::ENC_Q4_K && t->type_code != dmx::ENC_Q5_K &&
        t->type_code != dmx::ENC_IQ4_XS)
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "tensor " + t->name + " has GGUF type " +
                                                         std::to_string(t->type_code) +
                                                         ", not Q4_0/Q4_1/Q8_0/Q6_K/Q4_K/Q5_K/IQ4_XS");
    std::memset(out, 0, sizeof *out);
    out->encoding = t->type_code;
    out->rows = t->shape[0];
    out->cols = t->shape[1];
    out->data = device_data;
    out->data_bytes = t->nbytes;
    return check_weight(out);
}

struct dyninfer_safetensors {
    dmx::StIndex idx;
};

static int st_finish(const uint8_t* base, uint64_t len, void* map, const char* config, dyninfer_safetensors_t** out) {
    auto* t = new dyninfer_safetensors();
    t->idx.map = map;
    t->idx.len = len;  // the mapping's length, so a failed index still unmaps it
    const std::string err = dmx::st_index(base, len, t->idx);
    if (!err.empty()) {
        dyninfer_mi355x_safetensors_close(t);
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "invalid SafeTensors: " + err);
    }
    if (config) dmx::st_merge_config(t->idx, config);
    *out = t;
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_safetensors_open(const char* path, dyninfer_safetensors_t** out) {
    if (!path || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "path / out is NULL");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, std::string("invalid SafeTensors: empty or unreadable file ") + path);
    }
    void* m = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("mmap failed: ") + std::strerror(errno));
    // the sibling config.json (config_json.rs:10-20); an unreadable one is ignored
    std::string cfg_path(path), cfg;
    const size_t slash = cfg_path.rfind('/');
    cfg_path = (slash == std::string::npos ? std::string() : cfg_path.substr(0, slash + 1)) + "config.json";
    bool have_cfg = false;
    if (FILE* f = std::fopen(cfg_path.c_str(), "rb")) {
        char buf[4096];
        size_t got;
        while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) cfg.append(buf, got);
        have_cfg = !std::ferror(f);
        std::fclose(f);
    }
    return st_finish(static_cast<const uint8_t*>(m), (uint64_t)st.st_size, m, have_cfg ? cfg.c_str() : nullptr, out);
}

int dyninfer_mi355x_safetensors_open_memory(const void* data, uint64_t len, const char* config_json,
                                            dyninfer_safetensors_t** out) {
    if (!data || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "data / out is NULL");
    *out = nullptr;
    return st_finish(static_cast<const uint8_t*>(data), len, nullptr, config_json, out);
}

int dyninfer_mi355x_safetensors_close(dyninfer_safetensors_t* t) {
    if (!t) return DYNINFER_MI355X_OK;
    if (t->idx.map) ::munmap(t->idx.map, (size_t)t->idx.len);
    delete t;
    return DYNINFER_MI355X_OK;
}

uint64_t dyninfer_mi355x_safetensors_tensor_count(const dyninfer_safetensors_t* t) { return t ? t->idx.tensors.size() : 0; }

const char* dyninfer_mi355x_safetensors_metadata_json(const dyninfer_safetensors_t* t) {
    return t ? t->idx.metadata_json.c_str() : "{}";
}

static void st_fill(const dmx::StTensor& t, dyninfer_st_tensor_t* out) {
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->dtype = t.dtype.c_str();
    out->n_dims = (uint32_t)t.shape.size();
    for (size_t i = 0; i < t.shape.size(); i++) out->dims[i] = t.shape[i];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
}

int dyninfer_mi355x_safetensors_tensor(const dyninfer_safetensors_t* t, uint64_t index, dyninfer_st_tensor_t* out) {
    if (!t || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / out is NULL");
    if (index >= t->idx.tensors.size()) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "tensor index out of range");
    st_fill(t->idx.tensors[index], out);
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_safetensors_find(const dyninfer_safetensors_t* t, const char* name, dyninfer_st_tensor_t* out) {
    if (!t || !name || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / out is NULL");
    const dmx::StTensor* e = dmx::st_find(t->idx, name);
    if (!e) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    st_fill(*e, out);
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_safetensors_upload(const dyninfer_safetensors_t* t, const char* name, void* dst, uint64_t dst_bytes,
                                       void* stream) {
    if (!t || !name || !dst) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / dst is NULL");
    const dmx::StTensor* e = dmx::st_find(t->idx, name);
    if (!e) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    if (dst_bytes < e->nbytes)
        return fail(DYNINFER_MI355X_ERR_BUFFER_TOO_SMALL, "destination needs " + std::to_string(e->nbytes) + " bytes");
    if (e->nbytes == 0) return DYNINFER_MI355X_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t err = hipMemcpyAsync(dst, t->idx.base + e->offset, (size_t)e->nbytes, hipMemcpyHostToDevice, st);
    if (err != hipSuccess) return hip_fail(err, "hipMemcpyAsync");
    err = hipStreamSynchronize(st);
    if (err != hipSuccess) return hip_fail(err, "hipStreamSynchronize");
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_safetensors_mlx_qweight(const dyninfer_safetensors_t* t, const char* weight_name,
                                            const void* device_packed, const void* device_scales,
                                            const void* device_biases, dyninfer_qweight_t* out) {
    if (!t || !weight_name || !out) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "index / name / out is NULL");
    const dmx::StTensor *p = nullptr, *s = nullptr, *b = nullptr;
    uint64_t n = 0, k = 0, g = 0;
    const std::string err = dmx::st_mlx_weight(t->idx, weight_name, &p, &s, &b, &n, &k, &g);
    if (!err.empty()) return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, err);
    if (g > UINT32_MAX) return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, "group size out of range");
    std::memset(out, 0, sizeof *out);
    out->encoding = DYNINFER_ENC_MLX_AFFINE_U4;
    out->group_size = (uint32_t)g;
    out->rows = n;
    out->cols = k;
    out->data = device_packed;
    out->scales = device_scales;
    out->biases = device_biases;
    out->scale_dtype = s->dtype == "F32" ? DYNINFER_DTYPE_F32 : s->dtype == "F16" ? DYNINFER_DTYPE_F16 : DYNINFER_DTYPE_BF16;
    out->data_bytes = p->nbytes;
    out->scales_bytes = s->nbytes;
    out->biases_bytes = b->nbytes;
    return check_weight(out);
}

const char* dyninfer_mi355x_candidates_json(void) { return dmx::candidates_json().c_str(); }

static int registry_call(const char* c, const char* r, const char* t, char* out, size_t cap, size_t* len, bool req) {
    if (!r || !t) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "request / target JSON is NULL");
    std::string res, err;
    const int rc = dmx::registry_select(c, r, t, req, res, err);
    if (rc == 1) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, err);
    if (rc == 2) return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, err);
    if (len) *len = res.size();
    if (!out || cap < res.size() + 1)
        return fail(DYNINFER_MI355X_ERR_BUFFER_TOO_SMALL, "output buffer needs " + std::to_string(res.size() + 1) + " bytes");
    std::memcpy(out, res.c_str(), res.size() + 1);
    return DYNINFER_MI355X_OK;
}

int dyninfer_mi355x_registry_select(const char* candidates_json, const char* request_json, const char* target_json,
                                    char* out, size_t out_cap, size_t* out_len) {
    return registry_call(candidates_json, request_json, target_json, out, out_cap, out_len, false);
}

int dyninfer_mi355x_registry_require(const char* candidates_json, const char* request_json, const char* target_json,
                                     char* out, size_t out_cap, size_t* out_len) {
    return registry_call(candidates_json, request_json, target_json, out, out_cap, out_len, true);
}

int dyninfer_mi355x_precision_check(const char* selected_json, const char* activation_type) {
    if (!selected_json) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "selected kernel JSON is NULL");
    if (activation_type && std::strcmp(activation_type, "f32") != 0 && std::strcmp(activation_type, "bf16") != 0)
        return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, "activation_type must be \"f32\" or \"bf16\"");
    std::string err;
    const int rc = dmx::precision_check(selected_json, activation_type, err);
    if (rc == 1) return fail(DYNINFER_MI355X_ERR_INVALID_ARGUMENT, err);
    if (rc == 2) return fail(DYNINFER_MI355X_ERR_UNSUPPORTED, err);
    return DYNINFER_MI355X_OK;
}

}  // extern "C"
