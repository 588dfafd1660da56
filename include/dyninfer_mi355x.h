/*
 * dyninfer_mi355x.h — C ABI of the MI355X (gfx950) quantized weight-matmul library.
 *
 * Drop-in boundary for dyninfer's `rocm` target.  Today the reference lowers a
 * quantized linear to IREE-generated code: the selected kernel's lowering id is
 * dispatched by ParameterLowerings::emit_linear_call
 * (crates/dyninfer-compiler/src/lowering/parameter.rs:141-183) to the encoding's
 * MLIR emitter (crates/dyninfer-quantization/src/quantizations/gguf_codegen.rs:268-314,
 * mlx_affine.rs:557-626) and run through the IREE runtime C wrapper
 * (third_party/iree_runtime_c_api/wrapper.h:74-105).  This library replaces that
 * generated code for lowering ids ending in `.mi355x_hip`: the runtime calls the
 * entry points below with device pointers to the weight's exact on-disk bytes.
 *
 * Conventions (mirroring third_party/iree_runtime_c_api/wrapper.h:38-63):
 *   - every entry point returns an int status, 0 = success;
 *   - on failure dyninfer_mi355x_last_error() returns a message for the calling
 *     thread (thread-local, unlike the wrapper's process-global g_last_error,
 *     wrapper.c:238);
 *   - opaque context handle with open/close pair (wrapper.h:39-60);
 *   - weights, activations, outputs and the prefill workspace are caller-owned
 *     device memory; the library never repacks or copies weights and derives no
 *     parameters from them (README.md:5-9, crates/dyninfer-compiler/src/lib.rs:630),
 *     and it allocates no device memory: a call's temporary (the prefill staging of
 *     dyninfer_mi355x_qlinear, and the optional activation staging of its 3..16-row
 *     MFMA GEMV) lives in a workspace the caller sizes with
 *     dyninfer_mi355x_prefill_workspace_bytes and passes in, the counterpart of the
 *     reference's device-local, non-persistent GPU temporaries
 *     (docs/quantization/mlx-affine-u4.md:26-27) bound like its parameters as
 *     caller-described ranges (third_party/iree_runtime_c_api/wrapper.h:18-29);
 *   - the context is immutable after dyninfer_mi355x_open (no locks, no caches):
 *     any number of threads may call with one context at once; work is enqueued
 *     asynchronously on the caller's HIP stream (`stream` is a hipStream_t passed as
 *     void*; NULL = the null stream); calls in flight at the same time (distinct
 *     streams or threads) need distinct workspaces; there is no CPU fallback
 *     (README.md:83-84).
 */
#ifndef DYNINFER_MI355X_H
#define DYNINFER_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
    DYNINFER_MI355X_OK = 0,
    DYNINFER_MI355X_ERR_INVALID_ARGUMENT = 1, /* null pointer, zero size, bad dtype, misaligned base */
    DYNINFER_MI355X_ERR_UNSUPPORTED = 2,      /* encoding / shape outside the qualified envelope
                                                  (E_UNSUPPORTED_ENCODING, crates/dyninfer-error/src/lib.rs:54-72) */
    DYNINFER_MI355X_ERR_HIP = 3,              /* HIP runtime error; message carries hipGetErrorString */
    DYNINFER_MI355X_ERR_DEVICE = 4,           /* device is not gfx950 */
    DYNINFER_MI355X_ERR_BUFFER_TOO_SMALL = 5  /* output string buffer too small (registry calls) */
};

/* Encodings.  GGUF values are the GGML type codes
 * (crates/dyninfer-checkpoint-gguf/src/types.rs:10-43). */
enum {
    DYNINFER_ENC_GGUF_Q4_0 = 2,
    DYNINFER_ENC_GGUF_Q4_1 = 3,
    DYNINFER_ENC_GGUF_Q8_0 = 8,
    DYNINFER_ENC_GGUF_Q6_K = 14,
    DYNINFER_ENC_GGUF_Q4_K = 12, /* GGML's 144-byte super-block; a schema-only type in the reference
                                    (gguf_block.rs:183-316), decoded here as GGML dequantize_row_q4_K */
    DYNINFER_ENC_GGUF_Q5_K = 13, /* GGML's 176-byte super-block (schema only in the reference),
                                    decoded as GGML dequantize_row_q5_K */
    DYNINFER_ENC_GGUF_IQ4_XS = 23, /* GGML's 136-byte super-block with the kvalues_iq4nl codebook
                                      (schema only in the reference), as dequantize_row_iq4_xs */
    DYNINFER_ENC_MLX_AFFINE_U4 = 0x1004
};

/* Element types of activations, outputs and MLX scales/biases. */
enum { DYNINFER_DTYPE_F32 = 0, DYNINFER_DTYPE_F16 = 1, DYNINFER_DTYPE_BF16 = 2 };

/*
 * A quantized weight, logically [rows = out features N, cols = in features K],
 * row-major, "native" orientation (crates/dyninfer-kernel-registry/src/lib.rs:84-89).
 *
 * GGUF (PhysicalEncoding::BlockQuantized, crates/dyninfer-checkpoint-gguf/src/convention.rs:200-279):
 *   `data` = the tensor's interleaved blocks, N*(K/B)*bytes_per_block bytes; row o, block b
 *   starts at byte (o*K/B + b)*bytes_per_block (gguf_codegen.rs:350-367).  `data` must be
 *   2-byte aligned (4-byte for Q4_1, Q4_K, Q5_K and IQ4_XS).  scales/biases/group_size/scale_dtype are ignored.
 * MLX affine U4 (PhysicalEncoding::GroupQuantized, crates/dyninfer-checkpoint-safetensors/src/mlx.rs:152-261):
 *   `data` = packed u32 [N, K/8] (lane i = bits 4i..4i+3), `scales`, `biases` = [N, K/group_size]
 *   of `scale_dtype` (f32/f16/bf16), each aligned to its element size.
 *
 * The *_bytes fields give each component's byte length, the sum of its byte ranges in
 * the reference's parameter binding.  Every call validates them as the reference's
 * encodings do: GGUF `data_bytes` must equal N*(K/B)*bytes_per_block
 * ("one interleaved data component", gguf_block.rs:111-155, q4_0.rs:82-119); MLX
 * `data_bytes` must equal N*K/2 and `scales_bytes` = `biases_bytes` = N*(K/g)*sizeof(scale)
 * ("MLX component byte length", mlx_affine.rs:137-153).  A mismatch is
 * DYNINFER_MI355X_ERR_UNSUPPORTED (E_UNSUPPORTED_ENCODING); no kernel reads a short buffer.
 */
typedef struct dyninfer_qweight {
    uint32_t encoding;
    uint32_t group_size;  /* MLX only */
    uint64_t rows;        /* N */
    uint64_t cols;        /* K */
    const void* data;
    const void* scales;   /* MLX only */
    const void* biases;   /* MLX only */
    uint32_t scale_dtype; /* MLX only */
    uint32_t reserved;
    uint64_t data_bytes;
    uint64_t scales_bytes; /* MLX only (0 for GGUF) */
    uint64_t biases_bytes; /* MLX only (0 for GGUF) */
} dyninfer_qweight_t;

typedef struct dyninfer_mi355x_ctx dyninfer_mi355x_ctx_t;

/* Open a context on HIP device `device` (must be gfx950).  Mirrors
 * dyninfer_iree_session_create (wrapper.h:39-58) minus module loading: the
 * kernels are linked into this library. */
int dyninfer_mi355x_open(int device, dyninfer_mi355x_ctx_t** out_ctx);
int dyninfer_mi355x_close(dyninfer_mi355x_ctx_t* ctx);

/* Thread-local message for the last failing call on this thread ("" if none).
 * Mirrors dyninfer_iree_last_error (wrapper.h:62-63). */
const char* dyninfer_mi355x_last_error(void);

/*
 * y = x · Wᵀ with f32 accumulation: y[r, o] = Σ_k x[r, k] · w[o, k] where w is the
 * reference's dequantised value (gguf_codegen.rs:268-314 `emit_linear`;
 * mlx_affine.rs:557-626 `emit_linear_u4`; output projection = the same helper,
 * gguf_codegen.rs:157-159).  `rows` = activation rows (1..16 for decode; any for prefill).
 * x: [rows, K] row-major, 16-byte aligned, dtype x_dtype (f32 or bf16, every encoding);
 * y: [rows, N], dtype y_dtype (f32 or bf16).
 *   rows <= 16: the decode GEMV kernels (HBM-bound; 5..16 rows of large Q4_0, Q6_K, Q4_K,
 *     Q5_K, IQ4_XS and MLX weights on MFMA, and at 3..4 rows the largest of them), activations rounded to f16 after a
 *     power-of-two scaling per scale group;
 *   rows >= 17: the prefill path.  Q4_1, Q8_0 and MLX U4 from 17 rows, Q4_0, Q6_K and
 *     the K-quants / IQ4_XS from 33 rows, or from 17 when K > 8192 except Q6_K with f32
 *     outputs (below that two 16-row MFMA GEMV chunks are mostly faster), K a multiple
 *     of 64 (256 for the super-block
 *     encodings): x is staged once per call as f16 MFMA operand fragments,
 *     each row scaled by a power of two (RNE) and the rows padded with zeros to a
 *     multiple of 32, into the caller's workspace; then one MFMA GEMM per weight
 *     decodes the GGUF blocks or MLX words straight into MFMA operands.  Every other
 *     case (K not a multiple of 64, Q4_0, Q6_K, Q4_K, Q5_K and IQ4_XS at 17..32 rows
 *     with K <= 8192) runs the GEMV kernels over 16-row chunks.
 * workspace: device memory of at least dyninfer_mi355x_prefill_workspace_bytes() for
 *   the same arguments, 256-byte aligned, or NULL when that size is 0.  A call that
 *   runs the GEMV kernels (1..16 rows, and the 16-row chunks) may also pass NULL: the
 *   size is then that of an optional staging (the MFMA GEMV with K >= 2048, at 9..16
 *   rows or with K too long for one LDS segment: the activations are staged once per
 *   call by a small kernel and copied into each workgroup's LDS, instead of being
 *   staged by every workgroup; same results; with bf16 outputs and K too long for one
 *   LDS segment the workspace also holds f32 accumulators, and without it those
 *   calls run the VALU GEMV, ~3x slower at 9..16 rows).  A call
 *   whose workspace is given but misaligned or too small, or missing when the prefill
 *   GEMM needs it, fails with DYNINFER_MI355X_ERR_INVALID_ARGUMENT before anything is
 *   enqueued.  The call's kernels write and read it in stream order; the
 *   caller may reuse it for the next call on the same stream, and must not touch it
 *   (or hand it to a call on another stream) until this call's work has completed.
 *   Nothing the workspace holds carries over between calls.
 * Error bound (per output, plus f32 accumulation error), with |w||x| summed over k:
 *   GGUF Q4_0, Q4_1, Q8_0, IQ4_XS and MLX U4: 2^-10 * sum |w||x| (IQ4_XS prefill:
 *   3 * 2^-11 * sum |w||x|);
 *   Q6_K: (2^-10 + 2^-11) * sum |w||x|;
 *   Q4_K and Q5_K, whose prefill and MFMA-GEMV weights are RNE_f16(q*RNE_f16(d*sc) -
 *   RNE_f16(dmin*m)): (2^-10 + 2^-11) * sum |w||x| + 2^-10 * sum |dmin*m||x|, the
 *   offset term counting each weight's dmin*m, which may nearly cancel q*d*sc;
 *   MLX U4 with f32 scales and biases (each rounded to f16 before q*s + b) adds
 *   2^-11 * sum (q*|s| + |b|)|x|;
 *   and a prefill activation more than 2^29 below its row's largest magnitude may also
 *   be flushed to f16 subnormals (absolute 2^-40 * max|x| each).
 */
int dyninfer_mi355x_qlinear(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w,
                            const void* x, uint32_t x_dtype, uint32_t rows,
                            void* y, uint32_t y_dtype, void* workspace, uint64_t workspace_bytes,
                            void* stream);

/*
 * Several weights that share one activation (q/k/v, gate/up) in a single launch:
 * y_i = x · W_iᵀ for i < count.  All weights must have the same encoding (and group
 * size / scale dtype) and the same K; N may differ.  count <= 4, any rows (prefill
 * stages x once and runs one GEMM per weight).
 * No reference counterpart as one call: the reference emits one helper call per
 * linear (parameter.rs:141-183); this is the same arithmetic batched into one launch.
 */
int dyninfer_mi355x_qlinear_multi(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* ws,
                                  uint32_t count, const void* x, uint32_t x_dtype, uint32_t rows,
                                  void* const* ys, uint32_t y_dtype, void* workspace,
                                  uint64_t workspace_bytes, void* stream);

/*
 * Device workspace bytes of dyninfer_mi355x_qlinear (count = 1) or _qlinear_multi for
 * these weights, rows and dtypes, in *out_bytes.  A call that runs the prefill GEMM
 * needs round_up(round_up(rows, 32)*K*2, 256) + 4*round_up(rows, 256) (the f16
 * operand fragments of x, then one f32 row factor per row).  A GEMV call (16-row
 * chunks beyond 16 rows) that runs on the MFMA GEMV with K >= 2048, at 9..16 rows or
 * with K too long for one LDS segment (K > 4096 at most shapes), takes an optional
 * round_up((K/256) * T, 256), T = 8256 (T = 8512 for Q4_K and Q5_K): per 256 k, the
 * f16 MFMA fragments of 16 activation rows, their 16 f32 inverse scales (and the
 * f16 sums of the offset encodings); with bf16 outputs and K too long for one LDS
 * segment, plus round_up(rows*N*4, 256) per weight for the f32 accumulators its K
 * segments add into (without a workspace such a call runs the VALU GEMV); every
 * other call 0.  Validates the
 * arguments as the call does (same status codes, pointers checked for alignment only);
 * host-only, enqueues nothing.  The reference's temporary-memory qualification
 * (docs/quantization/mlx-affine-u4.md:52-54) reads this figure.
 */
int dyninfer_mi355x_prefill_workspace_bytes(const dyninfer_qweight_t* ws, uint32_t count, uint32_t rows,
                                            uint32_t x_dtype, uint32_t y_dtype, uint64_t* out_bytes);

/*
 * No counterpart in the reference.  For callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops or harnesses that forbid hipMalloc):
 * dyninfer_mi355x_qlinear_multi with the prefill staging workspace (a call that runs the
 * prefill GEMM: dyninfer_mi355x_prefill_workspace_bytes) taken from a static device
 * array of DYNINFER_MI355X_NOALLOC_SCRATCH_BYTES per device (allocated when the
 * library's code object loads on a device, held until the process ends) instead of a
 * caller-supplied workspace, for callers that can neither allocate nor hold one.  A larger staging is rejected with
 * DYNINFER_MI355X_ERR_UNSUPPORTED (2048 rows fit K <= 8128, 512 rows K <= 32704).
 * Calls no hipMalloc/hipFree or allocating routine.  Every call on one device shares
 * that device's array and leaves it holding the last staging: calls that overlap on
 * one device (concurrent streams, or threads without ordering) race and may return
 * wrong results; calls ordered on one stream are safe.  Decode calls stage their
 * activations in the array too where the MFMA GEMV takes the optional staging
 * (K/256 * 8.5 KiB, when that fits), with results identical to
 * dyninfer_mi355x_qlinear_multi's.
 */
#define DYNINFER_MI355X_NOALLOC_SCRATCH_BYTES (32u << 20)
int dyninfer_mi355x_qlinear_multi_noalloc(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* ws,
                                          uint32_t count, const void* x, uint32_t x_dtype, uint32_t rows,
                                          void* const* ys, uint32_t y_dtype, void* stream);

/*
 * Dequantise W to f32 [N, K] on the device, bit-exactly as the reference's
 * lowering does (gguf_codegen.rs:350-526 `emit_dequant`; mlx_affine.rs:593-598).
 * The qualification hook for bit-exact tests; not on the hot path.
 */
int dyninfer_mi355x_dequant(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w,
                            float* out, void* stream);

/*
 * Quantized embedding gather: out[i, :] = dequant(W[ids[i], :]) as f32, out [n_ids, K]
 * row-major, W [vocab = N, K] as for qlinear.  Replaces the Embedding lowering's
 * gather helper, one row per call there (gguf_codegen.rs:316-348 `emit_gather` with
 * the dequant body of :350-526, called from `emit_embedding_call` :214-232;
 * mlx_affine.rs:628-675 `emit_gather_u4`, called from :438-462); here n_ids rows in
 * one launch.  Values are bit-identical to dyninfer_mi355x_dequant's rows.
 * ids: device int64 [n_ids], 8-byte aligned; an id outside [0, vocab) yields a row
 * of NaN and reads no weight bytes (the reference leaves it undefined).  out: device,
 * 16-byte aligned.  n_ids == 0 is a no-op.
 */
int dyninfer_mi355x_embedding(dyninfer_mi355x_ctx_t* ctx, const dyninfer_qweight_t* w,
                              const int64_t* ids, uint32_t n_ids, float* out, void* stream);

/*
 * GGUF container index: the exact byte range of every tensor of a GGUF file, so a
 * weight reaches the device as a plain copy of its on-disk bytes (no repack).
 * Restates the reference's indexer (crates/dyninfer-checkpoint-gguf/src/container.rs:179-340:
 * magic, version 2..3, metadata, tensor directory with dims reversed to row-major,
 * data section at the header end rounded up to general.alignment, default 32, :16)
 * under its default inspection limits (crates/dyninfer-checkpoint/src/limits.rs), and
 * the provider plan's exact (file, offset, length) ranges (crates/dyninfer-checkpoint/src/provider.rs:9-60).
 * Tensors are listed sorted by name, as the reference's entries.  Duplicate tensor
 * names are rejected.
 */
typedef struct dyninfer_gguf dyninfer_gguf_t;

typedef struct dyninfer_gguf_tensor {
    const char* name;   /* NUL-terminated, owned by the index */
    uint32_t type_code; /* GgufType code (types.rs:10-45) */
    uint32_t n_dims;    /* logical rank */
    uint64_t dims[16];  /* row-major logical shape, dims[0] outermost */
    uint64_t offset;    /* absolute byte offset of the tensor's data in the file */
    uint64_t nbytes;    /* exact byte length */
} dyninfer_gguf_tensor_t;

/* Maps the file read-only and indexes it.  */
int dyninfer_mi355x_gguf_open(const char* path, dyninfer_gguf_t** out);
/* Indexes caller-owned bytes (they must outlive the index).  */
int dyninfer_mi355x_gguf_open_memory(const void* data, uint64_t len, dyninfer_gguf_t** out);
int dyninfer_mi355x_gguf_close(dyninfer_gguf_t* g);
uint64_t dyninfer_mi355x_gguf_tensor_count(const dyninfer_gguf_t* g);
/* Metadata key/values as one JSON object (keys sorted; f32/f64 as numbers, non-finite as null). */
const char* dyninfer_mi355x_gguf_metadata_json(const dyninfer_gguf_t* g);
int dyninfer_mi355x_gguf_tensor(const dyninfer_gguf_t* g, uint64_t index, dyninfer_gguf_tensor_t* out);
int dyninfer_mi355x_gguf_find(const dyninfer_gguf_t* g, const char* name, dyninfer_gguf_tensor_t* out);
/* Copies the tensor's exact bytes to device memory dst (dst_bytes >= nbytes) on `stream`,
 * then waits for the copy (the source is pageable mapped memory).  */
int dyninfer_mi355x_gguf_upload(const dyninfer_gguf_t* g, const char* name, void* dst, uint64_t dst_bytes,
                                void* stream);
/* Describes a rank-2 Q4_0/Q4_1/Q8_0/Q6_K/Q4_K/Q5_K/IQ4_XS tensor whose bytes are at device_data as a
 * dyninfer_qweight_t (rows = dims[0], cols = dims[1]); other types are unsupported. */
int dyninfer_mi355x_gguf_qweight(const dyninfer_gguf_t* g, const char* name, const void* device_data,
                                 dyninfer_qweight_t* out);

/*
 * SafeTensors container index and the MLX affine convention: the exact byte range of
 * every tensor of a .safetensors file, and an MLX quantized weight described from its
 * three components (`<stem>.weight` packed u32, `<stem>.scales`, `<stem>.biases`), so
 * each reaches the device as a plain copy of its on-disk bytes.  Restates the
 * reference's indexer (crates/dyninfer-checkpoint-safetensors/src/container.rs: 8-byte
 * little-endian header length of 1..64 MiB, JSON object header with "__metadata__",
 * dtype/shape/data_offsets per tensor, byte length = numel x element size, ranges inside
 * the file and not overlapping, the default inspection limits of
 * crates/dyninfer-checkpoint/src/limits.rs) and the MLX convention
 * (crates/dyninfer-checkpoint-safetensors/src/mlx.rs:17-261: metadata `format` "mlx",
 * mlx.quantization.bits / group_size from __metadata__ or from the sibling config.json's
 * quantization(_config) object, config_json.rs:129-143).  Tensors are listed sorted by
 * name.  A repeated tensor name is rejected (the reference's JSON map keeps the last).
 */
typedef struct dyninfer_safetensors dyninfer_safetensors_t;

typedef struct dyninfer_st_tensor {
    const char* name;   /* NUL-terminated, owned by the index */
    const char* dtype;  /* SafeTensors dtype string ("U32", "BF16", ...), owned by the index */
    uint32_t n_dims;
    uint64_t dims[16];  /* row-major shape */
    uint64_t offset;    /* absolute byte offset of the tensor's data in the file */
    uint64_t nbytes;    /* exact byte length */
} dyninfer_st_tensor_t;

/* Maps the file read-only, indexes it, and reads config.json beside it if present.  */
int dyninfer_mi355x_safetensors_open(const char* path, dyninfer_safetensors_t** out);
/* Indexes caller-owned bytes (they must outlive the index); config_json is the text of
 * the checkpoint's config.json, or NULL.  */
int dyninfer_mi355x_safetensors_open_memory(const void* data, uint64_t len, const char* config_json,
                                            dyninfer_safetensors_t** out);
int dyninfer_mi355x_safetensors_close(dyninfer_safetensors_t* t);
uint64_t dyninfer_mi355x_safetensors_tensor_count(const dyninfer_safetensors_t* t);
/* __metadata__ plus the config.json quantization keys, one JSON object (keys sorted). */
const char* dyninfer_mi355x_safetensors_metadata_json(const dyninfer_safetensors_t* t);
int dyninfer_mi355x_safetensors_tensor(const dyninfer_safetensors_t* t, uint64_t index, dyninfer_st_tensor_t* out);
int dyninfer_mi355x_safetensors_find(const dyninfer_safetensors_t* t, const char* name, dyninfer_st_tensor_t* out);
/* Copies the tensor's exact bytes to device memory dst (dst_bytes >= nbytes) on `stream`,
 * then waits for the copy (the source is pageable mapped memory).  */
int dyninfer_mi355x_safetensors_upload(const dyninfer_safetensors_t* t, const char* name, void* dst,
                                       uint64_t dst_bytes, void* stream);
/* Validates the MLX weight `weight_name` (a ".weight" tensor) as decode_affine_weight
 * (mlx.rs:152-261: u32 storage, scales and biases of one float type f16/bf16/f32, shapes
 * [N, K/group] with K = packed_last * 32 / bits) plus this library's limits (4-bit codes,
 * rank 2), and describes the three components uploaded at device_packed / device_scales /
 * device_biases as a dyninfer_qweight_t (rows N, cols K, byte lengths the tensors'). */
int dyninfer_mi355x_safetensors_mlx_qweight(const dyninfer_safetensors_t* t, const char* weight_name,
                                            const void* device_packed, const void* device_scales,
                                            const void* device_biases, dyninfer_qweight_t* out);

/*
 * 1 if (w, rows, x_dtype, y_dtype) is inside the qualified envelope, else 0 (and
 * last_error says why).  Host-only; same rules as the validation in
 * q4_0.rs:40-113 / gguf_block.rs:66-156 / mlx_affine.rs:55-155 plus this
 * library's shape limits.  Pointers are checked for alignment only.
 */
int dyninfer_mi355x_supports(const dyninfer_qweight_t* w, uint32_t rows, uint32_t x_dtype,
                             uint32_t y_dtype);

/*
 * Kernel-registry candidates qualified for gfx950, as a JSON array of serde
 * KernelCandidateDescriptor objects (crates/dyninfer-kernel-registry/src/lib.rs:132-149),
 * the counterpart of QuantizationDefinition::kernel_candidates
 * (gguf_codegen.rs:50-113, mlx_affine.rs:157-238).  Static storage; never free it.
 */
const char* dyninfer_mi355x_candidates_json(void);

/*
 * C++ restatement of KernelRegistry::select (crates/dyninfer-kernel-registry/src/lib.rs:302-348),
 * rejection_reasons (:499-584) and DeterministicCostModel (:249-268) over serde JSON:
 *   candidates_json: JSON array of KernelCandidateDescriptor (NULL = this library's own set)
 *   request_json:    KernelRequest object (:152-167)
 *   target_json:     TargetProfile object (crates/dyninfer-core/src/types.rs:244-272; driver,
 *                    architecture, features are read)
 * Writes a SelectionReport object (:218-223) to out (NUL-terminated) and its length
 * to *out_len.  Duplicate candidate ids fail like KernelRegistry::register (:283-296).
 */
int dyninfer_mi355x_registry_select(const char* candidates_json, const char* request_json,
                                    const char* target_json, char* out, size_t out_cap,
                                    size_t* out_len);

/*
 * KernelRegistry::require (lib.rs:350-399): like registry_select but writes the
 * SelectedKernelCandidate object, and when nothing is selected returns
 * DYNINFER_MI355X_ERR_UNSUPPORTED with last_error starting "E_KERNEL_COVERAGE".
 */
int dyninfer_mi355x_registry_require(const char* candidates_json, const char* request_json,
                                     const char* target_json, char* out, size_t out_cap,
                                     size_t* out_len);

/*
 * The compiler's precision gate for a selected lowering (crates/dyninfer-compiler/src/
 * lib.rs:289-306), restated and relaxed for bf16 activations.  selected_json is a
 * SelectedKernelCandidate (as registry_require writes); activation_type is the model's
 * activation dtype, "f32" (NULL) or "bf16".  Accepted, as in the reference: an i64 input
 * (embedding ids), or f32 input/output/activation/accumulator.  Also accepted when
 * activation_type is "bf16": bf16 input/output/activation with f32 accumulation on a
 * ".mi355x_hip" lowering (this library's kernels take and return bf16 activations).
 * Anything else returns DYNINFER_MI355X_ERR_UNSUPPORTED with the reference's
 * lower.precision message in last_error.
 * Registry extension used with it: a KernelRequest may carry "activation_type"; linear and
 * output_projection candidates whose first input type differs are then rejected with
 * reason "activation_type_mismatch" (requests without the field select as the reference).
 */
int dyninfer_mi355x_precision_check(const char* selected_json, const char* activation_type);

/* Library version string and the KernelRegistry::VERSION this registry expects ("6"). */
const char* dyninfer_mi355x_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DYNINFER_MI355X_H */
