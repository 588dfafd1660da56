// Internal host-side interface between the C ABI (capi.cpp) and the kernel
// translation units.  Not part of the public boundary.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmx {

constexpr int kMaxProblems = 4;  // weights sharing one activation per GEMV launch
constexpr int kMaxGemvBatch = 16;

enum Enc : uint32_t {
    ENC_Q4_0 = 2,
    ENC_Q4_1 = 3,
    ENC_Q8_0 = 8,
    ENC_Q4_K = 12,
    ENC_Q5_K = 13,
    ENC_Q6_K = 14,
    ENC_IQ4_XS = 23,
    ENC_MLX_U4 = 0x1004
};
enum DType : uint32_t { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// Kernel parameters of one GEMV launch (passed by value as the kernel
// argument).  The fields that address the first weight loads lead, in the
// first 96 bytes, so that they arrive in one round of scalar loads.
// ceil(2^32 / g) for div_magic (g >= 2); 0 for g = 0.
inline uint32_t group_magic(uint32_t g) { return g < 2u ? 0u : (uint32_t)(((1ull << 32) + g - 1u) / g); }

struct GemvParams {
    const uint8_t* w[kMaxProblems];   // GGUF blocks, or MLX packed words
    uint32_t n[kMaxProblems];
    uint32_t rb_begin[kMaxProblems];  // first row block of each problem
    uint32_t total_rb;                // row blocks over all problems
    uint32_t grid;                    // workgroups launched (set by the launcher)
    uint32_t K;
    uint32_t lanes_log2;  // lanes cooperating on one weight row (L = 2^lanes_log2 divides K/chunk)
    uint32_t nprob;
    uint32_t ldx;         // activation row stride, elements
    uint32_t ldy;         // output row stride, elements (per problem: its N)
    uint32_t batch;       // activation rows actually present (<= kernel's B)
    const void* x;
    void* y[kMaxProblems];
    const uint8_t* sc[kMaxProblems];  // MLX scales
    const uint8_t* bi[kMaxProblems];  // MLX biases
    uint32_t y_bf16;      // store bf16 instead of f32
    uint32_t group;       // MLX group size
    uint32_t gmagic;      // group_magic(group)
    uint32_t sdtype;      // MLX scale/bias dtype
    // Persistent pipeline: waves [wave_end[i-1], wave_end[i]) serve problem i
    // (wave_end[nprob-1] = all waves launched), each a contiguous run of the
    // problem's row blocks.
    uint32_t wave_end[kMaxProblems];
    // Streaming kernel: row steps per wave whose row sums the LDS holds until
    // the wave's stream ends (the busiest wave's count).
    uint32_t res_steps;
};

// Bytes of the GEMV activation tile in LDS per (activation row, chunk): the
// chunk's f16 pairs plus 16 bytes of bank padding, then its constants
// (gemv_kernels.hpp XTile).  Chunks: 32 weights, 64 for Q6_K, Q4_K and Q5_K.
__host__ __device__ constexpr bool wide_chunks(uint32_t enc) {
    return enc == ENC_Q6_K || enc == ENC_Q4_K || enc == ENC_Q5_K;
}
__host__ __device__ constexpr uint32_t xtile_chunk_weights(uint32_t enc) { return wide_chunks(enc) ? 64u : 32u; }
__host__ __device__ constexpr uint32_t xtile_chunk_bytes(uint32_t enc) {
    return enc == ENC_Q6_K ? 36u * 4u + 4u * 2u * 4u                      // 32 pair dwords + pad, 4 groups x (-C, s)
         : (enc == ENC_Q4_K || enc == ENC_Q5_K) ? 36u * 4u + 2u * 4u * 4u  // 32 + pad, 2 groups x (-C, s, s.Σx, 0)
         : (enc == ENC_Q8_0 || enc == ENC_Q4_0 || enc == ENC_IQ4_XS) ? 20u * 4u + 2u * 4u  // 16 + pad, (-C, s)
         : 20u * 4u + 4u * 4u;                                            // Q4_1, MLX: (-C, s, s.Σx, 0)
}
__host__ __device__ constexpr uint64_t xtile_bytes(uint32_t enc, uint32_t B, uint32_t K) {
    return (uint64_t)B * (K / xtile_chunk_weights(enc)) * xtile_chunk_bytes(enc);
}
// Widest activation batch one GEMV launch holds in registers (wider batches
// run as several launches): 8 rows, 4 for the 64-weight chunks.
__host__ __device__ constexpr uint32_t max_register_batch(uint32_t enc) { return wide_chunks(enc) ? 4u : 8u; }
// LDS of one gfx950 workgroup.
constexpr uint32_t kLdsBytes = 160u * 1024u;

struct GemvProblem {
    const uint8_t* w;
    const uint8_t* sc;
    const uint8_t* bi;
    void* y;
    uint32_t n;
};

// Decode GEMV: y_i[r, :] = x[r, :] · W_iᵀ for r < batch (<= 16).  work: an
// optional device workspace (256-byte aligned, or NULL) of work_bytes, used by
// the MFMA GEMV when it holds gemv_workspace_bytes.
hipError_t gemv_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x,
                       bool x_bf16, uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, void* work,
                       uint64_t work_bytes, hipStream_t stream);
// The workspace with which a decode GEMV call stages its activations once per
// call instead of once per workgroup (0: none helps).
uint64_t gemv_workspace_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                              bool y_bf16, uint32_t group);

// Decode GEMV on MFMA for 3..16 activation rows (Q4_0, Q6_K, Q4_K, Q5_K, IQ4_XS, MLX U4; K a
// multiple of 256): whether it serves a call, and the launch (K in several LDS
// segments adds into f32 outputs; bf16 outputs then take
// gemv_mfma_launch_bf16_acc below, given a workspace).
bool gemv_mfma_applies(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K, bool y_bf16,
                       uint32_t group);
hipError_t gemv_mfma_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x, bool x_bf16,
                            uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, void* work,
                            uint64_t work_bytes, hipStream_t stream);
// The workspace with which an MFMA GEMV call stages its activations once (the
// f16 fragments, inverse scales and offset sums of every 256-k task), or 0
// when it stages them in every workgroup; for bf16 outputs with K in several
// segments, gemv_mfma_bf16_acc_bytes.
uint64_t gemv_mfma_workspace_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                                   bool y_bf16, uint32_t group);
// bf16 outputs with K too long for one LDS segment: the workspace the MFMA
// GEMV needs to add its segments in f32 (the staged activations, then f32
// accumulators of every problem's [batch, n] outputs), or 0 when the launch is
// not such a case; and that launch (the workspace at least that large).
uint64_t gemv_mfma_bf16_acc_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                                  uint32_t group);
hipError_t gemv_mfma_launch_bf16_acc(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x,
                                     bool x_bf16, uint32_t batch, uint32_t group, uint32_t sdtype, void* work,
                                     uint64_t work_bytes, hipStream_t st);

// Whether one activation row of K elements fits the GEMV's LDS tile.
bool gemv_k_supported(uint32_t enc, uint32_t K);

// Bit-exact dequantisation to f32 [N, K].
hipError_t dequant_launch(uint32_t enc, const uint8_t* w, const uint8_t* sc, const uint8_t* bi, uint32_t N,
                          uint32_t K, uint32_t group, uint32_t sdtype, float* out, hipStream_t stream);

// Embedding gather: out[i, :] = dequant(W[ids[i], :]) in f32, [n_ids, K]; ids outside
// [0, vocab) give a NaN row.  out must be 16-byte aligned.
hipError_t gather_launch(uint32_t enc, const uint8_t* w, const uint8_t* sc, const uint8_t* bi, uint32_t vocab,
                         uint32_t K, uint32_t group, uint32_t sdtype, const int64_t* ids, uint32_t n_ids, float* out,
                         hipStream_t stream);

// Prefill activations staged for the MFMA GEMM (xprep.hip): f16 operand
// fragments of v_mfma_f32_32x32x16_f16, row m scaled by 2^(15 - e_m) (rs[m] =
// 2^(e_m - 15) undoes it), k ordered inside every 64-k chunk as the GEMM's
// weight decode produces the weights; rows padded with zeros to a multiple of
// 32.  Lane half h of k step 4c + t holds 8 k of k = 64c + 32h + (0..31):
enum XFrag : uint32_t {
    XFRAG_NIB = 2,   // Q4_0, Q4_1: 4t, 4t+2, 4t+1, 4t+3, 16+4t, 18+4t, 17+4t, 19+4t
    XFRAG_BYTE = 3,  // Q8_0, Q6_K, Q4_K: 8t + (0, 2, 1, 3, 4, 6, 5, 7)
    XFRAG_WORD = 4,  // MLX U4:     8t + (0, 4, 1, 5, 2, 6, 3, 7)
};
hipError_t xprep_launch(const void* x, bool x_bf16, uint32_t M, uint32_t K, uint32_t layout, uint16_t* xh, float* rs,
                        hipStream_t stream);

// Device workspace of one prefill GEMM call: xh (M rounded up to 32 rows of K
// f16) then rs (f32 for M rows rounded up to 256, so epilogues may read whole
// row groups past M).
inline uint64_t prefill_xh_bytes(uint32_t M, uint32_t K) {
    return (((uint64_t)M + 31u) / 32u * 32u * K * 2u + 255u) & ~(uint64_t)255u;
}
inline uint64_t prefill_workspace_bytes(uint32_t M, uint32_t K) {
    return prefill_xh_bytes(M, K) + (((uint64_t)M + 255u) & ~(uint64_t)255u) * 4u;
}

// Prefill GEMM launch plan (gemm.hip): workgroups of four waves, each owning a
// (32·tm) x (32·nb·4/s) tile of Y, the waves split over s K slices.
struct GemmPlan {
    uint32_t tm, nb, s;
    uint32_t mt, nt;  // workgroup tiles along M and N
};
GemmPlan gemm_plan(uint32_t enc, uint32_t N, uint32_t K, uint32_t M);

// Prefill GEMM on MFMA (gemm.hip): Y[M, N] = diag(rs) · (Xh[M, K] · Wᵀ), Xh/rs
// from xprep_launch(gemm_layout(enc)); Y f32 or bf16.  gemm_layout returns ~0u
// for encodings without a GEMM.  The weight: GGUF blocks at w, or MLX U4
// packed words at w with scales sc and biases bi [N, K/group] of dtype sdtype.
struct GemmWeight {
    uint32_t enc;
    const uint8_t* w;
    const uint8_t* sc;
    const uint8_t* bi;
    uint32_t group, sdtype;
};
uint32_t gemm_layout(uint32_t enc);
bool gemm_supported(uint32_t enc, uint32_t N, uint32_t K, uint32_t M);
hipError_t gemm_launch(const GemmWeight& wt, uint32_t N, uint32_t K, const uint16_t* xh, const float* rs, uint32_t M,
                       void* y, bool y_bf16, hipStream_t stream);

}  // namespace dmx
