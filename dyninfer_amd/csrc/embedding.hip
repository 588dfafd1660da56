// Quantized embedding gather: out[i, :] = dequant(W[ids[i], :]) in f32.
//
// The reference lowers an Embedding on a GGUF weight to a row slice of the
// interleaved bytes followed by the same dequant body as the matmul
// (gguf_codegen.rs:316-348 `emit_gather`, body gguf_codegen.rs:350-526), and on
// an MLX U4 weight to row slices of packed/scales/biases with
// f32(q) * s + b (mlx_affine.rs:628-675 `emit_gather_u4`); GGUF Q4_K rows
// (a schema-only encoding in the reference) dequantize as GGML's
// dequantize_row_q4_K.  Each value here is
// computed with the same f32 operations in the same order, so the rows are
// bit-identical to the dequant hook's rows.
//
// Work split: one thread per 4 consecutive outputs of one gathered row, so a
// wave writes 1 KiB of contiguous f32 with 16-byte stores (the writes are 7x
// the Q4_0 bytes read and set the HBM bound).  The 4 outputs of a thread never
// straddle a GGUF block (32 or 256 weights), an MLX group (a multiple of 32) or
// a packed word's halves.  Ids outside [0, vocab) produce a row of quiet NaN
// and read nothing.
#include "device_common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace dmx {

namespace {

__device__ __forceinline__ uint32_t ld8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

template <uint32_t ENC>
__device__ __forceinline__ float4 gguf_four(const uint8_t* __restrict__ row, uint32_t k) {
    float v[4];
    if constexpr (ENC == ENC_Q4_0 || ENC == ENC_Q4_1) {
        const uint8_t* blk = row + (size_t)(k >> 5) * (ENC == ENC_Q4_0 ? 18u : 20u);
        const uint32_t l = k & 31u;  // 0, 4, ..., 28: lanes l..l+3 share one nibble half
        const float d = f16_bits_to_f32(ld16(blk));
        const uint8_t* q = blk + (ENC == ENC_Q4_0 ? 2u : 4u) + (l & 15u);
        const uint32_t sh = l >= 16u ? 4u : 0u;  // lanes 16..31 are the high nibbles
        if constexpr (ENC == ENC_Q4_0) {
            for (int i = 0; i < 4; i++) v[i] = (float)((int32_t)((ld8(q + i) >> sh) & 15u) - 8) * d + 0.0f;
        } else {
            const float m = f16_bits_to_f32(ld16(blk + 2));
            for (int i = 0; i < 4; i++) v[i] = (float)((ld8(q + i) >> sh) & 15u) * d + m;
        }
    } else if constexpr (ENC == ENC_Q8_0) {
        const uint8_t* blk = row + (size_t)(k >> 5) * 34u;
        const float d = f16_bits_to_f32(ld16(blk));
        const uint8_t* q = blk + 2 + (k & 31u);
        for (int i = 0; i < 4; i++) v[i] = (float)(int8_t)ld8(q + i) * d;
    } else if constexpr (ENC == ENC_Q4_K || ENC == ENC_Q5_K) {
        // idx = 64i + 32h + l: nibble h of qs[32i + l] (Q5_K: | bit 2i + h of qh[l] << 4), sub-block 2i + h
        constexpr uint32_t BB = ENC == ENC_Q4_K ? 144u : 176u, QS = ENC == ENC_Q4_K ? 16u : 48u;
        const uint8_t* blk = row + (size_t)(k >> 8) * BB;
        const uint32_t idx = k & 255u, jsub = idx >> 5;
        const float d = f16_bits_to_f32(ld16(blk)), dmin = f16_bits_to_f32(ld16(blk + 2));
        uint32_t sc, m;
        q4k_scale_min(blk + 4, jsub, sc, m);
        const float ds = d * (float)sc, dm = dmin * (float)m;
        const uint32_t l0 = idx & 31u;
        const uint8_t* q = blk + QS + 32 * (jsub >> 1) + l0;
        const uint32_t sh = 4u * (jsub & 1u);
        for (int i = 0; i < 4; i++) {
            uint32_t c = (ld8(q + i) >> sh) & 15u;
            if constexpr (ENC == ENC_Q5_K) c |= ((ld8(blk + 16 + l0 + i) >> jsub) & 1u) << 4;
            v[i] = ds * (float)c - dm;
        }
    } else if constexpr (ENC == ENC_IQ4_XS) {  // idx = 32ib + 16h + l: nibble h of qs[16ib + l]
        const uint8_t* blk = row + (size_t)(k >> 8) * 136u;
        const uint32_t idx = k & 255u, ib = idx >> 5, hh = (idx >> 4) & 1u;
        const uint32_t ls = ((ld8(blk + 4 + ib / 2) >> (4u * (ib & 1u))) & 15u) | (((ld16(blk + 2) >> (2u * ib)) & 3u) << 4);
        const float dl = f16_bits_to_f32(ld16(blk)) * (float)((int32_t)ls - 32);
        const uint8_t* q = blk + 8 + 16 * ib + (idx & 15u);
        for (int i = 0; i < 4; i++)
            v[i] = dl * (float)((int32_t)(iq4nl_lookup((ld8(q + i) >> (4u * hh)) & 15u) & 0xFFu) - 128);
    } else {  // Q6_K: idx = n*128 + h*64 + p*32 + s*16 + l (gguf_codegen.rs:499-503)
        const uint8_t* blk = row + (size_t)(k >> 8) * 210u;
        const uint32_t idx = k & 255u;
        const uint32_t n = idx >> 7, h = (idx >> 6) & 1u, p = (idx >> 5) & 1u, s = (idx >> 4) & 1u, l0 = idx & 15u;
        const float d = f16_bits_to_f32(ld16(blk + 208));
        const float sc = (float)(int8_t)ld8(blk + 192 + n * 8 + h * 4 + p * 2 + s);
        const uint8_t* ql = blk + n * 64 + p * 32 + s * 16 + l0;
        const uint8_t* qh = blk + 128 + n * 32 + s * 16 + l0;
        const uint32_t hs = 2u * (2u * h + p);
        for (int i = 0; i < 4; i++) {
            const uint32_t lb = ld8(ql + i);
            const int32_t low = (int32_t)(h ? (lb >> 4) : (lb & 15u));
            const int32_t high = (int32_t)((ld8(qh + i) >> hs) & 3u);
            v[i] = ((float)(low + 16 * high - 32) * sc) * d;
        }
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

}  // namespace

// grid.x = n_ids * per_row workgroups of 256 threads; thread t of a row covers outputs 4t..4t+3.
template <uint32_t ENC>
__global__ __launch_bounds__(256) void gguf_gather_kernel(const uint8_t* __restrict__ w, uint64_t row_bytes,
                                                          uint32_t vocab, uint32_t K, uint32_t per_row,
                                                          const int64_t* __restrict__ ids, float* __restrict__ out) {
    const uint32_t r = blockIdx.x / per_row;
    const uint32_t k = ((blockIdx.x - r * per_row) * 256u + threadIdx.x) * 4u;
    if (k >= K) return;
    const int64_t id = ids[r];
    float4 v;
    if (id < 0 || id >= (int64_t)vocab) {
        v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
    } else {
        v = gguf_four<ENC>(w + (uint64_t)id * row_bytes, k);
    }
    *reinterpret_cast<float4*>(out + (uint64_t)r * K + k) = v;
}

__global__ __launch_bounds__(256) void mlx_u4_gather_kernel(const uint32_t* __restrict__ packed,
                                                            const uint8_t* __restrict__ sc,
                                                            const uint8_t* __restrict__ bi, uint32_t vocab, uint32_t K,
                                                            uint32_t group, uint32_t sdtype, uint32_t per_row,
                                                            const int64_t* __restrict__ ids, float* __restrict__ out) {
    const uint32_t r = blockIdx.x / per_row;
    const uint32_t k = ((blockIdx.x - r * per_row) * 256u + threadIdx.x) * 4u;
    if (k >= K) return;
    const int64_t id = ids[r];
    float4 v;
    if (id < 0 || id >= (int64_t)vocab) {
        v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
    } else {
        const uint64_t gi = (uint64_t)id * (K / group) + k / group;
        float s, b;
        if (sdtype == DT_F32) {
            s = reinterpret_cast<const float*>(sc)[gi];
            b = reinterpret_cast<const float*>(bi)[gi];
        } else if (sdtype == DT_F16) {
            s = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(sc)[gi]);
            b = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(bi)[gi]);
        } else {
            s = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(sc)[gi]);
            b = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(bi)[gi]);
        }
        const uint32_t word = packed[(uint64_t)id * (K / 8) + k / 8] >> (4u * (k & 7u));  // lanes LSB first
        v = make_float4((float)(word & 15u) * s + b, (float)((word >> 4) & 15u) * s + b,
                        (float)((word >> 8) & 15u) * s + b, (float)((word >> 12) & 15u) * s + b);
    }
    *reinterpret_cast<float4*>(out + (uint64_t)r * K + k) = v;
}

hipError_t gather_launch(uint32_t enc, const uint8_t* w, const uint8_t* sc, const uint8_t* bi, uint32_t vocab,
                         uint32_t K, uint32_t group, uint32_t sdtype, const int64_t* ids, uint32_t n_ids, float* out,
                         hipStream_t stream) {
    const uint32_t per_row = (K / 4u + 255u) / 256u;
    const dim3 grid(n_ids * per_row), block(256);  // the caller bounds n_ids * per_row below 2^31
    if (enc == ENC_MLX_U4) {
        hipLaunchKernelGGL(mlx_u4_gather_kernel, grid, block, 0, stream, reinterpret_cast<const uint32_t*>(w), sc, bi,
                           vocab, K, group, sdtype, per_row, ids, out);
        return hipGetLastError();
    }
    switch (enc) {
    case ENC_Q4_0:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q4_0>, grid, block, 0, stream, w, (uint64_t)(K / 32) * 18u, vocab, K,
                           per_row, ids, out);
        break;
    case ENC_Q4_1:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q4_1>, grid, block, 0, stream, w, (uint64_t)(K / 32) * 20u, vocab, K,
                           per_row, ids, out);
        break;
    case ENC_Q8_0:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q8_0>, grid, block, 0, stream, w, (uint64_t)(K / 32) * 34u, vocab, K,
                           per_row, ids, out);
        break;
    case ENC_Q6_K:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q6_K>, grid, block, 0, stream, w, (uint64_t)(K / 256) * 210u, vocab,
                           K, per_row, ids, out);
        break;
    case ENC_Q4_K:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q4_K>, grid, block, 0, stream, w, (uint64_t)(K / 256) * 144u, vocab,
                           K, per_row, ids, out);
        break;
    case ENC_Q5_K:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_Q5_K>, grid, block, 0, stream, w, (uint64_t)(K / 256) * 176u, vocab,
                           K, per_row, ids, out);
        break;
    case ENC_IQ4_XS:
        hipLaunchKernelGGL(gguf_gather_kernel<ENC_IQ4_XS>, grid, block, 0, stream, w, (uint64_t)(K / 256) * 136u, vocab,
                           K, per_row, ids, out);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dmx
