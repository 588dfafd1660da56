// Bit-exact device dequantisation (the qualification hook; not on the hot path).
//
// Each formula is the reference's literal MLIR body, evaluated in the same
// order with the same f32 operations:
//   Q4_0  f32(q - 8) * f32(d) + 0.0          gguf_codegen.rs:425-470 (zero point 8, bias 0.0)
//   Q4_1  f32(q) * f32(d) + f32(m)           gguf_codegen.rs:425-470 (minimum = f16 word 1)
//   Q8_0  f32(sext(q)) * f32(d)              gguf_codegen.rs:382-410
//   Q6_K  (f32(q6 - 32) * f32(sc)) * f32(d)  gguf_codegen.rs:474-526
//   MLX   f32(q) * s + b                     mlx_affine.rs:593-598
//   Q4_K  (f32(d) * f32(sc)) * f32(q) - f32(dmin) * f32(m)   GGML dequantize_row_q4_K
//   Q5_K  the same with 5-bit q                               GGML dequantize_row_q5_K
//   IQ4_XS (f32(d) * f32(ls - 32)) * f32(kvalues_iq4nl[q])    GGML dequantize_row_iq4_xs
//         (the reference declares these schemas only, gguf_block.rs:183-316)
// Products that are exact (all but MLX with f32 scales) make fma contraction
// harmless; the MLX f32-scale product is rounded explicitly before the add.
#include "device_common.hpp"
#include "kernels.hpp"

// hipcc contracts a*b+c into fma by default (-ffp-contract=fast-honor-pragmas);
// the reference rounds every product before the add, so contraction is off here.
#pragma clang fp contract(off)

namespace dmx {

__device__ __forceinline__ uint32_t load_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t load_u16le(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// One thread per (block, 32-weight slice): GGUF blocks.
template <uint32_t ENC>
__global__ __launch_bounds__(256) void gguf_dequant_kernel(const uint8_t* __restrict__ w, uint64_t nslices,
                                                           float* __restrict__ out) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;  // launched with 256 threads
    if (t >= nslices) return;
    float* o = out + t * 32;
    if constexpr (ENC == ENC_Q4_0) {
        const uint8_t* blk = w + t * 18;
        const float d = f16_bits_to_f32(load_u16le(blk));
        for (int l = 0; l < 16; l++) {
            const uint32_t byte = load_u8(blk + 2 + l);
            o[l] = (float)((int32_t)(byte & 15u) - 8) * d + 0.0f;
            o[16 + l] = (float)((int32_t)(byte >> 4) - 8) * d + 0.0f;
        }
    } else if constexpr (ENC == ENC_Q4_1) {
        const uint8_t* blk = w + t * 20;
        const float d = f16_bits_to_f32(load_u16le(blk));
        const float m = f16_bits_to_f32(load_u16le(blk + 2));
        for (int l = 0; l < 16; l++) {
            const uint32_t byte = load_u8(blk + 4 + l);
            o[l] = (float)(byte & 15u) * d + m;
            o[16 + l] = (float)(byte >> 4) * d + m;
        }
    } else if constexpr (ENC == ENC_Q8_0) {
        const uint8_t* blk = w + t * 34;
        const float d = f16_bits_to_f32(load_u16le(blk));
        for (int l = 0; l < 32; l++) o[l] = (float)(int8_t)load_u8(blk + 2 + l) * d;
    } else if constexpr (ENC == ENC_Q4_K || ENC == ENC_Q5_K) {  // slice t = sub-block t & 7 of super-block t/8
        constexpr uint32_t BB = ENC == ENC_Q4_K ? 144u : 176u, QS = ENC == ENC_Q4_K ? 16u : 48u;
        const uint8_t* blk = w + (t >> 3) * BB;
        const uint32_t j = (uint32_t)(t & 7u);
        const float d = f16_bits_to_f32(load_u16le(blk)), dmin = f16_bits_to_f32(load_u16le(blk + 2));
        uint32_t sc, m;
        q4k_scale_min(blk + 4, j, sc, m);
        const float ds = d * (float)sc, dm = dmin * (float)m;
        const uint8_t* q = blk + QS + 32 * (j >> 1);
        const uint32_t sh = 4u * (j & 1u);  // odd sub-blocks are the high nibbles
        for (int l = 0; l < 32; l++) {
            uint32_t c = (load_u8(q + l) >> sh) & 15u;
            if constexpr (ENC == ENC_Q5_K) c |= ((load_u8(blk + 16 + l) >> j) & 1u) << 4;  // bit j of qh[l]
            o[l] = ds * (float)c - dm;
        }
    } else if constexpr (ENC == ENC_IQ4_XS) {  // slice t = sub-block t & 7 of super-block t/8
        const uint8_t* blk = w + (t >> 3) * 136;
        const uint32_t ib = (uint32_t)(t & 7u);
        const uint32_t ls = ((load_u8(blk + 4 + ib / 2) >> (4u * (ib & 1u))) & 15u) |
                            (((load_u16le(blk + 2) >> (2u * ib)) & 3u) << 4);
        const float dl = f16_bits_to_f32(load_u16le(blk)) * (float)((int32_t)ls - 32);
        const uint8_t* q = blk + 8 + 16 * ib;
        for (int l = 0; l < 16; l++) {
            const uint32_t byte = load_u8(q + l);
            // codebook entry = (v + 128) - 128, exact
            o[l] = dl * (float)((int32_t)(iq4nl_lookup(byte & 15u) & 0xFFu) - 128);
            o[16 + l] = dl * (float)((int32_t)(iq4nl_lookup(byte >> 4) & 0xFFu) - 128);
        }
    } else {  // Q6_K: slice t = (super-block t/8, n, h, p) of 32 weights
        const uint64_t sb = t >> 3;
        const uint32_t r = (uint32_t)(t & 7u);
        const int n = (int)(r >> 2), h = (int)((r >> 1) & 1u), p = (int)(r & 1u);
        const uint8_t* blk = w + sb * 210;
        const float d = f16_bits_to_f32(load_u16le(blk + 208));
        for (int j = 0; j < 32; j++) {
            const int s = j >> 4;
            const uint32_t lb = load_u8(blk + n * 64 + p * 32 + j);
            const int32_t low = h ? (int32_t)(lb >> 4) : (int32_t)(lb & 15u);
            const int32_t high = (int32_t)((load_u8(blk + 128 + n * 32 + j) >> (2 * (2 * h + p))) & 3u);
            const int32_t q = low + 16 * high - 32;
            const float sc = (float)(int8_t)load_u8(blk + 192 + n * 8 + h * 4 + p * 2 + s);
            o[j] = ((float)q * sc) * d;
        }
    }
}

// One thread per packed u32 word (8 weights): MLX affine U4.
__global__ __launch_bounds__(256) void mlx_u4_dequant_kernel(const uint32_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ sc,
                                                             const uint8_t* __restrict__ bi, uint64_t nwords,
                                                             uint32_t K, uint32_t group, uint32_t sdtype,
                                                             float* __restrict__ out) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;  // launched with 256 threads
    if (t >= nwords) return;
    const uint64_t k0 = t * 8;  // flat index of the word's first weight
    const uint64_t row = k0 / K;
    const uint64_t col = k0 % K;
    const uint64_t gi = row * (K / group) + col / group;
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
    const uint32_t v = packed[t];
    for (int i = 0; i < 8; i++) out[k0 + i] = (float)((v >> (4 * i)) & 15u) * s + b;
}

hipError_t dequant_launch(uint32_t enc, const uint8_t* w, const uint8_t* sc, const uint8_t* bi, uint32_t N,
                          uint32_t K, uint32_t group, uint32_t sdtype, float* out, hipStream_t stream) {
    const dim3 block(256);
    if (enc == ENC_MLX_U4) {
        const uint64_t nwords = (uint64_t)N * K / 8;
        hipLaunchKernelGGL(mlx_u4_dequant_kernel, dim3((unsigned)((nwords + 255) / 256)), block, 0, stream,
                           reinterpret_cast<const uint32_t*>(w), sc, bi, nwords, K, group, sdtype, out);
        return hipGetLastError();
    }
    const uint64_t nslices = (uint64_t)N * K / 32;
    const dim3 grid((unsigned)((nslices + 255) / 256));
    switch (enc) {
    case ENC_Q4_0: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q4_0>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_Q4_1: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q4_1>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_Q8_0: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q8_0>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_Q6_K: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q6_K>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_Q4_K: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q4_K>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_Q5_K: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_Q5_K>, grid, block, 0, stream, w, nslices, out); break;
    case ENC_IQ4_XS: hipLaunchKernelGGL(gguf_dequant_kernel<ENC_IQ4_XS>, grid, block, 0, stream, w, nslices, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dmx
