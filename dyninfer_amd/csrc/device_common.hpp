// Shared gfx950 device helpers for the quantized weight-matmul kernels.
//
// Encodings are consumed in their on-disk byte layout (no repack):
//   GGUF blocks (gguf_codegen.rs:15-48): Q4_0 18 B / 32 w, Q4_1 20 B / 32 w,
//   Q8_0 34 B / 32 w, Q6_K 210 B / 256 w; row o, block b at (o*K/B + b)*bytes.
//   GGUF Q4_K super-blocks (GGML layout; the reference declares the schema,
//   gguf_block.rs:183-316): 144 B / 256 w.
//   MLX affine U4: packed u32 [N, K/8] + scales/biases [N, K/g].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmx {

// Multi-dword vector types that only promise 4-byte alignment: GGUF blocks are
// 2-byte aligned, so every weight load is issued from the 4-byte-aligned dword
// that contains the block start and realigned in registers.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

// A generic pointer re-typed as a global-memory (address space 1) pointer, so
// loads compile to global_load_* instead of flat_load_*.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const void* p) {
    return (const __attribute__((address_space(1))) T*)(p);
}

template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gptr_mut(void* p) {
    return (__attribute__((address_space(1))) T*)(p);
}

// floor(n / g) as one v_mul_hi_u32 with magic = ceil(2^32 / g) (group_magic):
// magic = (2^32 + e) / g with 0 <= e < g, so n·magic / 2^32 = n/g + n·e/(g·2^32),
// and for n·e < 2^32 (every n and g below 2^16: the GEMV's K bound) the excess
// stays below 1/g and the floor is exact.  The MLX kernels find a k's scale
// group this way instead of by a 32-bit division (~8 VALU instructions each).
__device__ __forceinline__ uint32_t div_magic(uint32_t n, uint32_t magic) { return __umulhi(n, magic); }

// 16 bytes per lane from global memory into LDS at dst + 16·lane (dst
// wave-uniform): global_load_lds_dwordx4, counted by vmcnt.
__device__ __forceinline__ void dma16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// 4 bytes per lane into LDS at dst + 4·lane: global_load_lds_dword.
__device__ __forceinline__ void dma4(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
}

// s_waitcnt vmcnt(n), other counters unconstrained.
template <uint32_t n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8));
}

// The barrier after LDS DMA (a ring's step): this wave's copies older than its
// last n vector-memory loads have landed in LDS and its LDS accesses are done
// (s_waitcnt vmcnt(n) lgkmcnt(0)), then s_barrier.  __syncthreads() would
// also wait for the loads still in flight (its fence waits for vmcnt(0)); the
// empty asm statements keep the compiler from moving memory accesses across
// the barrier.
template <uint32_t n>
__device__ __forceinline__ void ring_barrier() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The wait of ring_barrier<n>() without the barrier: for a wave whose LDS
// copies no other wave reads or writes.
template <uint32_t n>
__device__ __forceinline__ void ring_wait() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4));
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
    return (float)h;  // v_cvt_f32_f16: exact widening (arith.extf)
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// f32 -> bf16 round-to-nearest-even (NaN quieted) by gfx950's v_cvt_pk_bf16_f32,
// two values per instruction: bit-identical on this part to the integer form
// (u + 0x7FFF + ((u >> 16) & 1)) >> 16 with NaN -> (u >> 16) | 0x40, over every
// class of input (ties, subnormals, infinities, NaN payloads).  The integer form
// with its NaN test compiled to a divergent branch per value.
typedef float dmx_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 dmx_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(dmx_f32x2{lo, hi}, dmx_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return (uint16_t)f32x2_to_bf16x2_bits(f, 0.0f); }

// Byte lane i of a dword as float (v_cvt_f32_ubyte{0..3}).
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
    return (float)((v >> (8 * I)) & 0xFFu);
}

// Load NDW consecutive dwords starting at a 4-byte-aligned address.  Every
// dword read overlaps the block being read, so no read leaves the page of a
// valid byte.
template <int NDW>
__device__ __forceinline__ void load_dwords(const uint32_t* __restrict__ p, uint32_t (&d)[NDW]) {
#pragma unroll
    for (int i = 0; i + 4 <= NDW; i += 4) {
        u32x4_a4 v = *gptr<u32x4_a4>(p + i);
        d[i] = v.x; d[i + 1] = v.y; d[i + 2] = v.z; d[i + 3] = v.w;
    }
    constexpr int R = NDW & 3;
    constexpr int B0 = NDW - R;
    if constexpr (R == 3) {
        u32x2_a4 v = *gptr<u32x2_a4>(p + B0);
        d[B0] = v.x; d[B0 + 1] = v.y; d[B0 + 2] = *gptr<uint32_t>(p + B0 + 2);
    } else if constexpr (R == 2) {
        u32x2_a4 v = *gptr<u32x2_a4>(p + B0);
        d[B0] = v.x; d[B0 + 1] = v.y;
    } else if constexpr (R == 1) {
        d[B0] = *gptr<uint32_t>(p + B0);
    }
}

// Realign NDW raw dwords (loaded from the aligned dword containing the block
// start) by `sh` bytes (0 or 2) so that e[0] holds block bytes 0..3.  The last
// dword only needs its low half (blocks with bytes % 4 == 2).
template <int NDW>
__device__ __forceinline__ void realign(const uint32_t (&raw)[NDW], uint32_t sh, uint32_t (&e)[NDW]) {
#pragma unroll
    for (int i = 0; i + 1 < NDW; i++) e[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
    e[NDW - 1] = __builtin_amdgcn_alignbyte(raw[NDW - 1], raw[NDW - 1], sh);
}

// Q4_K sub-block j's (0..7) 6-bit scale and min from the super-block's 12
// scale bytes s12 (GGML get_scale_min_k4): j < 4 in the low 6 bits of bytes j
// and j + 4; j >= 4 split into a nibble of byte j + 4 (scale low, min high)
// and the top two bits of bytes j - 4 (scale) and j (min).
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s12, uint32_t j, uint32_t& sc, uint32_t& m) {
    if (j < 4u) {
        sc = s12[j] & 63u;
        m = s12[j + 4u] & 63u;
    } else {
        sc = (s12[j + 4u] & 15u) | ((uint32_t)(s12[j - 4u] >> 6) << 4);
        m = (uint32_t)(s12[j + 4u] >> 4) | ((uint32_t)(s12[j] >> 6) << 4);
    }
}

// The same for the two sub-blocks 2i and 2i + 1 (i = 0..3) from the scale
// bytes held as dwords s0 = bytes 0..3, s1 = 4..7, s2 = 8..11: they sit at
// byte positions 2(i & 1) and 2(i & 1) + 1 of each.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t i,
                                                   uint32_t (&sc)[2], uint32_t (&mn)[2]) {
    const uint32_t sh = 16u * (i & 1u);
    const uint32_t A = s0 >> sh, M = s1 >> sh, L = s2 >> sh;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint32_t a = (A >> (8 * g)) & 0xFFu, m = (M >> (8 * g)) & 0xFFu, l = (L >> (8 * g)) & 0xFFu;
        sc[g] = i < 2u ? (a & 63u) : ((l & 15u) | ((a >> 6) << 4));
        mn[g] = i < 2u ? (m & 63u) : ((l >> 4) | ((m >> 6) << 4));
    }
}

// IQ4_XS / IQ4_NL: GGML's kvalues_iq4nl codebook (a constant of the format)
//   {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}
// held as the bytes v + 128 (v ^ 0x80: unsigned, so an entry decodes like a
// Q8_0 code), four entries per dword.
constexpr uint32_t kIq4nlT0 = 0x3F2D1801u, kIq4nlT1 = 0x766A5D4Fu, kIq4nlT2 = 0xA6998D81u, kIq4nlT3 = 0xF1D9C5B5u;

// The codebook bytes (v + 128) of four 4-bit indices held one per byte of
// idx (each 0..15): entries 0..7 and 8..15 by one v_perm_b32 each, merged by
// each index's bit 3 (a v_perm selector of 12 gives 0x00, of 13 0xFF).
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t idx) {
    const uint32_t lo = __builtin_amdgcn_perm(kIq4nlT1, kIq4nlT0, idx);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4nlT3, kIq4nlT2, idx & 0x07070707u);
    const uint32_t msel = ((idx >> 3) & 0x01010101u) | 0x0C0C0C0Cu;
    const uint32_t mask = __builtin_amdgcn_perm(0u, 0u, msel);
    return (hi & mask) | (lo & ~mask);  // v_bfi_b32
}

// IQ4_XS sub-block ib's (0..7) 6-bit scale: nibble ib & 1 of scales_l[ib / 2]
// (sl = scales_l as a dword) | bits 2ib..2ib+1 of scales_h (sh) << 4.
__device__ __forceinline__ uint32_t iq4xs_scale(uint32_t sh, uint32_t sl, uint32_t ib) {
    return ((sl >> (4u * ib)) & 15u) | (((sh >> (2u * ib)) & 3u) << 4);
}

}  // namespace dmx
