// Per-encoding chunk decoders for the gfx950 GEMV kernels.
//
// A "chunk" is the unit one lane processes per step: CW consecutive weights of
// one row, split into NG scale groups of GW = CW/NG weights.  Within a group
// every weight is w = d·c + m with an unsigned integer code c (0..255) and two
// f32 constants (d, m) of the group, so the kernel computes
//     Σ_k w_k x_k = d · Σ_k c_k x_k + m · Σ_k x_k
// with one byte->float convert and one fma per weight and activation row,
// and two fmas per group.  The (c, d, m) of each encoding, against the
// reference's dequantisation (gguf_codegen.rs:382-526, mlx_affine.rs:593-598):
//   Q4_0  c = nibble q,            d = f16 d,        m = -8·d        (w = (q-8)·d)
//   Q4_1  c = nibble q,            d = f16 d,        m = f16 m       (w = q·d + m)
//   Q8_0  c = int8 q + 128,        d = f16 d,        m = -128·d      (w = q·d)
//   Q6_K  c = 6-bit q (0..63),     d = sc·d,         m = -32·sc·d    (w = (q-32)·sc·d)
//   MLX   c = nibble q,            d = scale,        m = bias        (w = q·s + b)
// (-8·d, -128·d, -32·sc·d and sc·d are exact in f32.)  The contraction is
// therefore the reference's up to f32 reassociation; the bit-exact
// dequantisation hook is dequant.hip.
//
// Codes are delivered four at a time, as the four bytes of a dword whose
// weights are four consecutive k (or, for MLX, in the order given by
// mlx quad_perm), so the kernel converts them with v_cvt_f32_ubyte{0..3}.
#pragma once
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

// v & mask, hidden from the optimiser: with the mask's known zero bits the
// compiler would rewrite later byte extractions into v_bfe + v_cvt_f32_ubyte0
// instead of a single v_cvt_f32_ubyte{1,2,3}.
template <uint32_t MASK>
__device__ __forceinline__ uint32_t and_opaque(uint32_t v) {
    uint32_t r;
    asm("v_and_b32 %0, %2, %1" : "=v"(r) : "v"(v), "i"(MASK));
    return r;
}

// (a & MASK) | b, opaque (v_and_or_b32).
template <uint32_t MASK>
__device__ __forceinline__ uint32_t and_or_opaque(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %3, %2" : "=v"(r) : "v"(a), "v"(b), "s"(MASK));  // VOP3: no literal on gfx9
    return r;
}

// Raw dwords of a GGUF block, loaded from the 4-byte-aligned dword containing
// its first byte, with the byte shift (0 or 2) that realign() applies later.
// Realigning after the load keeps the loads free of consumers, so a lane can
// have every row's block in flight at once.
template <int NDW, class RAW>
__device__ __forceinline__ RAW load_raw_block(const uint8_t* p) {
    const uintptr_t a = (uintptr_t)p;
    RAW r;
    load_dwords<NDW>(reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3), r.d);
    r.sh = (uint32_t)(a & 3u);
    return r;
}

// ------------------------------------------------------------------ GGUF Q4_0
// 18-byte block: f16 d, 16 bytes; low nibble of byte l = weight l, high = 16+l
// (gguf_codegen.rs:412-472, lane map :452).
struct EncQ40 {
    static constexpr int CW = 32, NG = 1, GW = 32, NDW = 5, BB = 18;
    struct Chunk { uint32_t q[4]; float d; };
    struct Raw { uint32_t d[NDW]; uint32_t sh; };
    __device__ __forceinline__ static Raw load_raw(const uint8_t* row, uint32_t u) {
        return load_raw_block<NDW, Raw>(row + (size_t)u * 18u);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r) {
        uint32_t e[NDW];
        realign<NDW>(r.d, r.sh, e);
        Chunk c;
        c.d = f16_bits_to_f32(e[0]);
#pragma unroll
        for (int t = 0; t < 4; t++) c.q[t] = __builtin_amdgcn_alignbyte(e[t + 1], e[t], 2);
        return c;
    }
    __device__ __forceinline__ static float scale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float offset(const Chunk& c, int) { return -8.0f * c.d; }
    // quad j of group 0: j < 4 -> low nibbles of quant dword j (k = 4j);
    // j >= 4 -> high nibbles of dword j-4 (k = 16 + 4(j-4)).
    static constexpr int QUADS = 8;
    __device__ __forceinline__ static int kofs(int, int j) { return j < 4 ? 4 * j : 16 + 4 * (j - 4); }
    __device__ __forceinline__ static uint32_t codes(const Chunk& c, int, int j) {
        return j < 4 ? and_opaque<0x0F0F0F0Fu>(c.q[j]) : and_opaque<0x0F0F0F0Fu>(c.q[j - 4] >> 4);
    }
};

// ------------------------------------------------------------------ GGUF Q4_1
// 20-byte block: f16 d, f16 m, 16 bytes of nibbles (same lane map); blocks are
// 4-byte aligned (the C ABI requires a 4-byte-aligned base).
struct EncQ41 {
    static constexpr int CW = 32, NG = 1, GW = 32, NDW = 5, BB = 20;
    struct Chunk { uint32_t q[4]; float d, m; };
    struct Raw { uint32_t d[NDW]; };
    __device__ __forceinline__ static Raw load_raw(const uint8_t* row, uint32_t u) {
        Raw r;
        load_dwords<NDW>(reinterpret_cast<const uint32_t*>(row + (size_t)u * 20u), r.d);
        return r;
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r) {
        Chunk c;
        c.d = f16_bits_to_f32(r.d[0]);
        c.m = f16_bits_to_f32(r.d[0] >> 16);
#pragma unroll
        for (int t = 0; t < 4; t++) c.q[t] = r.d[t + 1];
        return c;
    }
    __device__ __forceinline__ static float scale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float offset(const Chunk& c, int) { return c.m; }
    static constexpr int QUADS = 8;
    __device__ __forceinline__ static int kofs(int, int j) { return j < 4 ? 4 * j : 16 + 4 * (j - 4); }
    __device__ __forceinline__ static uint32_t codes(const Chunk& c, int, int j) {
        return j < 4 ? and_opaque<0x0F0F0F0Fu>(c.q[j]) : and_opaque<0x0F0F0F0Fu>(c.q[j - 4] >> 4);
    }
};

// ------------------------------------------------------------------ GGUF Q8_0
// 34-byte block: f16 d, 32 int8 codes (gguf_codegen.rs:382-410).  Codes are
// flipped to q + 128 (xor 0x80) so they convert as unsigned bytes.
struct EncQ80 {
    static constexpr int CW = 32, NG = 1, GW = 32, NDW = 9, BB = 34;
    struct Chunk { uint32_t q[8]; float d; };
    struct Raw { uint32_t d[NDW]; uint32_t sh; };
    __device__ __forceinline__ static Raw load_raw(const uint8_t* row, uint32_t u) {
        return load_raw_block<NDW, Raw>(row + (size_t)u * 34u);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r) {
        uint32_t e[NDW];
        realign<NDW>(r.d, r.sh, e);
        Chunk c;
        c.d = f16_bits_to_f32(e[0]);
#pragma unroll
        for (int t = 0; t < 8; t++) c.q[t] = __builtin_amdgcn_alignbyte(e[t + 1], e[t], 2);
        return c;
    }
    __device__ __forceinline__ static float scale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float offset(const Chunk& c, int) { return -128.0f * c.d; }
    static constexpr int QUADS = 8;
    __device__ __forceinline__ static int kofs(int, int j) { return 4 * j; }
    __device__ __forceinline__ static uint32_t codes(const Chunk& c, int, int j) {
        uint32_t r;
        asm("v_xor_b32 %0, %2, %1" : "=v"(r) : "v"(c.q[j]), "i"(0x80808080u));
        return r;
    }
};

// ------------------------------------------------------------------ GGUF Q6_K
// 210-byte super-block of 256 (gguf_codegen.rs:474-526): ql = bytes 0..128,
// qh = 128..192, sc = int8 192..208, d = f16 208..210.  Weight
// n*128 + h*64 + p*32 + s*16 + l: low4 = nibble h of ql[n*64 + p*32 + s*16 + l],
// high2 = (qh[n*32 + s*16 + l] >> 2(2h+p)) & 3, sub-scale sc[n*8 + h*4 + p*2 + s].
// Group g = (n, h, p, s) = 16 weights; quads j = 0..3 are l = 4j..4j+3.
struct EncQ6K {
    static constexpr int CW = 256, NG = 16, GW = 16, NDW = 53, BB = 210;
    struct Chunk { uint32_t e[NDW]; };
    struct Raw { uint32_t d[NDW]; uint32_t sh; };
    __device__ __forceinline__ static Raw load_raw(const uint8_t* row, uint32_t u) {
        return load_raw_block<NDW, Raw>(row + (size_t)u * 210u);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r) {
        Chunk c;
        realign<NDW>(r.d, r.sh, c.e);
        return c;
    }
    __device__ __forceinline__ static float dsuper(const Chunk& c) { return f16_bits_to_f32(c.e[52]); }
    __device__ __forceinline__ static float scale(const Chunk& c, int g) {
        const int8_t sc = (int8_t)((c.e[48 + g / 4] >> (8 * (g % 4))) & 0xFFu);
        return (float)sc * dsuper(c);
    }
    __device__ __forceinline__ static float offset(const Chunk& c, int g) { return -32.0f * scale(c, g); }
    static constexpr int QUADS = 4;
    __device__ __forceinline__ static int kofs(int g, int j) {
        const int n = g >> 3, h = (g >> 2) & 1, p = (g >> 1) & 1, s = g & 1;
        return n * 128 + h * 64 + p * 32 + s * 16 + 4 * j;
    }
    __device__ __forceinline__ static uint32_t codes(const Chunk& c, int g, int j) {
        const int n = g >> 3, h = (g >> 2) & 1, p = (g >> 1) & 1, s = g & 1;
        const uint32_t ql = c.e[n * 16 + p * 8 + s * 4 + j];
        const uint32_t qh = c.e[32 + n * 8 + s * 4 + j];
        const uint32_t low = (ql >> (4 * h)) & 0x0F0F0F0Fu;
        const int hs = 2 * (2 * h + p);
        const uint32_t hi = hs <= 4 ? (qh << (4 - hs)) : (qh >> (hs - 4));
        return and_or_opaque<0x30303030u>(hi, low);
    }
};

// ------------------------------------------------------------------ MLX affine U4
// One chunk = 32 weights = 4 packed u32 words (weight i of a word = bits
// 4i..4i+3, fixture.rs:307-311) sharing one scale and bias (group size is a
// multiple of 32).  Quad j covers k = 4j..4j+3: word j/2, nibbles 4(j&1)..+3,
// i.e. bytes b0/b1 (j even) or b2/b3 (j odd) of lo = w & 0x0F0F0F0F (even
// nibbles) and hi = (w >> 4) & 0x0F0F0F0F (odd nibbles).  codes() interleaves
// them back into k order with one v_perm.
struct EncMlxU4 {
    static constexpr int CW = 32, NG = 1, GW = 32;
    static constexpr int QUADS = 8;
    struct Chunk { uint32_t w[4]; float s, b; };
    // raw: packed words plus the scale/bias bit patterns (f32, or f16/bf16 in the
    // low half) and their dtype
    struct Raw { uint32_t w[4]; uint32_t s, b, kind; };
    __device__ __forceinline__ static Chunk unpack(const Raw& r) {
        Chunk c;
#pragma unroll
        for (int i = 0; i < 4; i++) c.w[i] = r.w[i];
        if (r.kind == DT_F32) {
            c.s = __uint_as_float(r.s);
            c.b = __uint_as_float(r.b);
        } else if (r.kind == DT_F16) {
            c.s = f16_bits_to_f32(r.s);
            c.b = f16_bits_to_f32(r.b);
        } else {
            c.s = bf16_bits_to_f32(r.s);
            c.b = bf16_bits_to_f32(r.b);
        }
        return c;
    }
    __device__ __forceinline__ static int kofs(int, int j) { return 4 * j; }
    __device__ __forceinline__ static float scale(const Chunk& c, int) { return c.s; }
    __device__ __forceinline__ static float offset(const Chunk& c, int) { return c.b; }
    __device__ __forceinline__ static uint32_t codes(const Chunk& c, int, int j) {
        const uint32_t w = c.w[j >> 1];
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        // bytes (lo.b0, hi.b0, lo.b1, hi.b1) or (lo.b2, hi.b2, lo.b3, hi.b3)
        const uint32_t sel = (j & 1) ? 0x03070206u : 0x01050004u;
        return __builtin_amdgcn_perm(lo, hi, sel);
    }
};

}  // namespace dmx
