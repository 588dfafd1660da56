// Per-encoding chunk decoders for the gfx950 GEMV kernels.
//
// A chunk is what one lane handles per step: CW weights of one row (one GGUF
// block, a quarter of a Q6_K super-block, 32 MLX weights).  Its integer codes
// become packed f16 pairs by the exponent trick: with a code c < 1024 in the
// mantissa bits, the f16 bit pattern 0x6400 | c is exactly 1024 + c, so one
// v_and_or_b32 decodes two weights.  A code at mantissa bits 4.. decodes to
// 1024 + 16c; those pairs meet activations stored divided by 16 (exact).
// v_dot2_f32_f16 multiplies two decoded codes by two f16 activations (each
// product exact in f32) and adds them to an f32 accumulator, which starts at
// -C for the chunk's scale group:
//     Σ_k (c_k - off)·v_k = Σ_k P_k·v_k - C,   C = Σ_k coef_k·v_k,
// coef = 1024 + off for pairs at bit 0 and 1024 + 16·off for pairs at bit 4,
// where P is the decoded pair value and v the stored activation.  v is the
// activation scaled by a power of two per scale group (largest magnitude in
// [2^13, 2^14), so f16 neither overflows nor flushes small values) and
// rounded to f16: the only rounding besides f32 accumulation, relative 2^-11
// per product, well inside the 2e-3 normalised tolerance.  The group result is
// then s·acc (s the power of two) times the weight scale, plus the weight
// offset times Σx for affine encodings.  Per encoding, against the
// reference's dequantisation (gguf_codegen.rs:382-526, mlx_affine.rs:593-598):
//   Q4_0  w = (q-8)·d            code q (nibble), off 8
//   Q4_1  w = q·d + m            code q,          off 0, + m·Σx
//   Q8_0  w = q·d                code q+128 (xor 0x80), off 128
//   Q6_K  w = (q-32)·sc·d        6-bit code q,    off 32, per 16-weight group
//   Q4_K  w = q·(d·sc) - dmin·m  code q,          off 0, - dmin·m·Σx, per 32-weight group
//   Q5_K  as Q4_K with 5-bit codes (a fifth bit from qh)
//   IQ4_XS w = kv[q]·(ls-32)·d   codebook byte kv[q]+128, off 128, per 32-weight sub-block
//   MLX   w = q·s + b            code q,          off 0, + b·Σx
//
// Layout contract with the activation staging (gemv_kernels.hpp): for code
// dword t of a chunk the lane reads PPT f16 pairs, pair h holding activations
// xoff(t, h, 0) and xoff(t, h, 1) (offsets from the chunk's first activation
// xbase(u)), divided by 16 when dv(t, h), accumulated into group grp(t, h).
// Those 2·PPT activations are exactly NXR runs of 4 consecutive ones, run r
// starting at xrun0(r) + TSTRIDE·t, and xoff(t, h, e) = xoff(0, h, e) +
// TSTRIDE·t, so one thread per code dword stages its pairs from NXR aligned
// 4-element loads (checked at compile time by xruns_ok).
#pragma once
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// c + a.lo·b.lo + a.hi·b.hi (v_dot2_f32_f16)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

constexpr uint32_t kMagic = 0x64006400u;  // f16 1024.0 in both halves

// (a & m) | b as one v_and_or_b32.  Written as asm because the compiler
// otherwise emits v_and_b32 + v_or_b32 with literal operands (a VOP3 op takes
// no literal on gfx9).  The mask lives in a scalar register and b in a vector
// register (gfx9 allows one scalar operand per VALU instruction), both loaded
// once outside the loops.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
    return r;
}

// Selector for v_perm_b32 that extracts the dword starting `sh` bytes into a
// 4-byte-aligned pair {hi, lo}, plus a fixed byte offset `add` (0 or 2).
__device__ __forceinline__ uint32_t realign_sel(uint32_t sh, uint32_t add) {
    return 0x03020100u + 0x01010101u * (sh + add);
}

// The four decoded pairs of a dword of nibble codes whose weights are
// (i, i+2) [bits 0-3 and 16-19], (j, j+2) x16 [bits 4-7 and 20-23],
// and the same one byte up [bits 8-11/24-27, 12-15/28-31].
__device__ __forceinline__ void nibble_pairs(uint32_t d, uint32_t (&p)[4]) {
    const uint32_t d8 = d >> 8;
    p[0] = and_or(d, 0x000F000Fu, kMagic);
    p[1] = and_or(d, 0x00F000F0u, kMagic);
    p[2] = and_or(d8, 0x000F000Fu, kMagic);
    p[3] = and_or(d8, 0x00F000F0u, kMagic);
}

// Raw dwords of a 2-byte-aligned GGUF block: NDW dwords from the 4-byte-
// aligned dword holding its first byte (each dword overlaps the block, so no
// load leaves a page the block touches), and the byte shift 0 or 2.
template <int NDW>
struct RawBlock {
    uint32_t d[NDW];
    uint32_t sh;
};

// A 2-byte-aligned block at byte offset `off` from a uniform base, addressed
// as the 4-byte-aligned uniform base abase = base & ~3 plus the per-lane
// 32-bit offset o = off + (base & 3) (32-bit offsets keep the address
// arithmetic per lane to one add; o never wraps, since the C ABI limits a
// weight to 4 GiB minus 16 bytes).  The loads start at abase + (o & ~3).
struct AlignedOffset {
    const uint8_t* abase;
    uint32_t o;
};

__device__ __forceinline__ AlignedOffset aligned_offset(const uint8_t* base, uint32_t off) {
    const uint32_t bsh = (uint32_t)((uintptr_t)base & 3u);
    return {base - bsh, off + bsh};
}

template <int NDW>
__device__ __forceinline__ RawBlock<NDW> load_raw_block(const uint8_t* base, uint32_t off) {
    const AlignedOffset a = aligned_offset(base, off);
    RawBlock<NDW> r;
    r.sh = a.o & 3u;
    load_dwords<NDW>(reinterpret_cast<const uint32_t*>(a.abase + (a.o & ~3u)), r.d);
    return r;
}

// ------------------------------------------------------------------ GGUF Q4_0
// 18-byte block: f16 d, 16 bytes qs; low nibble of qs[l] = weight l, high =
// weight 16+l (gguf_codegen.rs:412-472, lane map :452).  Code dword t = qs
// bytes 4t..4t+3.
struct EncQ40 {
    static constexpr uint32_t ENC = ENC_Q4_0;
    static constexpr int CW = 32, QK = 32, NT = 4, PPT = 4, NG = 1, NDW = 5, BB = 18;
    static constexpr bool AFFINE = false;
    static constexpr int NRUN = 1, RUNLEN = 32, RUNSTRIDE = 0;  // activation runs of a chunk
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 32u * u; }
    static constexpr float coef(bool dv) { return dv ? 1152.0f : 1032.0f; }
    static constexpr int xoff(int t, int h, int e) { return 4 * t + (h >> 1) + 2 * e + 16 * (h & 1); }
    static constexpr bool dv(int, int h) { return (h & 1) != 0; }
    static constexpr int grp(int, int) { return 0; }
    static constexpr int TSTRIDE = 4, NXR = 2;  // activations 4t..4t+3 and 16+4t..16+4t+3
    static constexpr int xrun0(int r) { return 16 * r; }
    using Raw = RawBlock<NDW>;
    struct Chunk { uint32_t q[NT]; float d; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        return load_raw_block<NDW>(w, rowoff + u * (uint32_t)BB);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t) {
        Chunk c;
        const uint32_t sel = realign_sel(r.sh, 2);
#pragma unroll
        for (int t = 0; t < NT; t++) c.q[t] = __builtin_amdgcn_perm(r.d[t + 1], r.d[t], sel);
        c.d = f16_bits_to_f32(r.d[0] >> (8u * r.sh));
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) { nibble_pairs(c.q[t], p); }
    __device__ __forceinline__ static float gscale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float goffset(const Chunk&, int) { return 0.0f; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) { c.d = z ? 0.0f : c.d; }
};

// ------------------------------------------------------------------ GGUF Q4_1
// 20-byte block: f16 d, f16 m, 16 bytes qs (same nibble map).  Blocks are
// 4-byte aligned (the C ABI requires a 4-byte-aligned base).
struct EncQ41 {
    static constexpr uint32_t ENC = ENC_Q4_1;
    static constexpr int CW = 32, QK = 32, NT = 4, PPT = 4, NG = 1, NDW = 5, BB = 20;
    static constexpr bool AFFINE = true;
    static constexpr int NRUN = 1, RUNLEN = 32, RUNSTRIDE = 0;
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 32u * u; }
    static constexpr float coef(bool) { return 1024.0f; }
    static constexpr int xoff(int t, int h, int e) { return EncQ40::xoff(t, h, e); }
    static constexpr bool dv(int t, int h) { return EncQ40::dv(t, h); }
    static constexpr int grp(int, int) { return 0; }
    static constexpr int TSTRIDE = EncQ40::TSTRIDE, NXR = EncQ40::NXR;
    static constexpr int xrun0(int r) { return EncQ40::xrun0(r); }
    struct Raw { uint32_t d[NDW]; };
    struct Chunk { uint32_t q[NT]; float d, m; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        Raw r;
        load_dwords<NDW>(reinterpret_cast<const uint32_t*>(w + (rowoff + u * (uint32_t)BB)), r.d);
        return r;
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t) {
        Chunk c;
#pragma unroll
        for (int t = 0; t < NT; t++) c.q[t] = r.d[t + 1];
        c.d = f16_bits_to_f32(r.d[0]);
        c.m = f16_bits_to_f32(r.d[0] >> 16);
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) { nibble_pairs(c.q[t], p); }
    __device__ __forceinline__ static float gscale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float goffset(const Chunk& c, int) { return c.m; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) {
        c.d = z ? 0.0f : c.d;
        c.m = z ? 0.0f : c.m;
    }
};

// ------------------------------------------------------------------ GGUF Q8_0
// 34-byte block: f16 d, 32 int8 codes (gguf_codegen.rs:382-410).  Codes are
// flipped to q + 128 (xor 0x80) so they decode as unsigned bytes.
struct EncQ80 {
    static constexpr uint32_t ENC = ENC_Q8_0;
    static constexpr int CW = 32, QK = 32, NT = 8, PPT = 2, NG = 1, NDW = 9, BB = 34;
    static constexpr bool AFFINE = false;
    static constexpr int NRUN = 1, RUNLEN = 32, RUNSTRIDE = 0;
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 32u * u; }
    static constexpr float coef(bool) { return 1152.0f; }
    static constexpr int xoff(int t, int h, int e) { return 4 * t + h + 2 * e; }
    static constexpr bool dv(int, int) { return false; }
    static constexpr int grp(int, int) { return 0; }
    static constexpr int TSTRIDE = 4, NXR = 1;  // activations 4t..4t+3
    static constexpr int xrun0(int) { return 0; }
    using Raw = RawBlock<NDW>;
    struct Chunk { uint32_t q[NT]; float d; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        return load_raw_block<NDW>(w, rowoff + u * (uint32_t)BB);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t) {
        Chunk c;
        const uint32_t sel = realign_sel(r.sh, 2);
#pragma unroll
        for (int t = 0; t < NT; t++) c.q[t] = __builtin_amdgcn_perm(r.d[t + 1], r.d[t], sel) ^ 0x80808080u;
        c.d = f16_bits_to_f32(r.d[0] >> (8u * r.sh));
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) {
        const uint32_t d = c.q[t], d8 = d >> 8;
        p[0] = and_or(d, 0x00FF00FFu, kMagic);   // weights 4t, 4t+2
        p[1] = and_or(d8, 0x00FF00FFu, kMagic);  // weights 4t+1, 4t+3
    }
    __device__ __forceinline__ static float gscale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float goffset(const Chunk&, int) { return 0.0f; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) { c.d = z ? 0.0f : c.d; }
};

// ------------------------------------------------------------------ GGUF Q6_K
// 210-byte super-block of 256 (gguf_codegen.rs:474-526): ql = bytes 0..128,
// qh = 128..192, sc = int8 192..208, d = f16 208..210.  Weight
// n*128 + 32j + 16s + i (n, s in {0,1}, j in 0..3, i in 0..15) has
//   low 4 bits  = nibble (j >> 1) of ql[64n + 32(j & 1) + 16s + i],
//   high 2 bits = bits 2j..2j+1 of qh[32n + 16s + i],
//   scale       = sc[8n + 2j + s].
// Chunk u is the quarter (n, s) = ((u >> 1) & 1, u & 1) of super-block u >> 2:
// 64 weights in four 16-weight groups j, read as three 16-byte runs
// A = ql[64n+16s..], B = ql[64n+32+16s..], H = qh[32n+16s..] plus the scales.
// Code dword t holds positions i = 4t..4t+3 of the three runs; its eight pairs
// are (j = 0..3) x (positions (4t, 4t+2), then (4t+1, 4t+3)); groups 2 and 3
// decode the nibble at bits 4..7 (x16).
struct EncQ6K {
    static constexpr uint32_t ENC = ENC_Q6_K;
    static constexpr int CW = 64, QK = 256, NT = 4, PPT = 8, NG = 4, BB = 210;
    static constexpr bool AFFINE = false;
    static constexpr int NRUN = 4, RUNLEN = 16, RUNSTRIDE = 32;  // activation runs of group j at 32j
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) {
        return 256u * (u >> 2) + 128u * ((u >> 1) & 1u) + 16u * (u & 1u);
    }
    static constexpr float coef(bool dv) { return dv ? 1536.0f : 1056.0f; }
    static constexpr int xoff(int t, int h, int e) { return 32 * (h & 3) + 4 * t + (h >> 2) + 2 * e; }
    static constexpr bool dv(int, int h) { return (h & 3) >= 2; }
    static constexpr int grp(int, int h) { return h & 3; }
    static constexpr int TSTRIDE = 4, NXR = 4;  // activations 32r+4t..32r+4t+3, run r = group r
    static constexpr int xrun0(int r) { return 32 * r; }
    struct Raw { uint32_t a[5], b[5], h[5], s[5]; uint32_t sh; };
    struct Chunk { uint32_t a[NT], b[NT], h[NT]; float dsc[NG]; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        const AlignedOffset a = aligned_offset(w, rowoff + (u >> 2) * (uint32_t)BB);
        const uint32_t n = (u >> 1) & 1u, s = u & 1u;
        const uint32_t sh = a.o & 3u;
        const uint32_t* al = reinterpret_cast<const uint32_t*>(a.abase + (a.o & ~3u));
        const uint32_t oa = (64u * n + 16u * s) >> 2;
        Raw r;
        load_dwords<5>(al + oa, r.a);
        load_dwords<5>(al + oa + 8u, r.b);
        load_dwords<5>(al + ((128u + 32u * n + 16u * s) >> 2), r.h);
        load_dwords<5>(al + (192u >> 2), r.s);  // sc[0..16) and d
        r.sh = sh;
        return r;
    }
    // The three code runs realigned: code dword t of each at a[t], b[t], h[t].
    __device__ __forceinline__ static void codes(const Raw& r, uint32_t (&a)[NT], uint32_t (&b)[NT],
                                                 uint32_t (&h)[NT]) {
        const uint32_t sel = realign_sel(r.sh, 0);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            a[t] = __builtin_amdgcn_perm(r.a[t + 1], r.a[t], sel);
            b[t] = __builtin_amdgcn_perm(r.b[t + 1], r.b[t], sel);
            h[t] = __builtin_amdgcn_perm(r.h[t + 1], r.h[t], sel);
        }
    }
    // The int8 scales of chunk u's groups j = 0..3 and the super-block's d.
    __device__ __forceinline__ static void scales(const Raw& r, uint32_t u, int32_t (&sc)[NG], float& d) {
        const uint32_t sel = realign_sel(r.sh, 0);
        const bool n = ((u >> 1) & 1u) != 0;
        const uint32_t bs = 8u * (u & 1u);
        // sc bytes 8n + s + {0, 2} (groups 0, 1) and 8n + 4 + s + {0, 2} (groups 2, 3)
        const uint32_t s01 = __builtin_amdgcn_perm(n ? r.s[3] : r.s[1], n ? r.s[2] : r.s[0], sel);
        const uint32_t s23 = __builtin_amdgcn_perm(n ? r.s[4] : r.s[2], n ? r.s[3] : r.s[1], sel);
        // d = bytes 16..17 of the run
        d = f16_bits_to_f32(r.sh ? (r.s[4] >> 16) : r.s[4]);
        sc[0] = (int32_t)__builtin_amdgcn_sbfe(s01, bs, 8u);
        sc[1] = (int32_t)__builtin_amdgcn_sbfe(s01, bs + 16u, 8u);
        sc[2] = (int32_t)__builtin_amdgcn_sbfe(s23, bs, 8u);
        sc[3] = (int32_t)__builtin_amdgcn_sbfe(s23, bs + 16u, 8u);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t u) {
        Chunk c;
        codes(r, c.a, c.b, c.h);
        int32_t sc[NG];
        float d;
        scales(r, u, sc, d);
#pragma unroll
        for (int g = 0; g < NG; g++) c.dsc[g] = (float)sc[g] * d;
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) {
        const uint32_t A = c.a[t], B = c.b[t], H = c.h[t];
        // positions (4t, 4t+2): bytes 0 and 2
        {
            const uint32_t h4 = H << 4, h2 = H << 2;
            p[0] = and_or(A, 0x000F000Fu, and_or(h4, 0x00300030u, kMagic));  // j=0: ql lo, qh bits 0-1
            p[1] = and_or(B, 0x000F000Fu, and_or(h2, 0x00300030u, kMagic));  // j=1: ql lo, qh bits 2-3
            p[2] = and_or(A, 0x00F000F0u, and_or(h4, 0x03000300u, kMagic));  // j=2: ql hi, qh bits 4-5 (x16)
            p[3] = and_or(B, 0x00F000F0u, and_or(h2, 0x03000300u, kMagic));  // j=3: ql hi, qh bits 6-7 (x16)
        }
        // positions (4t+1, 4t+3): bytes 1 and 3
        {
            const uint32_t A8 = A >> 8, B8 = B >> 8, h4 = H >> 4, h2 = H >> 6;
            p[4] = and_or(A8, 0x000F000Fu, and_or(h4, 0x00300030u, kMagic));
            p[5] = and_or(B8, 0x000F000Fu, and_or(h2, 0x00300030u, kMagic));
            p[6] = and_or(A8, 0x00F000F0u, and_or(h4, 0x03000300u, kMagic));
            p[7] = and_or(B8, 0x00F000F0u, and_or(h2, 0x03000300u, kMagic));
        }
    }
    __device__ __forceinline__ static float gscale(const Chunk& c, int g) { return c.dsc[g]; }
    __device__ __forceinline__ static float goffset(const Chunk&, int) { return 0.0f; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) {
#pragma unroll
        for (int g = 0; g < NG; g++) c.dsc[g] = z ? 0.0f : c.dsc[g];
    }
};

// ------------------------------------------------------------------ GGUF Q4_K
// 144-byte super-block of 256 (GGML block_q4_K; the reference's schema
// gguf_block.rs:183-316 "q4_k" and convention.rs:210,240: scale_min_f16 4 B,
// scales_and_mins_u6 12 B, quants_u4 128 B): d = f16 bytes 0..2, dmin = f16
// 2..4, packed 6-bit scales and mins 4..16, qs = 16..144.  Weights 64i + l and
// 64i + 32 + l (i < 4, l < 32) are the low and high nibbles of qs[32i + l], in
// sub-blocks 2i and 2i + 1: w = q·(d·sc_j) - dmin·m_j (q4k_scale_min).
// Chunk u is step i = u & 3 of super-block u >> 2: two scale groups, the low
// nibbles (weights 64i..64i+31) and the high nibbles (x16).  Code dword t =
// qs bytes 32i + 4t..4t+3; its pairs (4t, 4t+2), (32+4t, 34+4t) x16,
// (4t+1, 4t+3), (33+4t, 35+4t) x16.  Super-blocks are 4-byte aligned (the C
// ABI requires a 4-byte-aligned base; 144 = 36 dwords).
struct EncQ4K {
    static constexpr uint32_t ENC = ENC_Q4_K;
    static constexpr int CW = 64, QK = 256, NT = 8, PPT = 4, NG = 2, BB = 144;
    static constexpr bool AFFINE = true;
    static constexpr int NRUN = 2, RUNLEN = 32, RUNSTRIDE = 32;  // activation runs of group g at 32g
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 64u * u; }
    static constexpr float coef(bool) { return 1024.0f; }
    static constexpr int xoff(int t, int h, int e) { return 4 * t + (h >> 1) + 2 * e + 32 * (h & 1); }
    static constexpr bool dv(int, int h) { return (h & 1) != 0; }
    static constexpr int grp(int, int h) { return h & 1; }
    static constexpr int TSTRIDE = 4, NXR = 2;  // activations 4t..4t+3 and 32+4t..32+4t+3
    static constexpr int xrun0(int r) { return 32 * r; }
    // header dwords (d | dmin, scale bytes 0..11) and the step's 8 qs dwords
    struct Raw { uint32_t h[4]; uint32_t q[NT]; };
    struct Chunk { uint32_t q[NT]; float ds[NG], dm[NG]; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        const uint32_t* sb = reinterpret_cast<const uint32_t*>(w + (rowoff + (u >> 2) * (uint32_t)BB));
        Raw r;
        load_dwords<4>(sb, r.h);
        load_dwords<NT>(sb + 4u + 8u * (u & 3u), r.q);
        return r;
    }
    // The 6-bit scales and mins of sub-blocks 2i and 2i + 1 (i = step 0..3)
    // from the header dwords h[1..3] (device_common.hpp q4k_scale_min_pair).
    __device__ __forceinline__ static void scale_min(const uint32_t (&h)[4], uint32_t i, uint32_t (&sc)[NG],
                                                     uint32_t (&mn)[NG]) {
        q4k_scale_min_pair(h[1], h[2], h[3], i, sc, mn);
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t u) {
        Chunk c;
#pragma unroll
        for (int t = 0; t < NT; t++) c.q[t] = r.q[t];
        const float d = f16_bits_to_f32(r.h[0]), dmin = f16_bits_to_f32(r.h[0] >> 16);
        uint32_t sc[NG], mn[NG];
        scale_min(r.h, u & 3u, sc, mn);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            c.ds[g] = d * (float)sc[g];
            c.dm[g] = -(dmin * (float)mn[g]);
        }
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) { nibble_pairs(c.q[t], p); }
    __device__ __forceinline__ static float gscale(const Chunk& c, int g) { return c.ds[g]; }
    __device__ __forceinline__ static float goffset(const Chunk& c, int g) { return c.dm[g]; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) {
#pragma unroll
        for (int g = 0; g < NG; g++) {
            c.ds[g] = z ? 0.0f : c.ds[g];
            c.dm[g] = z ? 0.0f : c.dm[g];
        }
    }
};

// ------------------------------------------------------------------ GGUF Q5_K
// 176-byte super-block of 256 (GGML block_q5_K; the reference's schema
// gguf_block.rs:183-316 "q5_k", convention.rs:211,241: scale_min_f16 4 B,
// scales_and_mins_u6 12 B, high_bits 32 B, quants_u4 128 B): Q4_K's header,
// qh = bytes 16..48, qs = 48..176.  Weight 64i + 32h + l (l < 32) has the 5-bit
// code nibble h of qs[32i + l] | bit 2i + h of qh[l] << 4.  Chunks, scale groups
// and activation layout as Q4_K; code dword t pairs its qs dword with qh
// dword t (bytes 4t..4t+3, shifted down by 2i once per chunk), the fifth bit
// moved under the nibble: bit 4 for the low nibbles, bit 8 (x16) for the high.
struct EncQ5K {
    static constexpr uint32_t ENC = ENC_Q5_K;
    static constexpr int CW = 64, QK = 256, NT = 8, PPT = 4, NG = 2, BB = 176;
    static constexpr bool AFFINE = true;
    static constexpr int NRUN = 2, RUNLEN = 32, RUNSTRIDE = 32;
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 64u * u; }
    static constexpr float coef(bool) { return 1024.0f; }
    static constexpr int xoff(int t, int h, int e) { return EncQ4K::xoff(t, h, e); }
    static constexpr bool dv(int t, int h) { return EncQ4K::dv(t, h); }
    static constexpr int grp(int t, int h) { return EncQ4K::grp(t, h); }
    static constexpr int TSTRIDE = 4, NXR = 2;
    static constexpr int xrun0(int r) { return EncQ4K::xrun0(r); }
    struct Raw { uint32_t h[4]; uint32_t hb[NT]; uint32_t q[NT]; };
    struct Chunk { uint32_t q[NT], hb[NT]; float ds[NG], dm[NG]; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        const uint32_t* sb = reinterpret_cast<const uint32_t*>(w + (rowoff + (u >> 2) * (uint32_t)BB));
        Raw r;
        load_dwords<4>(sb, r.h);
        load_dwords<NT>(sb + 4u, r.hb);
        load_dwords<NT>(sb + 12u + 8u * (u & 3u), r.q);
        return r;
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t u) {
        Chunk c;
        const uint32_t i = u & 3u;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            c.q[t] = r.q[t];
            c.hb[t] = r.hb[t] >> (2u * i);  // bit 0 of each byte: low nibbles' fifth bit, bit 1: high
        }
        const float d = f16_bits_to_f32(r.h[0]), dmin = f16_bits_to_f32(r.h[0] >> 16);
        uint32_t sc[NG], mn[NG];
        q4k_scale_min_pair(r.h[1], r.h[2], r.h[3], i, sc, mn);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            c.ds[g] = d * (float)sc[g];
            c.dm[g] = -(dmin * (float)mn[g]);
        }
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) {
        const uint32_t Q = c.q[t], H = c.hb[t], Q8 = Q >> 8, H8 = H >> 8;
        p[0] = and_or(Q, 0x000F000Fu, and_or(H << 4, 0x00100010u, kMagic));   // (4t, 4t+2)
        p[1] = and_or(Q, 0x00F000F0u, and_or(H << 7, 0x01000100u, kMagic));   // (32+4t, 34+4t) x16
        p[2] = and_or(Q8, 0x000F000Fu, and_or(H8 << 4, 0x00100010u, kMagic)); // (4t+1, 4t+3)
        p[3] = and_or(Q8, 0x00F000F0u, and_or(H8 << 7, 0x01000100u, kMagic)); // (33+4t, 35+4t) x16
    }
    __device__ __forceinline__ static float gscale(const Chunk& c, int g) { return c.ds[g]; }
    __device__ __forceinline__ static float goffset(const Chunk& c, int g) { return c.dm[g]; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) {
#pragma unroll
        for (int g = 0; g < NG; g++) {
            c.ds[g] = z ? 0.0f : c.ds[g];
            c.dm[g] = z ? 0.0f : c.dm[g];
        }
    }
};

// ------------------------------------------------------------------ GGUF IQ4_XS
// 136-byte super-block of 256 (GGML block_iq4_xs; the reference's schema
// gguf_block.rs:183-316 "iq4_xs", convention.rs:221,267: scale_f16 2 B,
// scales_high_u16 2 B, scales_low_u8 4 B, nonlinear_quants_u4 128 B): d,
// scales_h, scales_l[4], qs = bytes 8..136.  Chunk u is sub-block ib = u & 7
// of super-block u >> 3: 32 weights laid out as a Q4_0 block (low nibble of
// qs[16ib + l] = weight l, high = 16 + l), each nibble an index into GGML's
// kvalues_iq4nl codebook, w = kv·(ls - 32)·d with the sub-block's 6-bit
// scale ls.  The codebook bytes kv + 128 (iq4nl_lookup) decode as Q8_0's
// codes: pairs (4t, 4t+2), (16+4t, 18+4t), (4t+1, 4t+3), (17+4t, 19+4t),
// all at mantissa bit 0.  Super-blocks are 4-byte aligned (136 = 34 dwords).
struct EncIQ4XS {
    static constexpr uint32_t ENC = ENC_IQ4_XS;
    static constexpr int CW = 32, QK = 256, NT = 4, PPT = 4, NG = 1, BB = 136;
    static constexpr bool AFFINE = false;
    static constexpr int NRUN = 1, RUNLEN = 32, RUNSTRIDE = 0;
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 32u * u; }
    static constexpr float coef(bool) { return 1152.0f; }
    static constexpr int xoff(int t, int h, int e) { return EncQ40::xoff(t, h, e); }
    static constexpr bool dv(int, int) { return false; }
    static constexpr int grp(int, int) { return 0; }
    static constexpr int TSTRIDE = 4, NXR = 2;
    static constexpr int xrun0(int r) { return EncQ40::xrun0(r); }
    struct Raw { uint32_t h[2]; uint32_t q[NT]; };  // d | scales_h, scales_l; the sub-block's codes
    struct Chunk { uint32_t q[NT]; float d; };
    __device__ __forceinline__ static Raw load(const uint8_t* w, uint32_t rowoff, uint32_t u) {
        const uint32_t* sb = reinterpret_cast<const uint32_t*>(w + (rowoff + (u >> 3) * (uint32_t)BB));
        Raw r;
        load_dwords<2>(sb, r.h);
        load_dwords<NT>(sb + 2u + 4u * (u & 7u), r.q);
        return r;
    }
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t u) {
        Chunk c;
#pragma unroll
        for (int t = 0; t < NT; t++) c.q[t] = r.q[t];
        const int ls = (int)iq4xs_scale(r.h[0] >> 16, r.h[1], u & 7u);
        c.d = f16_bits_to_f32(r.h[0]) * (float)(ls - 32);
        return c;
    }
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) {
        const uint32_t Q = c.q[t];
        const uint32_t L = iq4nl_lookup(Q & 0x0F0F0F0Fu), H = iq4nl_lookup((Q >> 4) & 0x0F0F0F0Fu);
        p[0] = and_or(L, 0x00FF00FFu, kMagic);       // (4t, 4t+2)
        p[1] = and_or(H, 0x00FF00FFu, kMagic);       // (16+4t, 18+4t)
        p[2] = and_or(L >> 8, 0x00FF00FFu, kMagic);  // (4t+1, 4t+3)
        p[3] = and_or(H >> 8, 0x00FF00FFu, kMagic);  // (17+4t, 19+4t)
    }
    __device__ __forceinline__ static float gscale(const Chunk& c, int) { return c.d; }
    __device__ __forceinline__ static float goffset(const Chunk&, int) { return 0.0f; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) { c.d = z ? 0.0f : c.d; }
};

// ------------------------------------------------------------------ MLX affine U4
// One chunk = 32 weights = 4 packed u32 words (weight i of a word = bits
// 4i..4i+3, fixture.rs:307-311) sharing one scale and bias (group size is a
// multiple of 32).  Word t's pairs: nibbles (0,4), (1,5) x16, (2,6), (3,7) x16.
struct EncMlxU4 {
    static constexpr uint32_t ENC = ENC_MLX_U4;
    static constexpr int CW = 32, NT = 4, PPT = 4, NG = 1;
    static constexpr bool AFFINE = true;
    static constexpr int NRUN = 1, RUNLEN = 32, RUNSTRIDE = 0;
    __device__ __forceinline__ static uint32_t xbase(uint32_t u) { return 32u * u; }
    static constexpr float coef(bool) { return 1024.0f; }
    static constexpr int xoff(int t, int h, int e) { return 8 * t + 2 * (h >> 1) + (h & 1) + 4 * e; }
    static constexpr bool dv(int, int h) { return (h & 1) != 0; }
    static constexpr int grp(int, int) { return 0; }
    static constexpr int TSTRIDE = 8, NXR = 2;  // activations 8t..8t+7
    static constexpr int xrun0(int r) { return 4 * r; }
    // packed words plus the scale/bias bit patterns (f32, or f16/bf16 in the
    // low half) and their dtype
    struct Raw { uint32_t w[4]; uint32_t s, b, kind; };
    struct Chunk { uint32_t w[4]; float s, b; };
    __device__ __forceinline__ static Chunk unpack(const Raw& r, uint32_t) {
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
    __device__ __forceinline__ static void pairs(const Chunk& c, int t, uint32_t (&p)[PPT]) {
        const uint32_t w = c.w[t], w8 = w >> 8;
        p[0] = and_or(w, 0x000F000Fu, kMagic);   // nibbles 0, 4
        p[1] = and_or(w, 0x00F000F0u, kMagic);   // nibbles 1, 5 (x16)
        p[2] = and_or(w8, 0x000F000Fu, kMagic);  // nibbles 2, 6
        p[3] = and_or(w8, 0x00F000F0u, kMagic);  // nibbles 3, 7 (x16)
    }
    __device__ __forceinline__ static float gscale(const Chunk& c, int) { return c.s; }
    __device__ __forceinline__ static float goffset(const Chunk& c, int) { return c.b; }
    __device__ __forceinline__ static void zero_if(Chunk& c, bool z) {
        c.s = z ? 0.0f : c.s;
        c.b = z ? 0.0f : c.b;
    }
};

// The run description of an encoding matches its xoff(): run and position of
// activation (h, e) of code dword 0, -1 if no run holds it.
template <class E>
constexpr int xrun_of(int h, int e) {
    for (int r = 0; r < E::NXR; r++)
        if (E::xoff(0, h, e) >= E::xrun0(r) && E::xoff(0, h, e) < E::xrun0(r) + 4) return r;
    return -1;
}
template <class E>
constexpr bool xruns_ok() {
    int seen[64] = {};
    for (int t = 0; t < E::NT; t++)
        for (int h = 0; h < E::PPT; h++)
            for (int e = 0; e < 2; e++) {
                if (E::xoff(t, h, e) != E::xoff(0, h, e) + E::TSTRIDE * t) return false;
                const int r = xrun_of<E>(h, e);
                if (r < 0) return false;
                seen[4 * r + E::xoff(0, h, e) - E::xrun0(r)]++;
            }
    for (int i = 0; i < 4 * E::NXR; i++)
        if (seen[i] != E::NT) return false;  // every run element is one activation of each dword
    return 4 * E::NXR == 2 * E::PPT;
}
static_assert(xruns_ok<EncQ40>() && xruns_ok<EncQ41>() && xruns_ok<EncQ80>() && xruns_ok<EncQ6K>() &&
                  xruns_ok<EncQ4K>() && xruns_ok<EncQ5K>() && xruns_ok<EncIQ4XS>() && xruns_ok<EncMlxU4>(),
              "activation runs disagree with xoff()");

}  // namespace dmx
