/*
 * CPU oracle for the quantized weight-matmul path — TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic the reference (goniz/dyninfer)
 * defines for GGUF Q4_0 / Q4_1 / Q8_0 / Q6_K (and Q4_K / Q5_K / IQ4_XS) blocks and MLX affine-U4 groups,
 * plus the reference's deterministic fixture helpers (LCG fill, packers).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the checker (or the timed CPU baseline).  The product path
 * (dyninfer_amd/) never calls into this library.
 *
 * Every function cites the reference file:line it follows.  How each function
 * is pinned (closed forms, known answers, the reference's own tests) is listed
 * in tests/test_oracle.py; nothing here is checked only against itself.
 *
 * Build: oracle/Makefile -> oracle/_build/liboracle.so (gcc -O3 -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

/* GGML type codes, crates/dyninfer-checkpoint-gguf/src/types.rs:10-43. */
enum { T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_XS = 23 };
/* Scale / activation dtypes used by this oracle. */
enum { D_F32 = 0, D_F16 = 1, D_BF16 = 2 };

/* ------------------------------------------------------------------ */
/* f16 / bf16 <-> f32.  The reference stores scales with half 2.x      */
/* `f16::from_f32` (round-to-nearest-even, IEEE inf/NaN/subnormals)     */
/* (crates/dyninfer-checkpoint-gguf/src/q4.rs:30-31) and widens with    */
/* `arith.extf` (gguf_codegen.rs:434), which is exact.                  */
/* ------------------------------------------------------------------ */
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1Fu) /* inf / NaN: keep payload, set quiet bit like a hardware widen */
        return bits_f32(sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0));
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (exp == 0xFFu) /* inf / NaN (quiet, keep top payload bits) */
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
    if (e <= 0) {
        /* subnormal or zero in f16: value = m * 2^-24 with m = round(|f| * 2^24) */
        if (e < -10) return sign; /* |f| < 2^-25 rounds to 0 (exact half goes to even 0) */
        uint32_t m = man | 0x800000u;
        int shift = 14 - e; /* in [14, 24] */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into exp/inf: correct */
    return (uint16_t)(sign | q);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

static inline float load_f16(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline void store_f16(uint8_t* p, float v) {
    uint16_t h = oracle_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xFF); p[1] = (uint8_t)(h >> 8);
}

/* ------------------------------------------------------------------ */
/* Deterministic LCG fill, crates/dyninfer-checkpoint-gguf/src/q4.rs:212-223
 * (identical to crates/dyninfer-checkpoint-safetensors/src/fixture.rs:92-103). */
void oracle_fill_f32(float* out, uint64_t n, uint32_t seed) {
    uint32_t x = seed;
    for (uint64_t i = 0; i < n; i++) {
        x = x * 1664525u + 1013904223u + (uint32_t)i;
        out[i] = (float)(x % 1000u) / 1000.0f - 0.5f;
    }
}

/* Rust `f32::round` = round half away from zero = C roundf.
 * Rust `as i32` / `as u8` from f32 saturate and map NaN to 0. */
static inline int32_t rust_f32_to_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)v;
}
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline float clampf_rust(float v, float lo, float hi) { /* f32::clamp: NaN stays NaN */
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* pack_q4_0, crates/dyninfer-checkpoint-gguf/src/q4.rs:16-44. */
int oracle_pack_q4_0(const float* w, uint64_t n, uint8_t* out) {
    if (n % 32) return -1;
    for (uint64_t b = 0; b < n / 32; b++) {
        const float* blk = w + b * 32;
        uint8_t* o = out + b * 18;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
        float scale = amax > 0.0f ? amax / 7.0f : 0.0f;
        store_f16(o, scale);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < 16; i++) {
            int32_t lo = clampi(rust_f32_to_i32(roundf(blk[i] * inv)), -8, 7) + 8;
            int32_t hi = clampi(rust_f32_to_i32(roundf(blk[i + 16] * inv)), -8, 7) + 8;
            o[2 + i] = (uint8_t)((uint8_t)lo | (uint8_t)(hi << 4));
        }
    }
    return 0;
}

/* pack_q4_1, crates/dyninfer-checkpoint-gguf/src/q4.rs:46-73. */
int oracle_pack_q4_1(const float* w, uint64_t n, uint8_t* out) {
    if (n % 32) return -1;
    for (uint64_t b = 0; b < n / 32; b++) {
        const float* blk = w + b * 32;
        uint8_t* o = out + b * 20;
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 32; i++) { mn = fminf(mn, blk[i]); mx = fmaxf(mx, blk[i]); }
        float scale = mx > mn ? (mx - mn) / 15.0f : 0.0f;
        store_f16(o, scale);
        store_f16(o + 2, mn);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int l = 0; l < 16; l++) {
            float lo = clampf_rust(roundf((blk[l] - mn) * inv), 0.0f, 15.0f);
            float hi = clampf_rust(roundf((blk[l + 16] - mn) * inv), 0.0f, 15.0f);
            uint8_t lq = (uint8_t)clampi(rust_f32_to_i32(lo), 0, 255);
            uint8_t hq = (uint8_t)clampi(rust_f32_to_i32(hi), 0, 255);
            o[4 + l] = (uint8_t)(lq | (uint8_t)(hq << 4));
        }
    }
    return 0;
}

/* pack_q8_0, crates/dyninfer-checkpoint-gguf/src/q4.rs:75-96. */
int oracle_pack_q8_0(const float* w, uint64_t n, uint8_t* out) {
    if (n % 32) return -1;
    for (uint64_t b = 0; b < n / 32; b++) {
        const float* blk = w + b * 32;
        uint8_t* o = out + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
        float scale = amax > 0.0f ? amax / 127.0f : 0.0f;
        store_f16(o, scale);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < 32; i++)
            o[2 + i] = (uint8_t)(int8_t)clampi(rust_f32_to_i32(roundf(blk[i] * inv)), -127, 127);
    }
    return 0;
}

/* quantize_affine_u4, crates/dyninfer-checkpoint-safetensors/src/fixture.rs:287-317.
 * Outputs f32 scales/biases exactly as the fixture does. */
int oracle_quantize_affine_u4(const float* v, uint64_t rows, uint64_t cols, uint32_t group,
                              uint32_t* packed, float* scales, float* biases) {
    if (group == 0 || cols % group || group % 8) return -1;
    uint64_t gi = 0, wi = 0;
    for (uint64_t r = 0; r < rows; r++) {
        for (uint64_t g0 = 0; g0 < cols; g0 += group) {
            const float* grp = v + r * cols + g0;
            float mn = INFINITY, mx = -INFINITY;
            for (uint32_t i = 0; i < group; i++) { mn = fminf(mn, grp[i]); mx = fmaxf(mx, grp[i]); }
            float scale = fmaxf((mx - mn) / 15.0f, 1.0e-7f);
            scales[gi] = scale;
            biases[gi] = mn;
            gi++;
            for (uint32_t i = 0; i < group; i += 8) {
                uint32_t word = 0;
                for (int lane = 0; lane < 8; lane++) {
                    float q = clampf_rust(roundf((grp[i + lane] - mn) / scale), 0.0f, 15.0f);
                    word |= (uint32_t)clampi(rust_f32_to_i32(q), 0, 15) << (lane * 4);
                }
                packed[wi++] = word;
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Dequantization: exactly the MLIR bodies the reference lowers to.     */
/* ------------------------------------------------------------------ */

/* Q4_0: gguf_codegen.rs:370-372 (quant_offset 2, no minimum) and the body at
 * :425-470: w = f32(nibble - 8) * f32(d) + 0.0 (the +0.0 bias maps -0 to +0).
 * Lane order (o,b,h,l) <- bytes (o,b,l,h): low nibble = lane l, high = 16+l (:452).
 * Rust dequant_q4_0 (q4.rs:100-128) is the same up to that sign of zero. */
static void dq_q4_0(const uint8_t* blk, float* out) {
    float d = load_f16(blk);
    for (int l = 0; l < 16; l++) {
        uint8_t byte = blk[2 + l];
        out[l] = (float)((int32_t)(byte & 0xF) - 8) * d + 0.0f;
        out[16 + l] = (float)((int32_t)(byte >> 4) - 8) * d + 0.0f;
    }
}

/* Q4_1: gguf_codegen.rs:373-375 (quant_offset 4, minimum = f16 word 1) and :425-470:
 * w = f32(q) * f32(d) + f32(m), one multiply then one add (the product is exact). */
static void dq_q4_1(const uint8_t* blk, float* out) {
    float d = load_f16(blk);
    float m = load_f16(blk + 2);
    for (int l = 0; l < 16; l++) {
        uint8_t byte = blk[4 + l];
        volatile float p0 = (float)(byte & 0xF) * d; /* keep mul and add separate */
        volatile float p1 = (float)(byte >> 4) * d;
        out[l] = p0 + m;
        out[16 + l] = p1 + m;
    }
}

/* Q8_0: gguf_codegen.rs:376, :382-410: w = f32(sext(int8)) * f32(d). */
static void dq_q8_0(const uint8_t* blk, float* out) {
    float d = load_f16(blk);
    for (int l = 0; l < 32; l++) out[l] = (float)(int8_t)blk[2 + l] * d;
}

/* Q6_K: gguf_codegen.rs:377, :474-526.  Index maps (:499-503):
 *   ql  i4 [2(n),2(p),32(s*16+l),2(h)]  <- bytes 0..128
 *   qh  i2 [2(n),32(s*16+l),2(h),2(p)]  <- bytes 128..192
 *   sc  i8 [2(n),2(h),2(p),2(s)]        <- bytes 192..208
 *   d   f16 word 104                     <- bytes 208..210
 * output index n*128 + h*64 + p*32 + s*16 + l, body (:507-521):
 *   q = low4 + 16*high2 - 32;  w = (f32(q) * f32(sc)) * f32(d). */
static void dq_q6_k(const uint8_t* blk, float* out) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    float d = load_f16(blk + 208);
    for (int n = 0; n < 2; n++)
        for (int h = 0; h < 2; h++)
            for (int p = 0; p < 2; p++)
                for (int s = 0; s < 2; s++)
                    for (int l = 0; l < 16; l++) {
                        int j = s * 16 + l;
                        uint8_t lb = ql[n * 64 + p * 32 + j];
                        int32_t low = h ? (lb >> 4) : (lb & 0xF);
                        int32_t high = (qh[n * 32 + j] >> (2 * (2 * h + p))) & 3;
                        int32_t q = low + 16 * high - 32;
                        volatile float local = (float)q * (float)sc[n * 8 + h * 4 + p * 2 + s];
                        out[n * 128 + h * 64 + p * 32 + j] = local * d;
                    }
}

/* Q4_K (GGUF type 12; the reference declares its schema only,
 * gguf_block.rs:183-316 SCHEMA_ONLY_DEFINITIONS "q4_k" 256 weights / 144 bytes
 * [scale_min_f16, scales_and_mins_u6, quants_u4]).  Restated from GGML's
 * published layout (block_q4_K, dequantize_row_q4_K): d = f16 bytes 0..2,
 * dmin = f16 bytes 2..4, scales[12] = bytes 4..16, qs[128] = bytes 16..144.
 * Sub-block j (32 weights) has a 6-bit scale sc_j and min m_j:
 *   j < 4:  sc = scales[j] & 63,  m = scales[j + 4] & 63
 *   j >= 4: sc = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4),
 *           m  = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4)
 * Weights 64i + l and 64i + 32 + l (i < 4, l < 32) are the low and high
 * nibbles of qs[32i + l], in sub-blocks 2i and 2i + 1:
 *   w = (d * sc_j) * q - (dmin * m_j)
 * d * sc and dmin * m are exact in f32 (11-bit x 6-bit significands), so is
 * their product with q (4 more bits): one rounding, at the subtraction. */
static void q4_k_scale_min(const uint8_t* sc12, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = sc12[j] & 63;
        *m = sc12[j + 4] & 63;
    } else {
        *sc = (sc12[j + 4] & 15) | ((sc12[j - 4] >> 6) << 4);
        *m = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
    }
}

static void dq_q4_k(const uint8_t* blk, float* out) {
    const float d = load_f16(blk), dmin = load_f16(blk + 2);
    const uint8_t* qs = blk + 16;
    for (int i = 0; i < 4; i++) {
        int sc0, m0, sc1, m1;
        q4_k_scale_min(blk + 4, 2 * i, &sc0, &m0);
        q4_k_scale_min(blk + 4, 2 * i + 1, &sc1, &m1);
        volatile float d0 = d * (float)sc0, o0 = dmin * (float)m0, d1 = d * (float)sc1, o1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            volatile float a = d0 * (float)(qs[32 * i + l] & 15), b = d1 * (float)(qs[32 * i + l] >> 4);
            out[64 * i + l] = a - o0;
            out[64 * i + 32 + l] = b - o1;
        }
    }
}

/* Q5_K (GGUF type 13; schema only in the reference, gguf_block.rs:183-316
 * "q5_k" 256 weights / 176 bytes [scale_min_f16 4, scales_and_mins_u6 12,
 * high_bits 32, quants_u4 128], convention.rs:211,241).  GGML block_q5_K:
 * d, dmin, scales[12] as Q4_K, qh[32] = bytes 16..48, qs[128] = 48..176.
 * Weights 64i + l and 64i + 32 + l take the low and high nibbles of
 * qs[32i + l] plus bit 2i and bit 2i + 1 of qh[l] as their fifth bit
 * (GGML dequantize_row_q5_K): q = nibble + 16*bit, 0..31, and
 *   w = (d * sc_j) * q - (dmin * m_j)
 * d * sc (17 bits) times q (5 bits) is exact in f32: one rounding, at the
 * subtraction. */
static void dq_q5_k(const uint8_t* blk, float* out) {
    const float d = load_f16(blk), dmin = load_f16(blk + 2);
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    for (int i = 0; i < 4; i++) {
        int sc0, m0, sc1, m1;
        q4_k_scale_min(blk + 4, 2 * i, &sc0, &m0);
        q4_k_scale_min(blk + 4, 2 * i + 1, &sc1, &m1);
        volatile float d0 = d * (float)sc0, o0 = dmin * (float)m0, d1 = d * (float)sc1, o1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            const int q0 = (qs[32 * i + l] & 15) | (((qh[l] >> (2 * i)) & 1) << 4);
            const int q1 = (qs[32 * i + l] >> 4) | (((qh[l] >> (2 * i + 1)) & 1) << 4);
            volatile float a = d0 * (float)q0, b = d1 * (float)q1;
            out[64 * i + l] = a - o0;
            out[64 * i + 32 + l] = b - o1;
        }
    }
}

/* IQ4_XS (GGUF type 23; schema only in the reference, gguf_block.rs:183-316
 * "iq4_xs" 256 weights / 136 bytes [scale_f16 2, scales_high_u16 2,
 * scales_low_u8 4, nonlinear_quants_u4 128], convention.rs:221,267).  GGML
 * block_iq4_xs: d = f16 bytes 0..2, scales_h = u16 bytes 2..4, scales_l[4] =
 * bytes 4..8, qs[128] = bytes 8..136.  Sub-block ib (32 weights) has the
 * 6-bit scale ls = nibble (ib & 1) of scales_l[ib / 2] | bits 2ib..2ib+1 of
 * scales_h << 4; its weights 32ib + j and 32ib + 16 + j (j < 16) are the low
 * and high nibbles of qs[16ib + j], looked up in GGML's kvalues_iq4nl
 * codebook (a constant of the format) and scaled (dequantize_row_iq4_xs):
 *   w = (d * (ls - 32)) * kvalues[q]
 * d * (ls - 32) (17 bits) times an entry (7 bits) is exact in f32. */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static void dq_iq4_xs(const uint8_t* blk, float* out) {
    const float d = load_f16(blk);
    const unsigned sh = (unsigned)blk[2] | ((unsigned)blk[3] << 8);
    const uint8_t* sl = blk + 4;
    const uint8_t* qs = blk + 8;
    for (int ib = 0; ib < 8; ib++) {
        const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 15) | (int)(((sh >> (2 * ib)) & 3) << 4);
        volatile float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            out[32 * ib + j] = dl * (float)kIq4nl[qs[16 * ib + j] & 15];
            out[32 * ib + 16 + j] = dl * (float)kIq4nl[qs[16 * ib + j] >> 4];
        }
    }
}

static int block_geom(int type, int* bw, int* bb) {
    switch (type) {
    case T_Q4_0: *bw = 32; *bb = 18; return 0;
    case T_Q4_1: *bw = 32; *bb = 20; return 0;
    case T_Q8_0: *bw = 32; *bb = 34; return 0;
    case T_Q4_K: *bw = 256; *bb = 144; return 0;
    case T_Q5_K: *bw = 256; *bb = 176; return 0;
    case T_IQ4_XS: *bw = 256; *bb = 136; return 0;
    case T_Q6_K: *bw = 256; *bb = 210; return 0;
    default: return -1;
    }
}

/* BlockLayout::{block_size, bytes_per_block}, gguf_codegen.rs:23-38. */
int oracle_gguf_block(int type, int* block_weights, int* block_bytes) {
    return block_geom(type, block_weights, block_bytes);
}

static void dq_block(int type, const uint8_t* blk, float* out) {
    switch (type) {
    case T_Q4_0: dq_q4_0(blk, out); break;
    case T_Q4_1: dq_q4_1(blk, out); break;
    case T_Q8_0: dq_q8_0(blk, out); break;
    case T_Q4_K: dq_q4_k(blk, out); break;
    case T_Q5_K: dq_q5_k(blk, out); break;
    case T_IQ4_XS: dq_iq4_xs(blk, out); break;
    case T_Q6_K: dq_q6_k(blk, out); break;
    }
}

/* emit_dequant, gguf_codegen.rs:350-380: row o, block b at byte (o*K/B + b)*bytes. */
int oracle_dequant_gguf(int type, const uint8_t* data, uint64_t rows, uint64_t cols, float* out) {
    int bw, bb;
    if (block_geom(type, &bw, &bb) || cols % (uint64_t)bw) return -1;
    uint64_t nblk = rows * (cols / (uint64_t)bw);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (int64_t)nblk; b++) dq_block(type, data + (uint64_t)b * bb, out + (uint64_t)b * bw);
    return 0;
}

static inline float load_scalar(const void* base, uint64_t i, int dtype) {
    const uint8_t* p = (const uint8_t*)base;
    switch (dtype) {
    case D_F32: { float f; memcpy(&f, p + 4 * i, 4); return f; }
    case D_F16: return oracle_f16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    default: return oracle_bf16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    }
}

/* MLX affine U4: mlx_affine.rs:557-626 (body :593-598) with the i4 bitcast of
 * packed u32 words (:517-537, lane i = bits 4i..4i+3, fixture.rs:307-311) and
 * exact extf of scales/biases (:481-497): w = f32(q) * s + b, mul then add. */
int oracle_dequant_mlx_u4(const uint32_t* packed, const void* scales, const void* biases, int sdtype,
                          uint64_t rows, uint64_t cols, uint32_t group, float* out) {
    if (group == 0 || cols % group || cols % 8) return -1;
    uint64_t groups = cols / group;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        for (uint64_t k = 0; k < cols; k++) {
            uint32_t word = packed[(uint64_t)r * (cols / 8) + k / 8];
            uint32_t q = (word >> (4 * (k % 8))) & 0xFu;
            float s = load_scalar(scales, (uint64_t)r * groups + k / group, sdtype);
            float b = load_scalar(biases, (uint64_t)r * groups + k / group, sdtype);
            volatile float prod = (float)q * s;
            out[(uint64_t)r * cols + k] = prod + b;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Contractions.                                                        */
/* ------------------------------------------------------------------ */

/* `linear`, crates/dyninfer-runtime/src/reference.rs:229-242: y[b,o] =
 * sum_k x[b,k] * w[o,k], sequential f32 accumulation from 0. */
void oracle_linear_f32(const float* x, const float* w, uint64_t batch, uint64_t in, uint64_t out, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < (int64_t)out; o++)
        for (uint64_t b = 0; b < batch; b++) {
            float acc = 0.0f;
            for (uint64_t k = 0; k < in; k++) acc += x[b * in + k] * w[(uint64_t)o * in + k];
            y[b * out + o] = acc;
        }
}

/* f64 contraction of an exactly dequantised W (the error-bound reference):
 * y64[b,o] = sum_k x[b,k] w[o,k] and absdot[b,o] = sum_k |x[b,k]| |w[o,k]|,
 * the normaliser of the 2e-3 tolerance. x and W are f32 (exact in f64). */
void oracle_linear_f64(const float* x, const float* w, uint64_t batch, uint64_t in, uint64_t out,
                       double* y64, double* absdot) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < (int64_t)out; o++)
        for (uint64_t b = 0; b < batch; b++) {
            double acc = 0.0, aacc = 0.0;
            const float* wr = w + (uint64_t)o * in;
            const float* xr = x + b * in;
            for (uint64_t k = 0; k < in; k++) {
                double p = (double)xr[k] * (double)wr[k];
                acc += p;
                aacc += fabs(p);
            }
            y64[b * out + o] = acc;
            absdot[b * out + o] = aacc;
        }
}

/* CPU baseline: the reference's CPU semantics (gguf_codegen.rs:268-314: a
 * dequantisation adjacent to an f32 contraction, weights never repacked) as
 * plain C.  Each row's blocks are dequantised into a small stack buffer and
 * dotted with x in f32.  `threads` OpenMP threads split the output rows. */
int oracle_qlinear_gguf_f32(int type, const uint8_t* data, const float* x, uint64_t batch,
                            uint64_t rows, uint64_t cols, float* y, int threads) {
    int bw, bb;
    if (block_geom(type, &bw, &bb) || cols % (uint64_t)bw) return -1;
    uint64_t nb = cols / (uint64_t)bw;
    if (batch > 64) return -1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t o = 0; o < (int64_t)rows; o++) {
        float wbuf[256];
        float acc[64];
        for (uint64_t b = 0; b < batch; b++) acc[b] = 0.0f;
        const uint8_t* row = data + (uint64_t)o * nb * bb;
        for (uint64_t blk = 0; blk < nb; blk++) {
            dq_block(type, row + blk * bb, wbuf);
            for (uint64_t b = 0; b < batch; b++) {
                const float* xr = x + b * cols + blk * bw;
                float a = acc[b];
                for (int i = 0; i < bw; i++) a += xr[i] * wbuf[i];
                acc[b] = a;
            }
        }
        for (uint64_t b = 0; b < batch; b++) y[b * rows + o] = acc[b];
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Seeded synthetic generators for the benchmark configurations.        */
/* splitmix64 + Box-Muller; defined here so tests are independent of    */
/* numpy's generator versions.                                          */
/* ------------------------------------------------------------------ */
static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline double u01(uint64_t* s) { return ((splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
static inline float normal(uint64_t* s) {
    double u1 = u01(s), u2 = u01(s);
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

void oracle_randn_f32(float* out, uint64_t n, uint64_t seed, float scale) {
    uint64_t s = seed * 0x2545F4914F6CDD1Dull + 1;
    for (uint64_t i = 0; i < n; i++) out[i] = normal(&s) * scale;
}

/* Synthetic GGUF tensor in the BASELINE distributions:
 *   Q4_0: d = f16(|N(0,1)|*0.01), codes uniform 0..15
 *   Q4_1: as Q4_0 plus m = f16(N(0,1)*0.01)
 *   Q8_0: d as Q4_0, int8 codes uniform -127..127
 *   Q6_K: d as Q4_0, 16 int8 sub-scales uniform -32..31, 6-bit codes uniform 0..63
 *   Q4_K: d as Q4_0, dmin = f16(|N(0,1)|*0.005), the 12 scale bytes and the codes uniform
 *   Q5_K: as Q4_K, the high bits uniform
 *   IQ4_XS: d = f16(|N(0,1)|*0.0005), the scale bits and the codes uniform */
int oracle_synth_gguf(int type, uint64_t rows, uint64_t cols, uint64_t seed, uint8_t* out) {
    int bw, bb;
    if (block_geom(type, &bw, &bb) || cols % (uint64_t)bw) return -1;
    uint64_t nblk = rows * (cols / (uint64_t)bw);
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 0x1234567ull;
    for (uint64_t b = 0; b < nblk; b++) {
        uint8_t* o = out + b * bb;
        float d = fabsf(normal(&s)) * 0.01f;
        switch (type) {
        case T_Q4_0:
            store_f16(o, d);
            for (int i = 0; i < 16; i++) o[2 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            break;
        case T_Q4_1:
            store_f16(o, d);
            store_f16(o + 2, normal(&s) * 0.01f);
            for (int i = 0; i < 16; i++) o[4 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            break;
        case T_Q8_0:
            store_f16(o, d);
            for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)((int)(splitmix64(&s) % 255u) - 127);
            break;
        case T_Q4_K:
            /* GGML-like: d, dmin small positive; 6-bit scales and mins uniform 0..63; codes 0..15 */
            store_f16(o, d);
            store_f16(o + 2, fabsf(normal(&s)) * 0.005f);
            for (int i = 0; i < 12; i++) o[4 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            for (int i = 0; i < 128; i++) o[16 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            break;
        case T_Q5_K:
            /* as Q4_K, with the high bits uniform */
            store_f16(o, d);
            store_f16(o + 2, fabsf(normal(&s)) * 0.005f);
            for (int i = 0; i < 172; i++) o[4 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            break;
        case T_IQ4_XS:
            /* d = f16(|N(0,1)|*0.0005) (codebook entries reach 127); scale bits and codes uniform */
            store_f16(o, fabsf(normal(&s)) * 0.0005f);
            for (int i = 0; i < 134; i++) o[2 + i] = (uint8_t)(splitmix64(&s) & 0xFF);
            break;
        case T_Q6_K: {
            /* draw each 6-bit code, then place its 4+2 bits per the layout */
            memset(o, 0, 208);
            for (int n = 0; n < 2; n++)
                for (int h = 0; h < 2; h++)
                    for (int p = 0; p < 2; p++)
                        for (int j = 0; j < 32; j++) {
                            uint32_t q = (uint32_t)(splitmix64(&s) & 63u);
                            o[n * 64 + p * 32 + j] |= (uint8_t)((q & 15u) << (4 * h));
                            o[128 + n * 32 + j] |= (uint8_t)((q >> 4) << (2 * (2 * h + p)));
                        }
            for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)(int8_t)((int)(splitmix64(&s) % 64u) - 32);
            store_f16(o + 208, d);
            break;
        }
        }
    }
    return 0;
}

/* Synthetic MLX affine-U4 tensor: codes uniform 0..15, scale = |N|*0.02 and
 * bias = N*0.01, both rounded to `sdtype` (bf16 or f16) or kept f32. */
int oracle_synth_mlx_u4(uint64_t rows, uint64_t cols, uint32_t group, int sdtype, uint64_t seed,
                        uint32_t* packed, void* scales, void* biases) {
    if (group == 0 || cols % group || cols % 8) return -1;
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 0x7654321ull;
    for (uint64_t i = 0; i < rows * cols / 8; i++) packed[i] = (uint32_t)splitmix64(&s);
    uint64_t ng = rows * (cols / group);
    for (uint64_t i = 0; i < ng; i++) {
        float sc = fabsf(normal(&s)) * 0.02f, bi = normal(&s) * 0.01f;
        if (sdtype == D_F32) {
            ((float*)scales)[i] = sc; ((float*)biases)[i] = bi;
        } else if (sdtype == D_F16) {
            ((uint16_t*)scales)[i] = oracle_f32_to_f16(sc); ((uint16_t*)biases)[i] = oracle_f32_to_f16(bi);
        } else {
            ((uint16_t*)scales)[i] = oracle_f32_to_bf16(sc); ((uint16_t*)biases)[i] = oracle_f32_to_bf16(bi);
        }
    }
    return 0;
}

int oracle_max_threads(void) { return omp_get_max_threads(); }
