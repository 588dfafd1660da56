// Prefill GEMM on gfx950 MFMA for the GGUF encodings Q4_0, Q4_1, Q8_0, Q6_K,
// Q4_K, Q5_K and IQ4_XS and for MLX affine U4: Y[M, N] = X[M, K] · Wᵀ with f32
// accumulation.  Kernel templates; gemm.hip plans a launch, and gemm_<enc>.hip
// instantiate the kernels of one encoding each (so they compile in parallel).
//
// Reference semantics: the same `emit_linear` contraction as decode
// (gguf_codegen.rs:268-314, dequantisations :412-472 Q4_0, :382-410 Q8_0,
// :474-526 Q6_K, q4.rs Q4_1; mlx_affine.rs:557-626 `emit_linear_u4`) with
// rows = the prefill window/chunk (512 when paged,
// parameter.rs:107-121, dense_decoder.rs:53-56).
//
// Data path.  W is read as GGUF blocks straight from HBM (no repack); X
// arrives staged by xprep.hip as f16 fragments of the MFMA operand, each row
// scaled by a power of two that rs[m] undoes.
//   * A workgroup of four waves owns a (32·TM) x (32·NB·4/S) tile of Y: each
//     wave a (32·TM) x (32·NB) tile (TM x NB blocks of
//     v_mfma_f32_32x32x16_f16), the four waves split over S K slices and 4/S
//     column subtiles.
//   * K advances in chunks of two weight blocks (64 k, four MFMA k steps)
//     through an LDS ring, every operand copied by global_load_lds (16 or 4
//     bytes per lane straight into LDS, counted by vmcnt, no registers held):
//     the activation fragments (1 KiB each, contiguous in HBM) once per slice,
//     and each wave's weight window (its rows' bytes of the chunk).
//   * Every lane decodes one block per N-block straight into A operands:
//     lane l takes weight row l % 32 of a 32-row block and block h = l / 32
//     of the chunk, so an MFMA k step pairs 8 k of the chunk's first block
//     (lanes 0..31) with 8 k of its second (lanes 32..63), and xprep stages
//     the activations in that order.  A code at mantissa bits 0.. under the
//     f16 exponent of 1024 is 1024 + c, one at bits 4.. under that of 64 is
//     64 + c (one v_and_or_b32 per two codes, both exact); a packed add removes
//     the offset (exact) and a packed multiply by the block scale rounds once
//     (Q4_0 RNE_f16((q-8)·d), Q8_0 RNE_f16(q·d)); Q4_1 a packed fma,
//     RNE_f16(q·d + m); Q6_K RNE_f16((q-32)·RNE_f16(d·sc)) (WinQ6K); MLX U4
//     RNE_f16(q·s + b) (WinMlx); Q4_K RNE_f16(q·RNE_f16(d·sc) - RNE_f16(dmin·m))
//     (WinQK); IQ4_XS RNE_f16(kv·RNE_f16(d·(ls - 32))) (WinIQ4XS).
//   * The weights are the MFMA's A operand and the activations its B, so each
//     lane ends with 4 consecutive output columns of one row per block.  K
//     slices meet in LDS after the loop, summed in slice order
//     (deterministic); then the rows are scaled by rs[m] and stored as whole
//     16-byte (f32) or 8-byte (bf16) column groups.
// Accuracy: |y - y_exact| <= 2^-10·Σ|w||x| (one f16 rounding of each weight and
// of each activation; Q6_K's weights round twice: (2^-10 + 2^-11)·Σ|w||x|;
// Q4_K's scale and offset round once each, adding 2^-11·Σ(|q·d·sc| + |dmin·m|)|x|) +
// f32 accumulation error, inside the 2e-3 normalised tolerance.  Weights must
// be finite in f16 (|w| <= 65504: |d| <= 8188 for Q4_0, |d·sc| <= 2047 for
// Q6_K).
#pragma once
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {
namespace gemm {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr uint32_t kLdsMax = 160u * 1024u;

struct GemmArgs {
    const uint8_t* w;
    const uint16_t* xh;
    const float* rs;
    void* y;
    uint64_t rowbytes;
    uint32_t M, N, K;
    uint32_t mt, nt;  // workgroup tiles along M and N
    uint32_t y_bf16;
    uint32_t mmajor;  // tile order: 1 = M-major (consecutive tiles share activation rows)
    const uint8_t* sc;  // MLX U4: scales and biases [N, K/group] of dtype sdtype
    const uint8_t* bi;
    uint32_t group, sdtype;
    uint32_t gmagic;  // group_magic(group)
};

// (a & m) | b as one v_and_or_b32 (mask in a scalar register: a VOP3 op takes
// no literal operand on gfx9).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
    return r;
}
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(h8, u32x4{a, b, c, d});
}


// ring_barrier<BASE + k·PER>() (ring_wait when !SYNC) for a wave-uniform k in
// [0, KMAX]: the copies of the k newest chunks, and BASE newer register
// loads, may stay in flight.
template <uint32_t PER, uint32_t KMAX, uint32_t BASE = 0, bool SYNC = true>
__device__ __forceinline__ void ring_barrier_k(uint32_t k) {
    if constexpr (KMAX == 0) {
        if constexpr (SYNC) ring_barrier<BASE>();
        else ring_wait<BASE>();
    } else {
        if (k >= KMAX) {
            if constexpr (SYNC) ring_barrier<BASE + KMAX * PER>();
            else ring_wait<BASE + KMAX * PER>();
        } else {
            ring_barrier_k<PER, KMAX - 1, BASE, SYNC>(k);
        }
    }
}

// Per-encoding block geometry and decode.  A lane reads kDw dwords from the
// 4-byte-aligned dword holding its block's first byte (sh = the block start's
// offset in that dword, 0 or 2); scale() takes the block's f16 scale(s) from
// them and step(t) decodes the MFMA operand of the chunk's k step t: 8 k of
// the block, as 4 packed f16 pairs.
template <uint32_t ENC>
struct Blk;

template <>
struct Blk<ENC_Q4_0> {
    // d (2 B) then 16 code bytes; byte j: k = j (low nibble), k = j + 16 (high).
    // Step t: code bytes 4t..4t+3 -> k = 4t+(0,2), 4t+(1,3), 16+4t+(0,2), 16+4t+(1,3).
    static constexpr uint32_t kBytes = 18, kDw = 5, kLayout = XFRAG_NIB;
    struct Scale {
        h2 d;
        uint32_t sel;
    };
    __device__ static Scale scale(const uint32_t* r, uint32_t sh) {
        return {as_h2(__builtin_amdgcn_perm(r[0], r[0], 0x01000100u + 0x01010101u * sh)),
                0x05040302u + 0x01010101u * sh};  // block bytes 2+4t..5+4t from dwords t, t+1
    }
    __device__ static h8 step(const uint32_t* r, const Scale& s, int t) {
        const h2 ol = {(_Float16)-1032.0f, (_Float16)-1032.0f}, oh = {(_Float16)-72.0f, (_Float16)-72.0f};
        const uint32_t ml = 0x64006400u, mh = 0x54005400u;
        auto lo = [&](uint32_t v) { return as_u((as_h2(and_or(v, 0x000F000Fu, ml)) + ol) * s.d); };
        auto hi = [&](uint32_t v) { return as_u((as_h2(and_or(v, 0x00F000F0u, mh)) + oh) * s.d); };
        const uint32_t q = __builtin_amdgcn_perm(r[t + 1], r[t], s.sel), q8 = q >> 8;
        return as_h8(lo(q), lo(q8), hi(q), hi(q8));
    }
};

template <>
struct Blk<ENC_Q4_1> {
    // d, m (2 B each) then 16 code bytes (4-byte-aligned blocks): w = q·d + m;
    // k order as Q4_0.
    static constexpr uint32_t kBytes = 20, kDw = 5, kLayout = XFRAG_NIB;
    struct Scale {
        h2 d, m;
    };
    __device__ static Scale scale(const uint32_t* r, uint32_t) {
        return {as_h2(__builtin_amdgcn_perm(r[0], r[0], 0x01000100u)),
                as_h2(__builtin_amdgcn_perm(r[0], r[0], 0x03020302u))};
    }
    __device__ static h8 step(const uint32_t* r, const Scale& s, int t) {
        const h2 ol = {(_Float16)-1024.0f, (_Float16)-1024.0f}, oh = {(_Float16)-64.0f, (_Float16)-64.0f};
        const uint32_t ml = 0x64006400u, mh = 0x54005400u;
        auto lo = [&](uint32_t v) {
            return as_u(__builtin_elementwise_fma(as_h2(and_or(v, 0x000F000Fu, ml)) + ol, s.d, s.m));
        };
        auto hi = [&](uint32_t v) {
            return as_u(__builtin_elementwise_fma(as_h2(and_or(v, 0x00F000F0u, mh)) + oh, s.d, s.m));
        };
        const uint32_t q = r[t + 1], q8 = q >> 8;
        return as_h8(lo(q), lo(q8), hi(q), hi(q8));
    }
};

template <>
struct Blk<ENC_Q8_0> {
    // d (2 B) then 32 int8 codes; step t: codes 8t..8t+7 in the order
    // (0,2) (1,3) (4,6) (5,7): a code c as (c ^ 0x80) under the exponent of 1024
    // is 1152 + c.
    static constexpr uint32_t kBytes = 34, kDw = 9, kLayout = XFRAG_BYTE;
    struct Scale {
        h2 d;
        uint32_t sel;
    };
    __device__ static Scale scale(const uint32_t* r, uint32_t sh) {
        return {as_h2(__builtin_amdgcn_perm(r[0], r[0], 0x01000100u + 0x01010101u * sh)),
                0x05040302u + 0x01010101u * sh};
    }
    __device__ static h8 step(const uint32_t* r, const Scale& s, int t) {
        const h2 o = {(_Float16)-1152.0f, (_Float16)-1152.0f};
        const uint32_t ml = 0x64006400u;
        auto p = [&](uint32_t v) { return as_u((as_h2(and_or(v, 0x00FF00FFu, ml)) + o) * s.d); };
        const uint32_t c0 = __builtin_amdgcn_perm(r[2 * t + 1], r[2 * t], s.sel) ^ 0x80808080u;
        const uint32_t c1 = __builtin_amdgcn_perm(r[2 * t + 2], r[2 * t + 1], s.sel) ^ 0x80808080u;
        return as_h8(p(c0), p(c0 >> 8), p(c1), p(c1 >> 8));
    }
};

// A wave's weight window: the bytes of its 32·NB weight rows for one 64-k
// chunk, copied into LDS by global_load_lds (16 or 4 bytes per lane, the
// lane's LDS slot at dst + 16·lane or 4·lane), then read and decoded by each
// lane: row 32j + l % 32 of N-block j (j < NB), block (or half-step) h = l / 32
// of the chunk.  A copy instruction whose lanes run past the window's pieces
// re-copies its last valid piece into the window's unread tail, so every
// instruction has the same lanes active and the ring's wait counts hold.
//
// GGUF blocks of 32 weights: a row's two blocks of the chunk are contiguous;
// they are copied from their 4-byte-aligned start as NP 16-byte pieces
// (consecutive lanes on consecutive pieces of a row), the last piece moved
// back so that no read passes the blocks' last dword.
template <uint32_t ENC, int NB>
struct WinBlocks {
    using B = Blk<ENC>;
    using Scale = typename B::Scale;
    static constexpr uint32_t kRows = 32u * NB;
    static constexpr uint32_t kSpanMax = (2u * B::kBytes + 2u + 3u) & ~3u;  // a row's two blocks, aligned
    static constexpr uint32_t NP = (kSpanMax + 15u) / 16u;                   // 16-byte pieces per row
    static constexpr uint32_t kCopies = (kRows * NP + 63u) / 64u;             // copy instructions per chunk
    static constexpr uint32_t kBytes = kCopies * 1024u;
    static constexpr uint32_t kDw = B::kDw;
    const uint8_t* src[kCopies];    // copy lane's piece for the slice's first chunk
    uint32_t off[NB][kDw], sh[NB];  // this lane's block dwords in the window, its block's start offset

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane, uint32_t c0) {
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) {
            uint32_t li = 64u * q + lane;
            li = li < kRows * NP ? li : kRows * NP - 1u;
            const uint32_t r = li / NP, p = li % NP;
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            const uintptr_t start = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes + (uintptr_t)B::kBytes * 2u * c0;
            const uintptr_t al = start & ~(uintptr_t)3;
            const uint32_t span = (uint32_t)(((start + 2u * B::kBytes + 3u) & ~(uintptr_t)3) - al);
            src[q] = reinterpret_cast<const uint8_t*>(al + (p + 1u < NP ? 16u * p : span - 16u));
        }
        // dword k of the lane's block (from its aligned start) at window offset
        // off[j][k]: span bytes past the first NP - 1 pieces sit in the last
        // piece, moved back by span - 16·NP
        const uint32_t h = lane >> 5;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t r = 32u * j + (lane & 31u);
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;
            const uintptr_t start = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes + (uintptr_t)B::kBytes * 2u * c0;
            const uint32_t s0 = (uint32_t)(start & 3u);
            const uint32_t span = (2u * B::kBytes + s0 + 3u) & ~3u;
            const uint32_t bstart = s0 + B::kBytes * h;
            sh[j] = bstart & 3u;
#pragma unroll
            for (uint32_t k = 0; k < kDw; k++) {
                const uint32_t o = (bstart & ~3u) + 4u * k;
                off[j][k] = r * NP * 16u + (o < 16u * (NP - 1u) ? o : o - span + 16u * NP);
            }
        }
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) dma16(src[q] + (size_t)c * 2u * B::kBytes, win + 1024u * q);
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
            for (uint32_t k = 0; k < kDw; k++) raw[j * kDw + k] = *reinterpret_cast<const uint32_t*>(win + off[j][k]);
    }
    __device__ Scale scale(uint32_t, int j, const uint32_t* r) const { return B::scale(r, sh[j]); }
    __device__ h8 step(const uint32_t* r, const Scale& s, int t) const { return B::step(r, s, t); }
};

// GGUF Q6_K (super-blocks of 256 weights, 210 bytes: ql[128], qh[64], int8
// scales[16], f16 d; gguf_codegen.rs:474-526).  Chunk g of a row covers
// quarter q = g % 4 of super-block g / 4: weights 128·(q/2) + 64·(q%2) + 0..63,
// lane half h the 32 of them with l = 0..31 at 128·(q/2) + 32·(2·(q%2) + h) + l,
// whose 6-bit codes are the (q%2) nibble of ql[64·(q/2) + 32h + l] under bits
// 2·(2·(q%2) + h) of qh[32·(q/2) + l], scaled by d·scales[8·(q/2) + 2·(2(q%2) + h)
// + l/16].  The window per row: ql[64·(q/2) .. +64) and qh[32·(q/2) .. +32) as
// six 16-byte pieces, then five dwords: the ql and qh dwords past those (a
// super-block starting 2 bytes into its dword), the two scale dwords the
// chunk's scales lie in, and the dword of d.  Every copy lies within the
// super-block's dwords.  The codes' pairs (l, l+2) decode with one
// v_and_or_b32 each for the nibble and one for the qh bits (moved under the
// nibble), so an MFMA k step takes l = 8t .. 8t+7 in the order of Q8_0.
template <int NB>
struct WinQ6K {
    static constexpr uint32_t kRows = 32u * NB;
    static constexpr uint32_t kX16 = 6, kX4 = 5;
    static constexpr uint32_t kQ16 = kRows * kX16 / 64u, kQ4 = (kRows * kX4 + 63u) / 64u, kCopies = kQ16 + kQ4;
    static constexpr uint32_t kPitch16 = 16u * kX16, kPitch4 = 4u * kX4;
    static constexpr uint32_t kOff4 = kRows * kPitch16;  // the dwords after every row's 16-byte pieces
    static constexpr uint32_t kBytes = kOff4 + 256u * kQ4;
    static constexpr uint32_t kDw = 20;  // ql 9, qh 9, scale dword, d dword
    static_assert(kRows * kX16 % 64u == 0, "16-byte pieces fill whole copy instructions");
    struct Scale {
        uint32_t sel, mN, magic, mH, sL;
        h2 off, ds0, ds1;
    };
    uintptr_t rb16[kQ16], rb4[kQ4];  // row of each copy lane (its first super-block)
    uint32_t p16[kQ16], p4[kQ4];     // piece of each copy lane
    uintptr_t row[NB];               // this lane's rows
    uint32_t c0, h, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
        h = lane >> 5;
        auto rowp = [&](uint32_t r) {
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            return (uintptr_t)a.w + (uintptr_t)n * a.rowbytes;
        };
#pragma unroll
        for (uint32_t q = 0; q < kQ16; q++) {
            const uint32_t li = 64u * q + lane;
            rb16[q] = rowp(li / kX16);
            p16[q] = li % kX16;
        }
#pragma unroll
        for (uint32_t q = 0; q < kQ4; q++) {
            uint32_t li = 64u * q + lane;
            li = li < kRows * kX4 ? li : kRows * kX4 - 1u;
            rb4[q] = rowp(li / kX4);
            p4[q] = li % kX4;
        }
#pragma unroll
        for (int j = 0; j < NB; j++) row[j] = rowp(32u * j + (lane & 31u));
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, hn = (g >> 1) & 1u, ph = g & 1u;
#pragma unroll
        for (uint32_t q = 0; q < kQ16; q++) {
            const uintptr_t al = (rb16[q] + (uintptr_t)sb * 210u) & ~(uintptr_t)3;
            const uint32_t p = p16[q];
            const uint32_t o = p < 4u ? 64u * hn + 16u * p : 128u + 32u * hn + 16u * (p - 4u);
            dma16(reinterpret_cast<const void*>(al + o), win + 1024u * q);
        }
#pragma unroll
        for (uint32_t q = 0; q < kQ4; q++) {
            const uintptr_t al = (rb4[q] + (uintptr_t)sb * 210u) & ~(uintptr_t)3;
            const uint32_t p = p4[q];
            const uint32_t o = p == 0u ? 64u * hn + 64u
                             : p == 1u ? 160u + 32u * hn
                             : p == 2u ? 192u + 8u * hn + 4u * ph
                             : p == 3u ? 196u + 8u * hn + 4u * ph
                                       : 208u;
            dma4(reinterpret_cast<const void*>(al + o), win + kOff4 + 256u * q);
        }
    }
    __device__ uint32_t shift_of(uint32_t c, int j) const { return (uint32_t)((row[j] + (uintptr_t)((c0 + c) >> 2) * 210u) & 3u); }
    __device__ void read(uint32_t c, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t r = 32u * j + (lane & 31u);
            const uint8_t* w16 = win + r * kPitch16;
            const uint8_t* w4 = win + kOff4 + r * kPitch4;
            uint32_t* o = raw + j * kDw;
#pragma unroll
            for (uint32_t k = 0; k < 9; k++) {
                const uint32_t rel = 32u * h + 4u * k;  // ql dword k of the lane's 32 codes
                o[k] = *reinterpret_cast<const uint32_t*>(rel < 64u ? w16 + rel : w4);
                o[9 + k] = *reinterpret_cast<const uint32_t*>(k < 8u ? w16 + 64u + 4u * k : w4 + 4u);  // qh
            }
            o[18] = *reinterpret_cast<const uint32_t*>(w4 + (2u * h + shift_of(c, j) < 4u ? 8u : 12u));
            o[19] = *reinterpret_cast<const uint32_t*>(w4 + 16u);
        }
    }
    __device__ Scale scale(uint32_t c, int j, const uint32_t* r) const {
        const uint32_t sh = shift_of(c, j), ph = (c0 + c) & 1u;
        const float d = f16_bits_to_f32(r[19] >> (8u * sh));
        const uint32_t bp = 8u * ((2u * h + sh) & 3u);
        const float s0 = (float)(int8_t)(r[18] >> bp), s1 = (float)(int8_t)(r[18] >> (bp + 8u));
        const _Float16 d0 = (_Float16)(d * s0), d1 = (_Float16)(d * s1);  // exact f32 product, one rounding
        Scale s;
        s.sel = 0x03020100u + 0x01010101u * sh;
        s.mN = ph ? 0x00F000F0u : 0x000F000Fu;
        s.magic = ph ? 0x54005400u : 0x64006400u;  // code bits under the exponent of 64 / 1024
        s.mH = ph ? 0x03000300u : 0x00300030u;
        s.sL = 4u - 2u * h;
        const _Float16 o = ph ? (_Float16)-96.0f : (_Float16)-1056.0f;
        s.off = h2{o, o};
        s.ds0 = h2{d0, d0};
        s.ds1 = h2{d1, d1};
        return s;
    }
    __device__ h8 step(const uint32_t* r, const Scale& s, int t) const {
        const uint32_t c = __builtin_amdgcn_perm(r[2 * t + 1], r[2 * t], s.sel);
        const uint32_t c2 = __builtin_amdgcn_perm(r[2 * t + 2], r[2 * t + 1], s.sel);
        const uint32_t e = __builtin_amdgcn_perm(r[9 + 2 * t + 1], r[9 + 2 * t], s.sel);
        const uint32_t e2 = __builtin_amdgcn_perm(r[9 + 2 * t + 2], r[9 + 2 * t + 1], s.sel);
        const h2 ds = t < 2 ? s.ds0 : s.ds1;
        auto f = [&](uint32_t cv, uint32_t ev) {
            return as_u((as_h2(and_or(ev << s.sL, s.mH, and_or(cv, s.mN, s.magic))) + s.off) * ds);
        };
        return as_h8(f(c, e), f(c >> 8, e >> 8), f(c2, e2), f(c2 >> 8, e2 >> 8));
    }
};

// MLX affine U4 (mlx_affine.rs:557-626; packed u32 [N, K/8], nibble i of a
// word = k offset i, fixture.rs:307-311): a row's chunk is 8 words (32 bytes,
// 4-byte-aligned rows of K/2 bytes) copied as two 16-byte pieces, plus, per
// row, the dwords holding the scale and the bias of the chunk's two 32-k
// halves (the same group unless group = 32).  Lane l decodes row 32j + l % 32
// of each N-block j, words 4h .. 4h+3 (h = l / 32): k step t takes word
// 4h + t, nibbles (0,4) (1,5) (2,6) (3,7) as packed pairs (XFRAG_WORD), code q
// exact in f16 and w = RNE_f16(q·s + b) by one packed fma, s and b taken to
// f16 first (bf16 and f16 values exact in f16's normal range; f32 rounded).
template <int NB>
struct WinMlx {
    static constexpr uint32_t kRows = 32u * NB;
    static constexpr uint32_t kPieces = kRows * 2u / 64u;        // 16-byte copies of the code words
    static constexpr uint32_t kAuxQ = (kRows + 63u) / 64u;       // 4-byte copies per scale or bias array
    static constexpr uint32_t kCopies = kPieces + 4u * kAuxQ;
    static constexpr uint32_t kAuxOff = kPieces * 1024u;         // the aux dwords after every row's pieces
    static constexpr uint32_t kAuxPitch = 256u * kAuxQ;          // bytes per aux array: s0, s1, b0, b1
    static constexpr uint32_t kBytes = kAuxOff + 4u * kAuxPitch;
    static constexpr uint32_t kDw = 6;  // 4 code words, scale dword, bias dword
    struct Scale {
        h2 s, b;
    };
    const uint8_t* src[kPieces];             // copy lane's piece of the slice's first chunk
    uintptr_t srow[kAuxQ], brow[kAuxQ];      // copy lane's row of scales and biases
    uint32_t ssh[NB], bsh[NB];               // this lane's rows' scale and bias row starts mod 4 (per N-block j)
    uint32_t c0, es, gmagic, sdtype, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
        gmagic = a.gmagic;
        sdtype = a.sdtype;
        es = a.sdtype == DT_F32 ? 4u : 2u;
        const uint32_t rbytes = a.K / 2u, sbytes = a.K / a.group * es;
        auto rowc = [&](uint32_t r) { return n0 + r < a.N ? n0 + r : a.N - 1u; };  // past N: re-read the last row
#pragma unroll
        for (uint32_t q = 0; q < kPieces; q++) {
            const uint32_t li = 64u * q + lane;
            src[q] = a.w + (size_t)rowc(li / 2u) * rbytes + 32u * c0 + 16u * (li % 2u);
        }
#pragma unroll
        for (uint32_t q = 0; q < kAuxQ; q++) {
            const uint32_t r = 64u * q + lane < kRows ? 64u * q + lane : kRows - 1u;
            srow[q] = (uintptr_t)a.sc + (uintptr_t)rowc(r) * sbytes;
            brow[q] = (uintptr_t)a.bi + (uintptr_t)rowc(r) * sbytes;
        }
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uintptr_t o = (uintptr_t)rowc(32u * j + (lane & 31u)) * sbytes;
            ssh[j] = (uint32_t)(((uintptr_t)a.sc + o) & 3u);
            bsh[j] = (uint32_t)(((uintptr_t)a.bi + o) & 3u);
        }
    }
    // byte offset in a scale row of the group of the chunk's 32-k half hh
    __device__ uint32_t goff(uint32_t c, uint32_t hh) const { return div_magic(64u * (c0 + c) + 32u * hh, gmagic) * es; }
    __device__ void issue(uint32_t c, uint8_t* win) const {
#pragma unroll
        for (uint32_t q = 0; q < kPieces; q++) dma16(src[q] + (size_t)c * 32u, win + 1024u * q);
#pragma unroll
        for (uint32_t hh = 0; hh < 2; hh++) {
            const uint32_t o = goff(c, hh);
#pragma unroll
            for (uint32_t q = 0; q < kAuxQ; q++) {
                dma4(reinterpret_cast<const void*>((srow[q] + o) & ~(uintptr_t)3), win + kAuxOff + kAuxPitch * hh + 256u * q);
                dma4(reinterpret_cast<const void*>((brow[q] + o) & ~(uintptr_t)3),
                     win + kAuxOff + kAuxPitch * (2u + hh) + 256u * q);
            }
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
        const uint32_t h = lane >> 5;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t r = 32u * j + (lane & 31u);
            const u32x4 q = *reinterpret_cast<const u32x4*>(win + 32u * r + 16u * h);
            uint32_t* o = raw + j * kDw;
            o[0] = q.x;
            o[1] = q.y;
            o[2] = q.z;
            o[3] = q.w;
            o[4] = *reinterpret_cast<const uint32_t*>(win + kAuxOff + kAuxPitch * h + 4u * r);
            o[5] = *reinterpret_cast<const uint32_t*>(win + kAuxOff + kAuxPitch * (2u + h) + 4u * r);
        }
    }
    __device__ Scale scale(uint32_t c, int j, const uint32_t* r) const {
        // 16-bit values may sit 2 bytes into their dword
        const uint32_t go = goff(c, lane >> 5);
        auto f16of = [&](uint32_t bits, uint32_t base_mod4) -> _Float16 {
            if (sdtype == DT_F32) return (_Float16)__uint_as_float(bits);
            const uint32_t v = (bits >> (8u * ((base_mod4 + go) & 3u))) & 0xFFFFu;
            if (sdtype == DT_F16) return __builtin_bit_cast(_Float16, (uint16_t)v);
            return (_Float16)__uint_as_float(v << 16);  // bf16
        };
        const _Float16 sv = f16of(r[4], ssh[j]), bv = f16of(r[5], bsh[j]);
        return {h2{sv, sv}, h2{bv, bv}};
    }
    __device__ h8 step(const uint32_t* r, const Scale& s, int t) const {
        const h2 ol = {(_Float16)-1024.0f, (_Float16)-1024.0f}, oh = {(_Float16)-64.0f, (_Float16)-64.0f};
        const uint32_t ml = 0x64006400u, mh = 0x54005400u;
        auto lo = [&](uint32_t v) { return as_u(__builtin_elementwise_fma(as_h2(and_or(v, 0x000F000Fu, ml)) + ol, s.s, s.b)); };
        auto hi = [&](uint32_t v) { return as_u(__builtin_elementwise_fma(as_h2(and_or(v, 0x00F000F0u, mh)) + oh, s.s, s.b)); };
        const uint32_t w = r[t], w8 = w >> 8;
        return as_h8(lo(w), hi(w), lo(w8), hi(w8));
    }
};

// GGUF Q4_K (GGML block_q4_K, 144-byte super-blocks of 256 weights; the
// reference's schema gguf_block.rs:183-316): chunk g of a row is step
// i = g % 4 of super-block g / 4, weights 64i + 0..63: lane half h decodes
// nibble h of qs[32i + l], l = 0..31 (weight 64i + 32h + l, sub-block
// 2i + h), so an MFMA k step takes l = 8t .. 8t+7 in the order of Q8_0.  The
// window per row: the super-block's 16-byte header (d, dmin, the 12 scale
// bytes) and the step's 32 code bytes, three 16-byte pieces (super-blocks
// are 4-byte aligned: 144 = 36 dwords).  w = RNE_f16(q·RNE_f16(d·sc) -
// RNE_f16(dmin·m)) by one packed fma (d·sc and dmin·m exact in f32).
// Q5_K (block_q5_K, 176 bytes): the window adds qh (bytes 16..48, two more
// pieces, kept before the codes); the fifth bit of weight 64i + 32h + l is bit
// 2i + h of qh[l], moved under the nibble.
template <bool Q5, int NB>
struct WinQK {
    static constexpr uint32_t kRows = 32u * NB;
    static constexpr uint32_t NP = Q5 ? 5u : 3u, kCopies = (kRows * NP + 63u) / 64u;
    static constexpr uint32_t kPitch = 16u * NP;
    static constexpr uint32_t kBytes = kCopies * 1024u;
    static constexpr uint32_t QS = Q5 ? 12u : 4u;          // raw dword of the codes
    static constexpr uint32_t SB = Q5 ? 176u : 144u;       // super-block bytes
    static constexpr uint32_t kDw = QS + 8u;               // d|dmin, three scale dwords, [8 qh dwords,] 8 code dwords
    struct Scale {
        h2 ds, ndm, off;
        uint32_t mask, magic, hsh, sl, mh;
    };
    uintptr_t rb[kCopies];  // row of each copy lane
    uint32_t pp[kCopies];   // piece of each copy lane
    uint32_t c0, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) {
            uint32_t li = 64u * q + lane;
            li = li < kRows * NP ? li : kRows * NP - 1u;
            const uint32_t r = li / NP;
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            rb[q] = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes;
            pp[q] = li % NP;
        }
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, i = g & 3u;
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) {
            const uint32_t p = pp[q];
            // pieces: header, [qh, qh,] the step's two code pieces
            const uint32_t o = p == 0u ? 0u : p + 2u < NP ? 16u * p : 16u * (QS / 4u) + 32u * i + 16u * (p + 2u - NP);
            dma16(reinterpret_cast<const void*>(rb[q] + (uintptr_t)sb * SB + o), win + 1024u * q);
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint8_t* w = win + (32u * j + (lane & 31u)) * kPitch;
            uint32_t* o = raw + j * kDw;
#pragma unroll
            for (uint32_t v = 0; v < NP; v++) {
                const u32x4 x = *reinterpret_cast<const u32x4*>(w + 16u * v);
                o[4 * v] = x.x;
                o[4 * v + 1] = x.y;
                o[4 * v + 2] = x.z;
                o[4 * v + 3] = x.w;
            }
        }
    }
    __device__ Scale scale(uint32_t c, int, const uint32_t* r) const {
        const uint32_t h = lane >> 5;
        uint32_t sc[2], mn[2];
        q4k_scale_min_pair(r[1], r[2], r[3], (c0 + c) & 3u, sc, mn);
        const float d = f16_bits_to_f32(r[0]), dmin = f16_bits_to_f32(r[0] >> 16);
        const _Float16 ds = (_Float16)(d * (float)(h ? sc[1] : sc[0]));      // exact f32 product, one rounding
        const _Float16 dm = (_Float16)(-(dmin * (float)(h ? mn[1] : mn[0])));
        const _Float16 o = h ? (_Float16)-64.0f : (_Float16)-1024.0f;
        Scale s;
        s.ds = h2{ds, ds};
        s.ndm = h2{dm, dm};
        s.off = h2{o, o};
        s.mask = h ? 0x00F000F0u : 0x000F000Fu;
        s.magic = h ? 0x54005400u : 0x64006400u;  // code bits under the exponent of 64 / 1024
        s.hsh = 2u * ((c0 + c) & 3u) + h;          // Q5_K: the qh bit of this half-step
        s.sl = h ? 8u : 4u;                        // ... moved to bit 8 (x16) or 4
        s.mh = h ? 0x01000100u : 0x00100010u;
        return s;
    }
    __device__ h8 step(const uint32_t* r, const Scale& s, int t) const {
        auto f = [&](uint32_t v, uint32_t e) {
            uint32_t m = s.magic;
            if constexpr (Q5) m = and_or(e << s.sl, s.mh, m);
            return as_u(__builtin_elementwise_fma(as_h2(and_or(v, s.mask, m)) + s.off, s.ds, s.ndm));
        };
        const uint32_t c = r[QS + 2 * t], c2 = r[QS + 1 + 2 * t];
        uint32_t e = 0, e2 = 0;
        if constexpr (Q5) {
            e = r[4 + 2 * t] >> s.hsh;
            e2 = r[5 + 2 * t] >> s.hsh;
        }
        return as_h8(f(c, e), f(c >> 8, e >> 8), f(c2, e2), f(c2 >> 8, e2 >> 8));
    }
};



// GGUF IQ4_XS (GGML block_iq4_xs, 136-byte super-blocks of 256 weights; the
// reference's schema gguf_block.rs:183-316): chunk g of a row covers
// sub-blocks 2i and 2i + 1 (i = g % 4) of super-block g / 4; lane half h
// decodes sub-block 2i + h, laid out as a Q4_0 block (XFRAG_NIB order), each
// nibble looked up in the codebook (iq4nl_lookup) and decoded as Q8_0's codes:
// w = RNE_f16(kv·RNE_f16(d·(ls - 32))).  The window per row: the 16 bytes
// from the super-block's start (d, scales_h, scales_l) and the chunk's 32
// code bytes, three 16-byte pieces within the super-block.
template <int NB>
struct WinIQ4XS {
    static constexpr uint32_t kRows = 32u * NB;
    static constexpr uint32_t NP = 3, kCopies = (kRows * NP + 63u) / 64u;
    static constexpr uint32_t kPitch = 16u * NP;
    static constexpr uint32_t kBytes = kCopies * 1024u;
    static constexpr uint32_t kDw = 12;  // d|scales_h, scales_l, two unused, 8 code dwords
    struct Scale {
        h2 ds;
        uint32_t h;
    };
    uintptr_t rb[kCopies];
    uint32_t pp[kCopies];
    uint32_t c0, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) {
            uint32_t li = 64u * q + lane;
            li = li < kRows * NP ? li : kRows * NP - 1u;
            const uint32_t r = li / NP;
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            rb[q] = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes;
            pp[q] = li % NP;
        }
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, i = g & 3u;
#pragma unroll
        for (uint32_t q = 0; q < kCopies; q++) {
            const uint32_t o = pp[q] == 0u ? 0u : 8u + 32u * i + 16u * (pp[q] - 1u);
            dma16(reinterpret_cast<const void*>(rb[q] + (uintptr_t)sb * 136u + o), win + 1024u * q);
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint8_t* w = win + (32u * j + (lane & 31u)) * kPitch;
            uint32_t* o = raw + j * kDw;
#pragma unroll
            for (uint32_t v = 0; v < NP; v++) {
                const u32x4 x = *reinterpret_cast<const u32x4*>(w + 16u * v);
                o[4 * v] = x.x;
                o[4 * v + 1] = x.y;
                o[4 * v + 2] = x.z;
                o[4 * v + 3] = x.w;
            }
        }
    }
    __device__ Scale scale(uint32_t c, int, const uint32_t* r) const {
        const uint32_t h = lane >> 5, ib = 2u * ((c0 + c) & 3u) + h;
        const float dl = f16_bits_to_f32(r[0]) * (float)((int)iq4xs_scale(r[0] >> 16, r[1], ib) - 32);  // exact
        const _Float16 ds = (_Float16)dl;
        return {h2{ds, ds}, h};
    }
    __device__ h8 step(const uint32_t* r, const Scale& s, int t) const {
        const h2 o = {(_Float16)-1152.0f, (_Float16)-1152.0f};
        auto f = [&](uint32_t v) { return as_u((as_h2(and_or(v, 0x00FF00FFu, 0x64006400u)) + o) * s.ds); };
        const uint32_t q = r[4u + 4u * s.h + (uint32_t)t];
        const uint32_t L = iq4nl_lookup(q & 0x0F0F0F0Fu), H = iq4nl_lookup((q >> 4) & 0x0F0F0F0Fu);
        return as_h8(f(L), f(L >> 8), f(H), f(H >> 8));
    }
};

template <uint32_t ENC, int NB>
struct WinOf {
    using type = WinBlocks<ENC, NB>;
};
template <int NB>
struct WinOf<ENC_IQ4_XS, NB> {
    using type = WinIQ4XS<NB>;
};
template <int NB>
struct WinOf<ENC_Q4_K, NB> {
    using type = WinQK<false, NB>;
};
template <int NB>
struct WinOf<ENC_Q5_K, NB> {
    using type = WinQK<true, NB>;
};
template <int NB>
struct WinOf<ENC_MLX_U4, NB> {
    using type = WinMlx<NB>;
};
template <int NB>
struct WinOf<ENC_Q6_K, NB> {
    using type = WinQ6K<NB>;
};

// LDS geometry of one kernel configuration: a wave multiplies TM activation
// row blocks by NB weight row blocks (32 rows each), the four waves of a
// workgroup split into S K slices x WN = 4/S column subtiles.
template <uint32_t ENC, int TM, int NB, int S>
struct Geo {
    using W = typename WinOf<ENC, NB>::type;
    static constexpr uint32_t WN = kWaves / S;
    static constexpr uint32_t kCols = 32u * NB;                             // a wave's output columns
    static constexpr uint32_t kXBytes = (uint32_t)S * 4u * TM * 1024u;       // a chunk's activation fragments
    static constexpr uint32_t kSlot = kXBytes + kWaves * W::kBytes;         // one ring slot
    static constexpr uint32_t kRs = 32u * TM * 4u;                          // the tile's row factors
    static constexpr uint32_t kEpiPitch = kCols + 4u;                       // floats per output row in LDS
    static constexpr uint32_t kEpi = (uint32_t)kWaves * 32u * TM * kEpiPitch * 4u;  // every wave's whole tile
    static constexpr uint32_t kRoom = kLdsMax - kRs;
    static constexpr uint32_t kDmaX = 4u * TM / WN;     // activation copies per wave per chunk
    static constexpr uint32_t kDma = kDmaX + W::kCopies;  // all copies per wave per chunk
    // Two ring slots: one chunk of copies ahead.  Deeper rings (3, 4) measured
    // 6-8% slower on M512/M2048 shapes: the prologue then requests most of a
    // short K slice at once, and chunk 0 lands behind the others.
    static constexpr uint32_t R = 2u;
    static constexpr uint32_t kRing = R * kSlot > kEpi ? R * kSlot : kEpi;  // the epilogue reuses the ring
    static constexpr uint32_t kLds = kRing + kRs;
    static constexpr bool kFits = R * kSlot <= kRoom && kEpi <= kRoom && (R - 1u) * kDma < 64u;
    static_assert((4u * TM) % WN == 0, "activation fragments split evenly over the slice's waves");
};

// One workgroup of four waves computes a (32·TM) x (32·NB·WN) tile of Y.
// Chunks of 64 k stream through a ring of R LDS slots, R - 1 chunks of copies
// ahead, every operand by global_load_lds with explicit vmcnt waits (the
// compiler then never needs a full drain): per chunk and K slice, the slice's
// 4·TM activation fragments (copied once, shared by the slice's WN waves) and
// each wave's weight window.  Step c: wait for chunk c + 1 (a barrier when
// slots are shared: every wave's copies landed, every wave done reading chunk
// c's slot), copy chunk c + R into chunk c's slot, read chunk c + 1's weights,
// then chunk c's MFMAs k step by k step, each followed by chunk c + 1's
// activation reads of that step and a share of its weight decode (into the
// second register set; the last step decodes a slot nothing was copied into,
// never multiplied).
//
// Epilogue: every wave's partial tile goes to LDS; the S waves of a column
// subtile each take 32·TM/S rows, add the S partials in slice order (a fixed
// order: results do not depend on timing), scale by rs[m] and store.
template <uint32_t ENC, int TM, int NB, int S>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(const GemmArgs a) {
    using G = Geo<ENC, TM, NB, S>;
    using W = typename G::W;
    constexpr uint32_t R = G::R, WN = G::WN;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ks = wave % (uint32_t)S, ns = wave / (uint32_t)S;

    // XCD-aware order: consecutive tile indices on the workgroups that land on
    // one XCD (workgroup i on XCD i % 8), so one XCD's L2 holds a band of the
    // larger operand and all of the smaller: tiles sharing weight columns
    // (N-major) when the weights are the larger operand, tiles sharing
    // activation rows (M-major) when the staged activations are.
    const uint32_t T = a.mt * a.nt;
    const uint32_t q8 = T / 8u, r8 = T % 8u, xcd = blockIdx.x % 8u;
    const uint32_t tile = (xcd < r8 ? xcd * (q8 + 1u) : r8 * (q8 + 1u) + (xcd - r8) * q8) + blockIdx.x / 8u;
    const uint32_t mtile = a.mmajor ? tile / a.nt : tile % a.mt, ntile = a.mmajor ? tile % a.nt : tile / a.mt;
    const uint32_t n0 = (ntile * WN + ns) * G::kCols;  // this wave's first column
    const uint32_t mb0 = mtile * TM;                   // first 32-row block
    const uint32_t mbs = (a.M + 31u) / 32u;

    // this wave's K slice: chunks [c0, c0 + nc) of 64 k; S divides the chunk
    // count, so every wave of the workgroup runs the same steps
    const uint32_t nchk = a.K / 64u, ksteps = a.K / 16u;
    const uint32_t nc = nchk / (uint32_t)S, c0 = nc * ks;

    // Activation copies: this wave copies fragments f = ns, ns + WN, ... of
    // its slice's 4·TM per chunk (f = 4·i + t: row block i, k step t).
    constexpr uint32_t NX = G::kDmaX;
    const uint16_t* xsrc[NX];
    uint32_t xdst[NX];
#pragma unroll
    for (uint32_t q = 0; q < NX; q++) {
        const uint32_t f = ns + q * WN, i = f / 4u, t = f % 4u;
        const uint32_t mb = mb0 + i < mbs ? mb0 + i : mbs - 1u;  // past M: re-read the last block (never stored)
        xsrc[q] = a.xh + (((size_t)mb * ksteps + 4u * c0 + t) * 64u + lane) * 8u;
        xdst[q] = (ks * 4u * TM + f) * 1024u;
    }
    W win;
    win.init(a, n0, lane, c0);
    auto slot_x = [&](uint32_t slot) { return lds + slot * G::kSlot; };
    auto slot_w = [&](uint32_t slot, uint32_t wv) { return lds + slot * G::kSlot + G::kXBytes + wv * W::kBytes; };
    auto issue = [&](uint32_t c, uint32_t slot) {  // chunk c of the range (c < nc) into a ring slot
#pragma unroll
        for (uint32_t q = 0; q < NX; q++) dma16(xsrc[q] + (size_t)c * 4u * 512u, slot_x(slot) + xdst[q]);
        win.issue(c, slot_w(slot, wave));
    };

    // Row factors of the tile's 32·TM rows, copied into LDS ahead of the ring
    // (the oldest copy in flight, so the first ring wait covers it).
    float* rs_lds = reinterpret_cast<float*>(lds + G::kRing);
    if (wave == 0 && lane < 8u * TM) dma16(a.rs + (size_t)mb0 * 32u + 4u * lane, rs_lds);

    f32x16 acc[TM][NB];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Registers: the activation fragments of the chunk being multiplied (each
    // refilled with the next chunk's once its MFMAs have issued), the raw
    // weights of the next chunk and the decoded weights of this chunk and the
    // next.
    h8 xa[TM][4];
    uint32_t raw[W::kDw * NB];
    h8 wf[2][NB][4];
    auto read_w = [&](uint32_t c) { win.read(c, slot_w(c % R, wave), raw); };
    auto read_x = [&](uint32_t slot, int t) {
        const uint8_t* sx = slot_x(slot) + ks * 4u * TM * 1024u + lane * 16u;
#pragma unroll
        for (int i = 0; i < TM; i++) xa[i][t] = *reinterpret_cast<const h8*>(sx + (4u * i + t) * 1024u);
    };
    auto decode_all = [&](uint32_t c, int p) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const typename W::Scale sc = win.scale(c, j, raw + j * W::kDw);
#pragma unroll
            for (int t = 0; t < 4; t++) wf[p][j][t] = win.step(raw + j * W::kDw, sc, t);
        }
    };
    constexpr int kPieces = 4 * NB;              // decode pieces of a chunk: (N-block, k step)
    constexpr int kPerStep = (kPieces + 2) / 3;  // decoded after the MFMAs of k steps 1, 2, 3

    auto step = [&](uint32_t c, int p) {
        // copies issued so far: chunks up to min(c + R - 1, nc - 1); chunk c + 1
        // must have landed, the newer ones may stay in flight
        const uint32_t last = c + R - 1u < nc - 1u ? c + R - 1u : nc - 1u;
        ring_barrier_k<G::kDma, R - 2u, 0u, (WN > 1u)>(last > c + 1u ? last - c - 1u : 0u);
        if (c + R < nc) issue(c + R, c % R);
        read_w(c + 1u);
        typename W::Scale sc[NB];
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int m = 0; m < TM * NB; m++) {
                const int i = m / NB, j = m % NB;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[p][j][t], xa[i][t], acc[i][j], 0, 0, 0);
            }
            if (t > 0) {
#pragma unroll
                for (int k = kPerStep * (t - 1); k < kPerStep * t && k < kPieces; k++) {
                    const int kj = k / 4, kt = k % 4;
                    if (kt == 0) sc[kj] = win.scale(c + 1u, kj, raw + kj * W::kDw);
                    wf[1 - p][kj][kt] = win.step(raw + kj * W::kDw, sc[kj], kt);
                }
            }
            read_x((c + 1u) % R, t);
        }
    };

#pragma unroll
    for (uint32_t c = 0; c < R; c++)
        if (c < nc) issue(c, c);
    // chunk 0 landed (for every wave)
    ring_barrier_k<G::kDma, R - 1u, 0u, (WN > 1u)>((nc < R ? nc : R) - 1u);
    read_w(0);
#pragma unroll
    for (int t = 0; t < 4; t++) read_x(0, t);
    decode_all(0, 0);
    uint32_t c = 0;
    for (; c + 2u <= nc; c += 2u) {
        step(c, 0);
        step(c + 1u, 1);
    }
    if (c < nc) step(c, 0);
    wait_vmcnt<0>();
    __syncthreads();  // every wave past its last chunk: the ring is free

    // Epilogue.  D = W-block x X-block: lane l holds activation row l % 32 of
    // the row block and, for r = 0..15, column 8·(r/4) + 4·(l/32) + r%4 of the
    // weight block.  Every wave writes its whole partial tile (32·TM rows x
    // 32·NB columns, f32) to its LDS rows.
    float* epi = reinterpret_cast<float*>(lds);
    constexpr uint32_t P = G::kEpiPitch;
    {
        float* mine = epi + wave * 32u * TM * P;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    *reinterpret_cast<f32x4*>(mine + (32u * i + (lane & 31u)) * P + 32u * j + 8u * q + 4u * (lane >> 5)) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    }
    if constexpr (S > 1) __syncthreads();
    // the S waves of column subtile ns take RPT rows each; lane and step s
    // cover group idx = lane + 64s: row idx / C4, columns 4·(idx % C4) .. +3
    constexpr uint32_t RPT = 32u * TM / S, C4 = G::kCols / 4u, NI = RPT * C4 / 64u;
    static_assert(RPT * C4 % 64u == 0, "whole store steps");
    f32x4 v[NI];
#pragma unroll
    for (uint32_t s = 0; s < NI; s++) {
        const uint32_t idx = lane + 64u * s, ml = ks * RPT + idx / C4, c4 = idx % C4;
        v[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < S; k++)  // slice order, the same for every output
            v[s] += *reinterpret_cast<const f32x4*>(epi + ((ns * S + k) * 32u * TM + ml) * P + 4u * c4);
    }
    // scale by rs[m] and store whole 4-column groups (16-byte f32 or 8-byte
    // bf16 stores, consecutive lanes on consecutive groups of a row),
    // non-temporal: streamed out during the kernel instead of left dirty in L2
    const uint32_t mrow = mb0 * 32u + ks * RPT;
    const bool vec_ok = (a.N & 3u) == 0 && ((uintptr_t)a.y & (a.y_bf16 ? 7u : 15u)) == 0;
    const bool whole = vec_ok && mrow + RPT <= a.M && n0 + G::kCols <= a.N;
#pragma unroll
    for (uint32_t s = 0; s < NI; s++) {
        const uint32_t idx = lane + 64u * s, r = idx / C4, n = n0 + 4u * (idx % C4), m = mrow + r;
        const f32x4 o = v[s] * rs_lds[ks * RPT + r];
        if (whole) {
            const size_t at = (size_t)m * a.N + n;
            if (a.y_bf16)
                __builtin_nontemporal_store(u32x2{f32x2_to_bf16x2_bits(o[0], o[1]), f32x2_to_bf16x2_bits(o[2], o[3])},
                                            gptr_mut<u32x2>(static_cast<uint16_t*>(a.y) + at));
            else
                __builtin_nontemporal_store(o, gptr_mut<f32x4>(static_cast<float*>(a.y) + at));
        } else if (m < a.M) {
            const size_t at = (size_t)m * a.N + n;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (n + (uint32_t)e >= a.N) break;
                if (a.y_bf16) gptr_mut<uint16_t>(a.y)[at + e] = f32_to_bf16_bits(o[e]);
                else gptr_mut<float>(a.y)[at + e] = o[e];
            }
        }
    }
}

template <uint32_t ENC, int TM, int NB, int S>
hipError_t launch(const GemmArgs& a, hipStream_t st) {
    static_assert(Geo<ENC, TM, NB, S>::kFits, "LDS of one workgroup");
    auto kernel = gemm_kernel<ENC, TM, NB, S>;
    constexpr uint32_t lds = Geo<ENC, TM, NB, S>::kLds;
    if constexpr (lds > 64u * 1024u) {
        static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL(kernel, dim3(a.mt * a.nt), dim3(kWaves * 64), lds, st, a);
    return hipGetLastError();
}

// Launch of a planned configuration (gemm_plan) for one encoding; the
// configurations whose LDS does not fit are never planned.
template <uint32_t ENC, int TM, int NB>
hipError_t launch_s(const GemmArgs& a, uint32_t s, hipStream_t st) {
    if constexpr (Geo<ENC, TM, NB, 4>::kFits)
        if (s == 4u) return launch<ENC, TM, NB, 4>(a, st);
    if constexpr (Geo<ENC, TM, NB, 2>::kFits)
        if (s == 2u) return launch<ENC, TM, NB, 2>(a, st);
    if constexpr (Geo<ENC, TM, NB, 1>::kFits)
        if (s == 1u) return launch<ENC, TM, NB, 1>(a, st);
    return hipErrorInvalidConfiguration;
}

// Configurations whose registers spill (IQ4_XS at TM 2, NB 3: 40 dwords per
// lane) are neither planned nor built.
template <uint32_t ENC, int TM, int NB>
constexpr bool kNoSpill = !(ENC == ENC_IQ4_XS && TM == 2 && NB == 3);

template <uint32_t ENC>
hipError_t launch_plan(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
    if (p.tm == 2 && p.nb == 2) return launch_s<ENC, 2, 2>(a, p.s, st);
    if constexpr (kNoSpill<ENC, 2, 3>)
        if (p.tm == 2 && p.nb == 3) return launch_s<ENC, 2, 3>(a, p.s, st);
    if (p.tm == 4 && p.nb == 2) return launch_s<ENC, 4, 2>(a, p.s, st);
    if (p.tm == 4 && p.nb == 3) return launch_s<ENC, 4, 3>(a, p.s, st);
    return hipErrorInvalidConfiguration;
}

// Whether configuration (TM, NB, S) of encoding ENC fits one workgroup's LDS.
template <uint32_t ENC>
bool fits(int tm, int nb, int s) {
    if (tm == 2 && nb == 3 && !kNoSpill<ENC, 2, 3>) return false;
    auto f = [&](auto geo2, auto geo3) { return nb == 2 ? geo2 : geo3; };
    if (tm == 2)
        return s == 4 ? f(Geo<ENC, 2, 2, 4>::kFits, Geo<ENC, 2, 3, 4>::kFits)
             : s == 2 ? f(Geo<ENC, 2, 2, 2>::kFits, Geo<ENC, 2, 3, 2>::kFits)
                      : f(Geo<ENC, 2, 2, 1>::kFits, Geo<ENC, 2, 3, 1>::kFits);
    return s == 4 ? f(Geo<ENC, 4, 2, 4>::kFits, Geo<ENC, 4, 3, 4>::kFits)
         : s == 2 ? f(Geo<ENC, 4, 2, 2>::kFits, Geo<ENC, 4, 3, 2>::kFits)
                  : f(Geo<ENC, 4, 2, 1>::kFits, Geo<ENC, 4, 3, 1>::kFits);
}

}  // namespace gemm
}  // namespace dmx
