// Prefill GEMM on gfx950 MFMA for the GGUF encodings Q4_0, Q4_1, Q8_0, Q6_K,
// Q4_K, Q5_K and IQ4_XS and for MLX affine U4: Y[M, N] = X[M, K] · Wᵀ with f32 accumulation.
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
//   * A workgroup of four waves owns a (32·TM) x (64·4/S) tile of Y: each
//     wave a (32·TM) x 64 tile (TM x 2 blocks of v_mfma_f32_32x32x16_f16),
//     the four waves split over S slices of K and 4/S column subtiles.
//   * K advances in chunks of two weight blocks (64 k, four MFMA k steps)
//     through an LDS ring of R chunks, one barrier per chunk.  Each chunk's
//     activation fragments (1 KiB each, contiguous in HBM) are copied by
//     global_load_lds_dwordx4 once per slice and read by every wave of the
//     slice; each wave's 64 weight rows are copied the same way into a window
//     per wave: the row's two blocks from their 4-byte-aligned start, as
//     16-byte pieces (consecutive lanes on consecutive pieces, the last piece
//     moved back so that no read passes the blocks' last dword).  Copies run
//     R - 1 chunks ahead and hold no registers.
//   * Every lane decodes one whole block straight into B operands: lane l
//     takes weight row l % 32 of a 32-row block and block h = l / 32 of the
//     chunk, so an MFMA k step pairs 8 k of the chunk's first block (lanes
//     0..31) with 8 k of its second (lanes 32..63), and xprep stages the
//     activations in that order.  A code at mantissa bits 0.. under the f16
//     exponent of 1024 is 1024 + c, one at bits 4.. under that of 64 is
//     64 + c (one v_and_or_b32 per two codes, both exact); a packed add removes
//     the offset (exact) and a packed multiply by the block scale rounds once
//     (Q4_0 RNE_f16((q-8)·d), Q8_0 RNE_f16(q·d)); Q4_1 a packed fma,
//     RNE_f16(q·d + m); Q6_K RNE_f16((q-32)·RNE_f16(d·sc)) (its window and
//     decode are described at WinQ6K); MLX U4 RNE_f16(q·s + b) (WinMlx);
//     Q4_K RNE_f16(q·RNE_f16(d·sc) - RNE_f16(dmin·m)) (WinQ4K).
//   * The weights are the MFMA's A operand and the activations its B, so each
//     lane ends with 4 consecutive output columns of one row per block and
//     stores them as one 16-byte (f32) or 8-byte (bf16) write.  K slices meet
//     in LDS after the loop, summed in slice order by one wave per output
//     (deterministic), then scaled by rs[m].
//   * Workgroups that read the same weight rows run on the same XCD
//     (workgroup i goes to XCD i % 8).
// Accuracy: |y - y_exact| <= 2^-10·Σ|w||x| (one f16 rounding of each weight and
// of each activation; Q6_K's weights round twice: (2^-10 + 2^-11)·Σ|w||x|;
// Q4_K's scale and offset round once each, adding 2^-11·Σ(|q·d·sc| + |dmin·m|)|x|) +
// f32 accumulation error, inside the 2e-3 normalised tolerance.  Weights must
// be finite in f16 (|w| <= 65504: |d| <= 8188 for Q4_0, |d·sc| <= 2047 for
// Q6_K).
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

namespace {

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

// The ring's step barrier: this wave's copies older than its last n have
// landed in LDS and its LDS reads are done (s_waitcnt vmcnt(n) lgkmcnt(0)),
// then s_barrier.  __syncthreads() would also wait for the copies still in
// flight (its fence waits for vmcnt(0)); the empty asm statements keep the
// compiler from moving memory accesses across the barrier.
template <uint32_t n>
__device__ __forceinline__ void ring_barrier() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The wait of ring_barrier<n>() without the barrier: for a wave whose ring
// slots no other wave reads or writes.
template <uint32_t n>
__device__ __forceinline__ void ring_wait() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4));
    asm volatile("" ::: "memory");
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

// A wave's weight window: its 64 rows' bytes of one 64-k chunk, copied into
// LDS, and each lane's reads and decode of its block.
//
// GGUF blocks of 32 weights: a row's two blocks of the chunk are contiguous;
// they are copied from their 4-byte-aligned start as NP 16-byte pieces
// (consecutive lanes on consecutive pieces of a row), the last piece moved
// back so that no read passes the blocks' last dword.  Lane l decodes row
// l % 32 of each 32-row half j, block h = l / 32 of the chunk.
template <uint32_t ENC>
struct WinBlocks {
    using B = Blk<ENC>;
    using Scale = typename B::Scale;
    static constexpr uint32_t kSpanMax = (2u * B::kBytes + 2u + 3u) & ~3u;  // a row's two blocks, aligned
    static constexpr uint32_t NP = (kSpanMax + 15u) / 16u;                   // 16-byte pieces per row
    static constexpr uint32_t kCopies = NP;                                  // copy instructions per chunk
    static constexpr uint32_t kBytes = 64u * NP * 16u;
    static constexpr uint32_t kDw = B::kDw;
    const uint8_t* src[NP];       // copy lane's piece for the slice's first chunk
    uint32_t off[2][kDw], sh[2];  // this lane's block dwords in the window, its block's start offset

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane, uint32_t c0) {
#pragma unroll
        for (uint32_t q = 0; q < NP; q++) {
            const uint32_t li = 64u * q + lane, r = li / NP, p = li % NP;
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
        for (int j = 0; j < 2; j++) {
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
        for (uint32_t q = 0; q < NP; q++) dma16(src[q] + (size_t)c * 2u * B::kBytes, win + 1024u * q);
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < 2; j++)
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
struct WinQ6K {
    static constexpr uint32_t kX16 = 6, kX4 = 5, kCopies = kX16 + kX4;
    static constexpr uint32_t kPitch16 = 16u * kX16, kPitch4 = 4u * kX4;
    static constexpr uint32_t kBytes = 64u * (kPitch16 + kPitch4);
    static constexpr uint32_t kDw = 20;  // ql 9, qh 9, scale dword, d dword
    struct Scale {
        uint32_t sel, mN, magic, mH, sL;
        h2 off, ds0, ds1;
    };
    uintptr_t rb16[kX16], rb4[kX4];  // row of each copy lane (its first super-block)
    uint32_t p16[kX16], p4[kX4];     // piece of each copy lane
    uintptr_t row[2];                // this lane's rows
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
        for (uint32_t q = 0; q < kX16; q++) {
            const uint32_t li = 64u * q + lane;
            rb16[q] = rowp(li / kX16);
            p16[q] = li % kX16;
        }
#pragma unroll
        for (uint32_t q = 0; q < kX4; q++) {
            const uint32_t li = 64u * q + lane;
            rb4[q] = rowp(li / kX4);
            p4[q] = li % kX4;
        }
#pragma unroll
        for (int j = 0; j < 2; j++) row[j] = rowp(32u * j + (lane & 31u));
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, hn = (g >> 1) & 1u, ph = g & 1u;
#pragma unroll
        for (uint32_t q = 0; q < kX16; q++) {
            const uintptr_t al = (rb16[q] + (uintptr_t)sb * 210u) & ~(uintptr_t)3;
            const uint32_t p = p16[q];
            const uint32_t o = p < 4u ? 64u * hn + 16u * p : 128u + 32u * hn + 16u * (p - 4u);
            dma16(reinterpret_cast<const void*>(al + o), win + 1024u * q);
        }
#pragma unroll
        for (uint32_t q = 0; q < kX4; q++) {
            const uintptr_t al = (rb4[q] + (uintptr_t)sb * 210u) & ~(uintptr_t)3;
            const uint32_t p = p4[q];
            const uint32_t o = p == 0u ? 64u * hn + 64u
                             : p == 1u ? 160u + 32u * hn
                             : p == 2u ? 192u + 8u * hn + 4u * ph
                             : p == 3u ? 196u + 8u * hn + 4u * ph
                                       : 208u;
            dma4(reinterpret_cast<const void*>(al + o), win + 64u * kPitch16 + 256u * q);
        }
    }
    __device__ uint32_t shift_of(uint32_t c, int j) const { return (uint32_t)((row[j] + (uintptr_t)((c0 + c) >> 2) * 210u) & 3u); }
    __device__ void read(uint32_t c, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t r = 32u * j + (lane & 31u);
            const uint8_t* w16 = win + r * kPitch16;
            const uint8_t* w4 = win + 64u * kPitch16 + r * kPitch4;
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
// halves (the same group unless group = 32).  Lane l decodes row l % 32 of
// each 32-row half j, words 4h .. 4h+3 (h = l / 32): k step t takes word
// 4h + t, nibbles (0,4) (1,5) (2,6) (3,7) as packed pairs (XFRAG_WORD), code q
// exact in f16 and w = RNE_f16(q·s + b) by one packed fma, s and b taken to
// f16 first (bf16 and f16 values exact in f16's normal range; f32 rounded).
struct WinMlx {
    static constexpr uint32_t kPieces = 2, kAux = 4, kCopies = kPieces + kAux;
    static constexpr uint32_t kAuxOff = 64u * 16u * kPieces;  // aux dwords after the 64 rows' pieces
    static constexpr uint32_t kBytes = kAuxOff + 256u * kAux;
    static constexpr uint32_t kDw = 6;  // 4 code words, scale dword, bias dword
    struct Scale {
        h2 s, b;
    };
    const uint8_t* src[kPieces];  // copy lane's piece of the slice's first chunk
    uintptr_t srow, brow;         // copy lane's row (= lane) of scales and biases
    uint32_t ssh[2], bsh[2];      // this lane's rows' scale and bias row starts mod 4 (per 32-row half j)
    uint32_t c0, es, group, sdtype, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
        group = a.group;
        sdtype = a.sdtype;
        es = a.sdtype == DT_F32 ? 4u : 2u;
        const uint32_t rbytes = a.K / 2u, sbytes = a.K / a.group * es;
        auto rowc = [&](uint32_t r) { return n0 + r < a.N ? n0 + r : a.N - 1u; };  // past N: re-read the last row
#pragma unroll
        for (uint32_t q = 0; q < kPieces; q++) {
            const uint32_t li = 64u * q + lane;
            src[q] = a.w + (size_t)rowc(li / 2u) * rbytes + 32u * c0 + 16u * (li % 2u);
        }
        srow = (uintptr_t)a.sc + (uintptr_t)rowc(lane) * sbytes;
        brow = (uintptr_t)a.bi + (uintptr_t)rowc(lane) * sbytes;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uintptr_t o = (uintptr_t)rowc(32u * j + (lane & 31u)) * sbytes;
            ssh[j] = (uint32_t)(((uintptr_t)a.sc + o) & 3u);
            bsh[j] = (uint32_t)(((uintptr_t)a.bi + o) & 3u);
        }
    }
    // byte offset in a scale row of the group of the chunk's 32-k half hh
    __device__ uint32_t goff(uint32_t c, uint32_t hh) const { return (64u * (c0 + c) + 32u * hh) / group * es; }
    __device__ void issue(uint32_t c, uint8_t* win) const {
#pragma unroll
        for (uint32_t q = 0; q < kPieces; q++) dma16(src[q] + (size_t)c * 32u, win + 1024u * q);
#pragma unroll
        for (uint32_t hh = 0; hh < 2; hh++) {
            const uint32_t o = goff(c, hh);
            dma4(reinterpret_cast<const void*>((srow + o) & ~(uintptr_t)3), win + kAuxOff + 256u * hh);
            dma4(reinterpret_cast<const void*>((brow + o) & ~(uintptr_t)3), win + kAuxOff + 256u * (2u + hh));
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
        const uint32_t h = lane >> 5;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t r = 32u * j + (lane & 31u);
            const u32x4 q = *reinterpret_cast<const u32x4*>(win + 32u * r + 16u * h);
            uint32_t* o = raw + j * kDw;
            o[0] = q.x;
            o[1] = q.y;
            o[2] = q.z;
            o[3] = q.w;
            o[4] = *reinterpret_cast<const uint32_t*>(win + kAuxOff + 256u * h + 4u * r);
            o[5] = *reinterpret_cast<const uint32_t*>(win + kAuxOff + 256u * (2u + h) + 4u * r);
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
template <bool Q5>
struct WinQK {
    static constexpr uint32_t NP = Q5 ? 5u : 3u, kCopies = NP;
    static constexpr uint32_t kPitch = 16u * NP;
    static constexpr uint32_t kBytes = 64u * kPitch;
    static constexpr uint32_t QS = Q5 ? 12u : 4u;          // raw dword of the codes
    static constexpr uint32_t SB = Q5 ? 176u : 144u;       // super-block bytes
    static constexpr uint32_t kDw = QS + 8u;               // d|dmin, three scale dwords, [8 qh dwords,] 8 code dwords
    struct Scale {
        h2 ds, ndm, off;
        uint32_t mask, magic, hsh, sl, mh;
    };
    uintptr_t rb[NP];  // row of each copy lane
    uint32_t pp[NP];   // piece of each copy lane
    uint32_t c0, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
#pragma unroll
        for (uint32_t q = 0; q < NP; q++) {
            const uint32_t li = 64u * q + lane, r = li / NP;
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            rb[q] = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes;
            pp[q] = li % NP;
        }
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, i = g & 3u;
#pragma unroll
        for (uint32_t q = 0; q < NP; q++) {
            const uint32_t p = pp[q];
            // pieces: header, [qh, qh,] the step's two code pieces
            const uint32_t o = p == 0u ? 0u : p + 2u < NP ? 16u * p : 16u * (QS / 4u) + 32u * i + 16u * (p + 2u - NP);
            dma16(reinterpret_cast<const void*>(rb[q] + (uintptr_t)sb * SB + o), win + 1024u * q);
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < 2; j++) {
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

using WinQ4K = WinQK<false>;
using WinQ5K = WinQK<true>;

// GGUF IQ4_XS (GGML block_iq4_xs, 136-byte super-blocks of 256 weights; the
// reference's schema gguf_block.rs:183-316): chunk g of a row covers
// sub-blocks 2i and 2i + 1 (i = g % 4) of super-block g / 4; lane half h
// decodes sub-block 2i + h, laid out as a Q4_0 block (XFRAG_NIB order), each
// nibble looked up in the codebook (iq4nl_lookup) and decoded as Q8_0's codes:
// w = RNE_f16(kv·RNE_f16(d·(ls - 32))).  The window per row: the 16 bytes
// from the super-block's start (d, scales_h, scales_l) and the chunk's 32
// code bytes, three 16-byte pieces within the super-block.
struct WinIQ4XS {
    static constexpr uint32_t NP = 3, kCopies = NP;
    static constexpr uint32_t kPitch = 16u * NP;
    static constexpr uint32_t kBytes = 64u * kPitch;
    static constexpr uint32_t kDw = 12;  // d|scales_h, scales_l, two unused, 8 code dwords
    struct Scale {
        h2 ds;
        uint32_t h;
    };
    uintptr_t rb[NP];
    uint32_t pp[NP];
    uint32_t c0, lane;

    __device__ void init(const GemmArgs& a, uint32_t n0, uint32_t lane_, uint32_t c0_) {
        lane = lane_;
        c0 = c0_;
#pragma unroll
        for (uint32_t q = 0; q < NP; q++) {
            const uint32_t li = 64u * q + lane, r = li / NP;
            const uint32_t n = n0 + r < a.N ? n0 + r : a.N - 1u;  // past N: re-read the last row (never stored)
            rb[q] = (uintptr_t)a.w + (uintptr_t)n * a.rowbytes;
            pp[q] = li % NP;
        }
    }
    __device__ void issue(uint32_t c, uint8_t* win) const {
        const uint32_t g = c0 + c, sb = g >> 2, i = g & 3u;
#pragma unroll
        for (uint32_t q = 0; q < NP; q++) {
            const uint32_t o = pp[q] == 0u ? 0u : 8u + 32u * i + 16u * (pp[q] - 1u);
            dma16(reinterpret_cast<const void*>(rb[q] + (uintptr_t)sb * 136u + o), win + 1024u * q);
        }
    }
    __device__ void read(uint32_t, const uint8_t* win, uint32_t* raw) const {
#pragma unroll
        for (int j = 0; j < 2; j++) {
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

template <uint32_t ENC>
struct WinOf {
    using type = WinBlocks<ENC>;
};
template <>
struct WinOf<ENC_IQ4_XS> {
    using type = WinIQ4XS;
};
template <>
struct WinOf<ENC_Q4_K> {
    using type = WinQ4K;
};
template <>
struct WinOf<ENC_Q5_K> {
    using type = WinQ5K;
};
template <>
struct WinOf<ENC_MLX_U4> {
    using type = WinMlx;
};
template <>
struct WinOf<ENC_Q6_K> {
    using type = WinQ6K;
};

// LDS geometry of one kernel configuration.
template <uint32_t ENC, int TM, int S>
struct Geo {
    using W = typename WinOf<ENC>::type;
    static constexpr uint32_t WN = kWaves / S;                         // column subtiles per workgroup
    static constexpr uint32_t kWinBytes = W::kBytes;                    // a wave's 64-row window
    // S = 4: every wave multiplies a K slice of its own, so no two waves share
    // an activation fragment.  The fragments then go from the staged
    // activations straight into registers (kXReg), two chunks ahead, and the
    // ring holds only the waves' own weight windows, so it needs no barrier.
    // Not for Q6_K at TM = 2: its larger windows then wait on their copies
    // (the compiler waits for all loads at each step's first MFMA), and the
    // copies through LDS measured faster (M128 N3072 K1024 15.0 against 16.6
    // µs; M512 at TM = 4 21.4 against 24.5).
    static constexpr bool kXReg = S == 4 && !(ENC == ENC_Q6_K && TM == 2);
    static constexpr uint32_t kABytes = kXReg ? 0u : (uint32_t)S * 4u * TM * 1024u;  // activation fragments of a chunk
    static constexpr uint32_t kSlot = kABytes + kWaves * kWinBytes;
    static constexpr uint32_t kRs = 32u * TM * 4u;                      // the tile's row factors
    static constexpr uint32_t kEpiPitch = 68u;                          // floats per output row in LDS
    static constexpr uint32_t kEpi = (uint32_t)kWaves * 32u * TM * kEpiPitch * 4u;  // every wave's whole tile
    static constexpr uint32_t kRoom = kLdsMax - kRs;
    static constexpr uint32_t R0 = 4u * kSlot <= kRoom ? 4u : 3u * kSlot <= kRoom ? 3u : 2u;
    static constexpr uint32_t R = kXReg && R0 > 3u ? 3u : R0;  // (keeps the wait counts below 64)
    static constexpr uint32_t kRing = R * kSlot > kEpi ? R * kSlot : kEpi;  // the epilogue reuses the ring
    static constexpr uint32_t kLds = kRing + kRs;
    static constexpr uint32_t kDmaA = kXReg ? 0u : 4u * TM / WN;  // activation copies per wave per chunk
    static constexpr uint32_t kDma = kDmaA + W::kCopies;  // all copies per wave per chunk
    static constexpr uint32_t kXLoads = kXReg ? 4u * TM : 0u;  // activation register loads per wave per step
    static_assert((R - 1u) * kXLoads + (R - 2u) * W::kCopies < 64 && 2u * kXLoads + (R - 1u) * W::kCopies < 64,
                  "wait counts fit vmcnt");
    static constexpr bool kFits = 2u * kSlot <= kRoom;
    static_assert((4u * TM) % WN == 0, "activation fragments split evenly over the slice's waves");
};

template <uint32_t ENC, int TM, int S>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(const GemmArgs a) {
    using G = Geo<ENC, TM, S>;
    constexpr uint32_t R = G::R;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ks = wave % (uint32_t)S, ns = wave / (uint32_t)S;

    // XCD-aware tile order: consecutive tile indices on the workgroups that
    // land on one XCD (workgroup i on XCD i % 8), so each XCD's L2 holds one
    // band of the larger operand and all of the smaller: tiles sharing weight
    // columns (N-major) when the weights are the larger, tiles sharing
    // activation rows (M-major) when the staged activations are.
    const uint32_t T = a.mt * a.nt;
    const uint32_t q8 = T / 8u, r8 = T % 8u, xcd = blockIdx.x % 8u;
    const uint32_t tau = (xcd < r8 ? xcd * (q8 + 1u) : r8 * (q8 + 1u) + (xcd - r8) * q8) + blockIdx.x / 8u;
    const uint32_t mtile = a.mmajor ? tau / a.nt : tau % a.mt, ntile = a.mmajor ? tau % a.nt : tau / a.mt;
    const uint32_t n0 = (ntile * G::WN + ns) * 64u;  // this wave's 64 columns
    const uint32_t mb0 = mtile * TM;                 // first 32-row block
    const uint32_t mbs = (a.M + 31u) / 32u;

    // K slice: chunks [c0, c0 + nc) of two blocks; S divides the chunk count,
    // so every wave runs the same steps and meets the same barriers
    const uint32_t nchk = a.K / 64u, ksteps = a.K / 16u;
    const uint32_t nc = nchk / S, c0 = nc * ks;

    // Activation copies: this wave copies fragments f = ns, ns + WN, ... of its
    // slice's 4·TM per chunk (f = 4·i + t: row block i, k step t); with kXReg
    // (WN = 1) it loads all of them into registers instead.
    constexpr uint32_t NX = G::kXReg ? 4u * TM : G::kDmaA;
    const uint16_t* xsrc[NX];
    uint32_t xdst[NX];
#pragma unroll
    for (uint32_t q = 0; q < NX; q++) {
        const uint32_t f = ns + q * G::WN, i = f / 4u, t = f % 4u;
        const uint32_t mb = mb0 + i < mbs ? mb0 + i : mbs - 1u;  // past M: re-read the last block (never stored)
        xsrc[q] = a.xh + (((size_t)mb * ksteps + 4u * c0 + t) * 64u + lane) * 8u;
        xdst[q] = (ks * 4u * TM + f) * 1024u;
    }
    using W = typename G::W;
    W win;
    win.init(a, n0, lane, c0);
    auto slot_a = [&](uint32_t slot) { return lds + slot * G::kSlot; };
    auto slot_w = [&](uint32_t slot, uint32_t wv) { return lds + slot * G::kSlot + G::kABytes + wv * G::kWinBytes; };
    auto issue = [&](uint32_t c, uint32_t slot) {  // chunk c of the slice (c < nc) into a ring slot
#pragma unroll
        for (uint32_t q = 0; q < G::kDmaA; q++) dma16(xsrc[q] + (size_t)c * 4u * 512u, slot_a(slot) + xdst[q]);
        win.issue(c, slot_w(slot, wave));
    };

    // Row factors of the tile's 32·TM rows, copied into LDS ahead of the ring
    // (the oldest copy in flight, so the first ring wait covers it).
    float* rs_lds = reinterpret_cast<float*>(lds + G::kRing);
    if (wave == 0 && lane < 8u * TM) dma16(a.rs + (size_t)mb0 * 32u + 4u * lane, rs_lds);

    f32x16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Registers: the activation fragments of the chunk being multiplied (each
    // refilled from the next chunk's slot once its MFMAs have issued; with
    // kXReg, two sets: chunk c's in xa[c % 2], refilled from global memory with
    // chunk c + 2's), and the raw and decoded weights of the current and the
    // next chunk.
    constexpr int NXA = G::kXReg ? 2 : 1;
    h8 xa[NXA][TM][4];
    uint32_t raw[W::kDw * 2];
    h8 wf[2][2][4];
    auto read_w = [&](uint32_t c) { win.read(c, slot_w(c % R, wave), raw); };  // chunk c's weights
    auto read_a = [&](uint32_t slot, int t) {
        const uint8_t* sa = slot_a(slot) + ks * 4u * TM * 1024u + lane * 16u;
#pragma unroll
        for (int i = 0; i < TM; i++) xa[0][i][t] = *reinterpret_cast<const h8*>(sa + (4u * i + t) * 1024u);
    };
    // kXReg: k step t of chunk c (past the slice: its last chunk again, never
    // multiplied) into register set p; every step loads 4·TM fragments, so
    // the ring's wait counts are fixed
    auto load_a = [&](uint32_t c, int p, int t) {
        const uint32_t cc = c < nc ? c : nc - 1u;
#pragma unroll
        for (int i = 0; i < TM; i++)
            xa[p][i][t] = *gptr<h8>(xsrc[4 * i + t] + (size_t)cc * 4u * 512u);
    };
    auto decode_all = [&](uint32_t c, int p) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const typename W::Scale sc = win.scale(c, j, raw + j * W::kDw);
#pragma unroll
            for (int t = 0; t < 4; t++) wf[p][j][t] = win.step(raw + j * W::kDw, sc, t);
        }
    };

    // One step of the pipeline, chunk c with weights wf[p]: barrier (chunk c + 1
    // landed for every wave; every wave done reading chunk c), copy chunk c + R
    // into chunk c's slot, read chunk c + 1's weights, then the MFMAs of chunk
    // c in k-step order, each k step followed by the next chunk's activation
    // reads of that step, with chunk c + 1's decode into wf[1 - p] placed
    // after the MFMAs of k steps 1..3 (the MFMAs run in the matrix core while
    // the decode issues).  The compiler interleaves them: scheduling-group
    // barriers that pinned one MFMA, then its share of the decode, ran 1-6%
    // slower on every encoding.  The copies write slot c % R, the reads take
    // slot (c + 1) % R, so their order within a step does not matter.
    // The last step reads a slot no chunk was copied into; its decode is
    // never multiplied.  With kXReg the step loads chunk c + 2's activation
    // fragments into register set p after each k step, and waits for its own
    // copies only: chunk c + 1's weights, with the activation loads of the
    // last R - 1 steps still in flight.
    auto step = [&](uint32_t c, int p) {
        // copies issued so far: chunks up to min(c + R, nc) - 1; chunk c + 1 must
        // have landed, the newer ones may stay in flight
        // (kXReg: every step issues the same copies and loads, past the end
        // chunk nc - 1's window again, so the counts are fixed and the
        // compiler's own waits for the activation registers stay partial)
        const uint32_t last = c + R - 1u < nc - 1u ? c + R - 1u : nc - 1u;
        ring_barrier_k<G::kDma, R - 2u, (R - 1u) * G::kXLoads, !G::kXReg>(
            G::kXReg ? R - 2u : last > c + 1u ? last - c - 1u : 0u);
        const uint32_t cn = c + R;
        if constexpr (G::kXReg) issue(cn < nc ? cn : nc - 1u, c % R);
        else if (cn < nc) issue(cn, c % R);
        const uint32_t nxt = (c + 1u) % R;
        read_w(c + 1u);
        typename W::Scale sc[2];
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int m = 0; m < 2 * TM; m++) {
                const int i = m >> 1, j = m & 1;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[p][j][t], xa[G::kXReg ? p : 0][i][t], acc[i][j],
                                                                   0, 0, 0);
            }
            if (t > 0) {
                // decode pieces (weight block kj, k step kt) k = 3(t-1) .. (steps 1, 2, 3 take 3, 3, 2)
#pragma unroll
                for (int k = 3 * (t - 1); k < 3 * t && k < 8; k++) {
                    const int kj = k >> 2, kt = k & 3;
                    if (kt == 0) sc[kj] = win.scale(c + 1u, kj, raw + kj * W::kDw);
                    wf[1 - p][kj][kt] = win.step(raw + kj * W::kDw, sc[kj], kt);
                }
            }
            if constexpr (G::kXReg) load_a(c + 2u, p, t);
            else read_a(nxt, t);
        }
    };

#pragma unroll
    for (uint32_t c = 0; c < R; c++)
        if (G::kXReg || c < nc) issue(c < nc ? c : nc - 1u, c);
    if constexpr (G::kXReg) {
#pragma unroll
        for (int t = 0; t < 4; t++) load_a(0u, 0, t);
#pragma unroll
        for (int t = 0; t < 4; t++) load_a(1u, 1, t);
    }
    // chunk 0 landed (for every wave; with kXReg for this one, chunks 0 and 1's
    // activation loads still in flight)
    ring_barrier_k<G::kDma, R - 1u, 2u * G::kXLoads, !G::kXReg>(G::kXReg ? R - 1u : (nc < R ? nc : R) - 1u);
    read_w(0);
    if constexpr (!G::kXReg) {
#pragma unroll
        for (int t = 0; t < 4; t++) read_a(0, t);
    }
    decode_all(0, 0);
    uint32_t c = 0;
    for (; c + 2u <= nc; c += 2u) {
        step(c, 0);
        step(c + 1u, 1);
    }
    if (c < nc) step(c, 0);
    wait_vmcnt<0>();
    __syncthreads();  // every wave past its last chunk: the ring is free

    // Epilogue.  D = W-block x X-block: lane l holds activation row l % 32
    // of the row block and, for r = 0..15, column 8·(r/4) + 4·(l/32) + r%4.
    // Every wave writes its whole partial tile (32·TM rows x 64 columns, f32)
    // to its LDS rows; then the S waves of a column subtile each take 32·TM/S
    // of the rows, add the S partials in slice order (deterministic), scale by
    // rs[m] and store whole rows, 16 lanes per 64-column row, non-temporal
    // (streamed out during the kernel instead of left dirty in L2 for the
    // end-of-kernel write-back).  All LDS reads of a wave are issued before
    // its first store.
    float* epi = reinterpret_cast<float*>(lds);
    {
        float* mine = epi + wave * 32u * TM * G::kEpiPitch;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    *reinterpret_cast<f32x4*>(mine + (32u * i + (lane & 31u)) * G::kEpiPitch + 32u * j + 8u * q +
                                              4u * (lane >> 5)) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    }
    if constexpr (S > 1) __syncthreads();
    constexpr uint32_t RPT = 32u * TM / S, NI = RPT / 4u;  // rows per wave, store instructions per wave
    f32x4 v[NI];
#pragma unroll
    for (uint32_t s4 = 0; s4 < NI; s4++) {
        const uint32_t ml = ks * RPT + 4u * s4 + (lane >> 4), c4 = lane & 15u;
        v[s4] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < S; k++)  // slice order, the same for every output
            v[s4] += *reinterpret_cast<const f32x4*>(epi + ((ns * S + k) * 32u * TM + ml) * G::kEpiPitch + 4u * c4);
        v[s4] *= rs_lds[ml];
    }
    const uint32_t mrow0 = mb0 * 32u + ks * RPT + (lane >> 4), ncol = n0 + 4u * (lane & 15u);
    const bool vec_ok = (a.N & 3u) == 0 && ((uintptr_t)a.y & (a.y_bf16 ? 7u : 15u)) == 0;
    if (vec_ok && mb0 * 32u + ks * RPT + RPT <= a.M && n0 + 64u <= a.N) {  // whole rows in range: no per-lane tests
#pragma unroll
        for (uint32_t s4 = 0; s4 < NI; s4++) {
            const size_t idx = (size_t)(mrow0 + 4u * s4) * a.N + ncol;
            if (a.y_bf16) {
                const uint32_t lo = (uint32_t)f32_to_bf16_bits(v[s4][0]) | ((uint32_t)f32_to_bf16_bits(v[s4][1]) << 16);
                const uint32_t hi = (uint32_t)f32_to_bf16_bits(v[s4][2]) | ((uint32_t)f32_to_bf16_bits(v[s4][3]) << 16);
                __builtin_nontemporal_store(u32x2{lo, hi}, gptr_mut<u32x2>(static_cast<uint16_t*>(a.y) + idx));
            } else {
                __builtin_nontemporal_store(v[s4], gptr_mut<f32x4>(static_cast<float*>(a.y) + idx));
            }
        }
    } else {
#pragma unroll
        for (uint32_t s4 = 0; s4 < NI; s4++) {
            const uint32_t m = mrow0 + 4u * s4;
            if (m >= a.M) continue;
            const size_t idx = (size_t)m * a.N + ncol;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (ncol + (uint32_t)e >= a.N) break;
                if (a.y_bf16) gptr_mut<uint16_t>(a.y)[idx + e] = f32_to_bf16_bits(v[s4][e]);
                else gptr_mut<float>(a.y)[idx + e] = v[s4][e];
            }
        }
    }
}

template <uint32_t ENC, int TM, int S>
hipError_t launch(const GemmArgs& a, hipStream_t st) {
    static_assert(Geo<ENC, TM, S>::kFits, "LDS of one workgroup");
    auto kernel = gemm_kernel<ENC, TM, S>;
    constexpr uint32_t lds = Geo<ENC, TM, S>::kLds;
    if constexpr (lds > 64u * 1024u) {
        static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL(kernel, dim3(a.mt * a.nt), dim3(kWaves * 64), lds, st, a);
    return hipGetLastError();
}

template <uint32_t ENC, int TM>
hipError_t launch_s(GemmArgs a, int S, hipStream_t st) {
    a.mt = ((a.M + 31u) / 32u + TM - 1u) / TM;
    a.nt = (a.N + 64u * (kWaves / S) - 1u) / (64u * (kWaves / S));
    if constexpr (Geo<ENC, TM, 4>::kFits)
        if (S == 4) return launch<ENC, TM, 4>(a, st);
    if (S >= 2) return launch<ENC, TM, 2>(a, st);
    return launch<ENC, TM, 1>(a, st);
}

template <uint32_t ENC>
hipError_t launch_enc(GemmArgs a, hipStream_t st) {
    // Wave tile (TM row blocks) and K split (S slices per workgroup) from a
    // cost model fitted to timing sweeps (M in {128, 512, 2048}, N in {1024,
    // 3072, 12288}, K in {1024, 3072, 4096}), in units of about 0.1 us:
    // rounds of 256 workgroups (one per CU) x (chunks per slice x time per
    // chunk + start-up and stores), where a chunk takes ~2·TM + 4 and the
    // four-slice ring, only two chunks deep, ~4 more.  TM = 4 only when M
    // fills more than 64 rows; S divides the chunk count (the slices, and so
    // the waves' ring barriers, are equal in number) and leaves >= 2 chunks
    // per slice.
    const uint32_t mb = (a.M + 31u) / 32u;
    const uint32_t nchk = a.K / 64u;
    int best_tm = 2, best_s = 1;
    uint64_t best_cost = ~0ull;
    for (int TM : {4, 2}) {  // ties keep the larger tile
        if (TM == 4 && mb <= 2u) continue;
        const uint64_t mt = (mb + TM - 1u) / TM;
        for (int S : {1, 2, 4}) {
            // equal slices: every wave of a workgroup passes the same barriers
            if (S > 1 && (nchk % S != 0 || nchk < 2u * S)) continue;
            if (S == 4 && !(TM == 2 ? Geo<ENC, 2, 4>::kFits : Geo<ENC, 4, 4>::kFits)) continue;
            const uint64_t nt = (a.N + 64u * (kWaves / S) - 1u) / (64u * (kWaves / S));
            const uint64_t rounds = (mt * nt + 255u) / 256u;
            const uint64_t cost = rounds * ((nchk / S) * (2u * TM + 4u + (S == 4 ? 4u : 0u)) + 24u);
            if (cost < best_cost) best_cost = cost, best_tm = TM, best_s = S;
        }
    }
    if (best_tm == 2) return launch_s<ENC, 2>(a, best_s, st);
    return launch_s<ENC, 4>(a, best_s, st);
}

}  // namespace

uint32_t gemm_layout(uint32_t enc) {
    switch (enc) {
        case ENC_Q4_0: return Blk<ENC_Q4_0>::kLayout;
        case ENC_Q4_1: return Blk<ENC_Q4_1>::kLayout;
        case ENC_Q8_0: return Blk<ENC_Q8_0>::kLayout;
        case ENC_Q6_K: return XFRAG_BYTE;  // a lane's 32 codes in order, as Q8_0
        case ENC_Q4_K:
        case ENC_Q5_K: return XFRAG_BYTE;
        case ENC_IQ4_XS: return XFRAG_NIB;  // a sub-block laid out as a Q4_0 block
        case ENC_MLX_U4: return XFRAG_WORD;
        default: return ~0u;
    }
}

bool gemm_supported(uint32_t enc, uint32_t N, uint32_t K, uint32_t M) {
    return gemm_layout(enc) != ~0u && N > 0 && M > 0 && K >= 64u &&
           K % (enc == ENC_Q6_K || enc == ENC_Q4_K || enc == ENC_Q5_K || enc == ENC_IQ4_XS ? 256u : 64u) == 0;
}

hipError_t gemm_launch(const GemmWeight& wt, uint32_t N, uint32_t K, const uint16_t* xh, const float* rs, uint32_t M,
                       void* y, bool y_bf16, hipStream_t st) {
    const uint32_t enc = wt.enc;
    if (!gemm_supported(enc, N, K, M)) return hipErrorInvalidValue;
    if (enc == ENC_MLX_U4 && (wt.group == 0 || wt.group % 32u || K % wt.group || wt.sdtype > DT_BF16 || !wt.sc || !wt.bi))
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.w = wt.w;
    a.xh = xh;
    a.rs = rs;
    a.y = y;
    a.M = M;
    a.N = N;
    a.K = K;
    a.y_bf16 = y_bf16 ? 1u : 0u;
    a.sc = wt.sc;
    a.bi = wt.bi;
    a.group = wt.group;
    a.sdtype = wt.sdtype;
    switch (enc) {
        case ENC_Q4_0: a.rowbytes = (uint64_t)(K / 32u) * Blk<ENC_Q4_0>::kBytes; break;
        case ENC_Q4_1: a.rowbytes = (uint64_t)(K / 32u) * Blk<ENC_Q4_1>::kBytes; break;
        case ENC_Q8_0: a.rowbytes = (uint64_t)(K / 32u) * Blk<ENC_Q8_0>::kBytes; break;
        case ENC_Q6_K: a.rowbytes = (uint64_t)(K / 256u) * 210u; break;
        case ENC_Q4_K: a.rowbytes = (uint64_t)(K / 256u) * 144u; break;
        case ENC_Q5_K: a.rowbytes = (uint64_t)(K / 256u) * 176u; break;
        case ENC_IQ4_XS: a.rowbytes = (uint64_t)(K / 256u) * 136u; break;
        default: a.rowbytes = (uint64_t)K / 2u; break;  // MLX packed words (scales and biases besides)
    }
    // M-major tile order when the staged activations (2 bytes per element)
    // outweigh the weights (M2048 N3072 K1024: 34.3 against 35.9 us per call)
    a.mmajor = (uint64_t)M * K * 2u > (uint64_t)N * a.rowbytes ? 1u : 0u;
    switch (enc) {
        case ENC_Q4_0: return launch_enc<ENC_Q4_0>(a, st);
        case ENC_Q4_1: return launch_enc<ENC_Q4_1>(a, st);
        case ENC_Q8_0: return launch_enc<ENC_Q8_0>(a, st);
        case ENC_Q6_K: return launch_enc<ENC_Q6_K>(a, st);
        case ENC_Q4_K: return launch_enc<ENC_Q4_K>(a, st);
        case ENC_Q5_K: return launch_enc<ENC_Q5_K>(a, st);
        case ENC_IQ4_XS: return launch_enc<ENC_IQ4_XS>(a, st);
        case ENC_MLX_U4: return launch_enc<ENC_MLX_U4>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dmx
