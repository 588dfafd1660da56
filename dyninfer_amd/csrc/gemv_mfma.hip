// Decode GEMV on MFMA for 3..16 activation rows, GGUF Q4_0, Q6_K, Q4_K, Q5_K
// and IQ4_XS and MLX affine U4 (y[b, o] = Σ_k x[b, k]·w[o, k], f32 accumulation;
// gguf_codegen.rs:268-314 `emit_linear` with the dequantisations of :412-472
// (Q4_0) and :474-526 (Q6_K), mlx_affine.rs:557-626 `emit_linear_u4`).
//
// The VALU GEMV multiplies every decoded weight once per activation row (a
// v_dot2 per pair per row), so above ~4 rows its VALU and LDS work grows with
// the batch while the weight stream does not.  Here the activation rows are
// one side of v_mfma_f32_16x16x32_f16 (16 rows, zero-padded) and each weight
// is decoded once, whatever the batch:
//   * a wave owns tiles of 16 weight rows (the B side: lane l holds row l % 16
//     and 8 k of the instruction's 32; the result D[b][row] leaves lane l
//     with weight row l % 16 of activation rows 4q..4q+3, q = l / 16).  A task
//     is KT weights of each row of a tile in NM = KT/32 MFMAs, lane quarter q
//     decoding a quarter of them (Q4_0: block 4t + q of task t, 128 weights a
//     task; Q6_K: quarter q of super-block t, 256 weights a task) and feeding
//     8 of its weights to each MFMA (the k slots of one MFMA may hold any k
//     as long as the activation side holds the same ones).  The 8 weights of
//     MFMA j are two runs of 4 k (run0, run1) in the pair order (r, r+2),
//     (r+1, r+3) that one v_and_or_b32 decodes: a code at mantissa bits 0..
//     under the f16 exponent of 1024 is 1024 + c, one at bits 4.. under that
//     of 64 is 64 + c, both exact; a packed add removes the offset (exact)
//     and a packed multiply by the f16 scale rounds once: Q4_0 folds its
//     block scale, RNE_f16((q-8)·d); Q6_K folds its 16-weight group's int8
//     scale, RNE_f16((q-32)·sc), and multiplies the super-block's d in f32
//     afterwards (each lane's row has one d per super-block);
//   * the activations are staged once per workgroup in LDS as f16 in the A
//     layout of each (task, j): lane (b, q) the 8 matching activations of row
//     b, scaled by a power of two per (row, task) whose largest magnitude
//     lands in [2^13, 2^14) (no overflow, no flush of the task's large values),
//     rounded once to f16; a task's MFMAs accumulate into a zeroed tile that
//     is then added to the f32 total times the inverse scale.  With a
//     workspace, a prep kernel stages them so once per call, in the LDS
//     layout, and each workgroup copies its segment by LDS DMA;
//   * weights stream coalesced: a task's bytes of the tile's 16 rows (one
//     4-byte-aligned window per row) are loaded as 16-byte pieces with
//     consecutive lanes on consecutive pieces of a row, so a load
//     instruction touches a few cache lines rather than one per lane (the
//     vector cache's tag rate, one line per clock, bounds lane-per-row
//     loads at ~3.5 TB/s), through a ring of PF tasks in registers; each
//     task's pieces then pass through a per-wave LDS window of 16 rows, from
//     which every lane reads its row's quarter in the B layout;
//   * a K range too long for LDS runs as segments in consecutive launches,
//     the later ones adding to the f32 outputs.
// Accuracy: |y - y_exact| <= (2^-11 + 2^-11 + 2^-22)·Σ|w||x| + f32 accumulation
// error (weight and activation roundings), inside the 2e-3 normalised tolerance.
#include "gemv_kernels.hpp"

namespace dmx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef half2_t h2;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t __attribute__((may_alias)) u32a;  // window dwords, written as u32x4

namespace {

constexpr int kMfmaThreads = 512;

struct MfmaParams {
    const uint8_t* w[kMaxProblems];
    uint32_t n[kMaxProblems];
    uint32_t tile_begin[kMaxProblems];  // first 16-row tile of each problem
    uint32_t total_tiles;
    uint32_t grid;        // workgroups per K segment (the launch has grid * nseg)
    uint32_t K;           // full reduction length
    uint32_t k0;          // first k of this launch's first segment
    uint32_t nunit;       // blocks (Q4_0) or super-blocks (Q6_K) over all of the launch's segments
    uint32_t seg_units;   // units per segment (the last may have fewer)
    uint32_t nseg;        // K segments in this launch: workgroup w serves segment w / grid
    uint32_t nprob;
    uint32_t batch;
    uint32_t accumulate;  // add to y (later segments; f32 outputs only)
    uint32_t x_bf16;      // activations bf16 (else f32)
    uint32_t group;       // MLX group size
    uint32_t gmagic;      // group_magic(group)
    uint32_t sdtype;      // MLX scale/bias dtype
    const void* x;
    void* y[kMaxProblems];
    const uint8_t* sc[kMaxProblems];  // MLX scales
    const uint8_t* bi[kMaxProblems];  // MLX biases
    uint32_t split_ws_log2;           // split mode: log2 of the waves per tile (3, or 2: two tiles per workgroup)
    const uint8_t* pre;               // XS_PRE: the activations staged by gemv_mfma_prep_kernel
};

// (c + off)·s for a packed pair (v_pk_add_f16, v_pk_mul_f16)
__device__ __forceinline__ uint32_t wq(uint32_t c, _Float16 off, h2 s2) {
    const h2 o = {off, off};
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, c) + o) * s2);
}

// ---- encoding policies: task shape, row windows, decode from the window
// into the NM B operands (uint4 = 4 f16 pairs) and the activation runs of
// each operand.  A task is 256 weights of each row (8 MFMAs); its row window
// starts at the task's first byte rounded down to 4 (sh = the remainder, 0 or
// 2), is loaded as NP pieces of 16 bytes, each touching only dwords that hold
// bytes of the task (so no load leaves a page the task touches), and is kept
// in LDS rows of WB bytes (WB / 16 odd: rows at distinct bank groups).

// Q4_0: a task is 8 blocks (144 bytes of a row); lane quarter q decodes
// blocks 2q and 2q + 1, MFMA j taking code dword j & 3 of block 2q + (j >> 2):
// low nibbles (4j', 4j'+2), (4j'+1, 4j'+3), high nibbles (16+4j', 18+4j'),
// (17+4j', 19+4j'), j' = j & 3.
struct MfmaQ40 {
    static constexpr int KT = 256, NM = 8, PF = 4, TPI = 2;  // weights, MFMAs per task; ring depth; tasks per step
    static constexpr uint32_t UNIT = 32, UPT = 8, UB = 18;   // weights, bytes per block; blocks per task
    static constexpr uint32_t TB = UPT * UB;                 // bytes of a row per task
    static constexpr uint32_t NP = 10, WB = 176;             // window pieces, LDS row bytes
    static constexpr bool ROWSCALE = false, MLX = false, PAIR4 = false, BIAS = false;
    static constexpr uint32_t STAGE = 8;  // staging passes per chunk of loads
    // Pieces 0..8 hold window bytes [0, 144) at LDS 16i; piece 9 is [128, 144)
    // (sh = 0) or [132, 148) (sh = 2) at LDS [144, 160), so window dword 36
    // (sh = 2 only) sits at LDS dword 39.
    __device__ static uint32_t goff(uint32_t piece, uint32_t sh) { return piece < 9u ? 16u * piece : 128u + 2u * sh; }
    __device__ static uint32_t run0(uint32_t q, uint32_t j) { return 64u * q + 32u * (j >> 2) + 4u * (j & 3u); }
    __device__ static uint32_t run1(uint32_t q, uint32_t j) { return run0(q, j) + 16u; }
    __device__ static void decode(const u32a* win, uint32_t sh, bool ok, uint32_t q, uint4 (&a)[NM], float&) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t o = sh + UB * (2u * q + (uint32_t)h), k0 = o >> 2;  // block start in the window
            uint32_t d[5];
#pragma unroll
            for (int i = 0; i < 4; i++) d[i] = win[k0 + (uint32_t)i];
            d[4] = win[k0 + 4u == 36u ? 39u : k0 + 4u];
            const uint32_t bsh = o & 3u, sel = realign_sel(bsh, 2);
            const uint32_t db = (d[0] >> (8u * bsh)) & (ok ? 0xFFFFu : 0u);  // padding task: zero weights
            const h2 d2 = __builtin_bit_cast(h2, db * 0x00010001u);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t D = __builtin_amdgcn_perm(d[j + 1], d[j], sel), D8 = D >> 8;
                a[4 * h + j] = make_uint4(wq(and_or(D, 0x000F000Fu, 0x64006400u), (_Float16)-1032.0f, d2),
                                          wq(and_or(D8, 0x000F000Fu, 0x64006400u), (_Float16)-1032.0f, d2),
                                          wq(and_or(D, 0x00F000F0u, 0x54005400u), (_Float16)-72.0f, d2),
                                          wq(and_or(D8, 0x00F000F0u, 0x54005400u), (_Float16)-72.0f, d2));
            }
        }
    }
};

// Q6_K: a task is one super-block (210 bytes of a row); lane quarter q
// decodes its chunk (n, s) = (q >> 1, q & 1): weights n·128 + 32g + 16s + i
// of groups g = 0..3, i < 16 (encodings.hpp EncQ6K, gguf_codegen.rs:499-521).
// MFMA j = 2t + h takes code dword t (i = 4t..4t+3) of groups 2h (run0) and
// 2h + 1 (run1 = run0 + 32); groups 2 and 3 hold their low bits in the high
// nibble, decoded under the exponent of 64.
struct MfmaQ6K {
    static constexpr int KT = 256, NM = 8, PF = 4, TPI = 2;
    static constexpr uint32_t UNIT = 256, UPT = 1, UB = 210;
    static constexpr uint32_t TB = UB;
    static constexpr uint32_t NP = 14, WB = 240;
    static constexpr bool ROWSCALE = true, MLX = false, PAIR4 = false, BIAS = false;
    static constexpr uint32_t STAGE = 8;
    // Pieces 0..12 hold window bytes [0, 208) at LDS 16i; piece 13 is
    // [196, 212) at LDS [208, 224), so window dword 52 (d) sits at LDS dword 55.
    __device__ static uint32_t goff(uint32_t piece, uint32_t) { return piece < 13u ? 16u * piece : 196u; }
    __device__ static uint32_t run0(uint32_t q, uint32_t j) {
        return 128u * (q >> 1) + 64u * (j & 1u) + 16u * (q & 1u) + 4u * (j >> 1);
    }
    __device__ static uint32_t run1(uint32_t q, uint32_t j) { return run0(q, j) + 32u; }
    __device__ static void decode(const u32a* win, uint32_t sh, bool ok, uint32_t q, uint4 (&a)[NM], float& d) {
        EncQ6K::Raw r;
        const uint32_t n = q >> 1, s = q & 1u;
        const uint32_t oa = (64u * n + 16u * s) >> 2, oh = (128u + 32u * n + 16u * s) >> 2;
#pragma unroll
        for (int i = 0; i < 5; i++) {
            r.a[i] = win[oa + (uint32_t)i];
            r.b[i] = win[oa + 8u + (uint32_t)i];
            r.h[i] = win[oh + (uint32_t)i];
            r.s[i] = win[i < 4 ? 48u + (uint32_t)i : 55u];  // sc[0..16), d
        }
        r.sh = sh;
        uint32_t A[4], B[4], H[4];
        EncQ6K::codes(r, A, B, H);
        int32_t sc[4];
        EncQ6K::scales(r, q, sc, d);
        d = ok ? d : 0.0f;  // padding task: zero weights
        h2 s2[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const _Float16 v = (_Float16)sc[g];  // exact: |sc| <= 128
            s2[g] = h2{v, v};
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const uint32_t a0 = A[tt], b0 = B[tt], a8 = a0 >> 8, b8 = b0 >> 8;
            const uint32_t hl4 = H[tt] << 4, hl2 = H[tt] << 2, hr4 = H[tt] >> 4, hr6 = H[tt] >> 6;
            // groups 0, 1: low nibble + qh bits (0-1 | 2-3) at mantissa bits 0..5
            a[2 * tt] =
                make_uint4(wq(and_or(a0, 0x000F000Fu, and_or(hl4, 0x00300030u, 0x64006400u)), (_Float16)-1056.0f, s2[0]),
                           wq(and_or(a8, 0x000F000Fu, and_or(hr4, 0x00300030u, 0x64006400u)), (_Float16)-1056.0f, s2[0]),
                           wq(and_or(b0, 0x000F000Fu, and_or(hl2, 0x00300030u, 0x64006400u)), (_Float16)-1056.0f, s2[1]),
                           wq(and_or(b8, 0x000F000Fu, and_or(hr6, 0x00300030u, 0x64006400u)), (_Float16)-1056.0f, s2[1]));
            // groups 2, 3: high nibble + qh bits (4-5 | 6-7) at mantissa bits 4..9
            a[2 * tt + 1] =
                make_uint4(wq(and_or(a0, 0x00F000F0u, and_or(hl4, 0x03000300u, 0x54005400u)), (_Float16)-96.0f, s2[2]),
                           wq(and_or(a8, 0x00F000F0u, and_or(hr4, 0x03000300u, 0x54005400u)), (_Float16)-96.0f, s2[2]),
                           wq(and_or(b0, 0x00F000F0u, and_or(hl2, 0x03000300u, 0x54005400u)), (_Float16)-96.0f, s2[3]),
                           wq(and_or(b8, 0x00F000F0u, and_or(hr6, 0x03000300u, 0x54005400u)), (_Float16)-96.0f, s2[3]));
        }
    }
};

// Q4_K (GGML block_q4_K; the reference's schema gguf_block.rs:183-316): a
// task is one super-block (144 bytes of a row, 4-byte aligned, so no
// realignment); lane quarter q decodes step q (encodings.hpp EncQ4K): MFMA j
// takes code dword j, the low nibbles of weights 64q + 4j.. (sub-block 2q,
// run0) and the high nibbles of 64q + 32 + 4j.. (sub-block 2q + 1, run1).
// w = d·(sc·q) - dmin·m: the B operand is sc·q (exact in f16, <= 945) and d
// multiplies the task's product per weight row in f32; the offsets take a
// ninth MFMA (BIAS): B holds 32·m of the lane's two sub-blocks in k slots
// 8q, 8q + 1 (exact), A the matching activation sums X/32 of each row
// (staged with the activations, one f16 rounding), and that product is
// subtracted times dmin.
// Q5_K (block_q5_K, 176 bytes, gguf_block.rs:183-316 "q5_k") decodes the
// same way with 5-bit codes: the fifth bit, bit 2q + h of qh[l] (window
// dwords 4..11), moved under the nibble (sc·q <= 1953, still exact).
template <bool Q5>
struct MfmaQK {
    static constexpr int KT = 256, NM = 8, PF = 4, TPI = 2;
    static constexpr uint32_t UNIT = 256, UPT = 1, UB = Q5 ? 176u : 144u;
    static constexpr uint32_t TB = UB;
    static constexpr uint32_t NP = UB / 16u, WB = UB;  // 9 or 11 pieces: odd
    static constexpr uint32_t QS = Q5 ? 12u : 4u;      // window dword of the codes
    static constexpr bool ROWSCALE = false, MLX = false, PAIR4 = false, BIAS = true;
    static constexpr uint32_t STAGE = 8;
    __device__ static uint32_t goff(uint32_t piece, uint32_t) { return 16u * piece; }
    __device__ static uint32_t run0(uint32_t q, uint32_t j) { return 64u * q + 4u * j; }
    __device__ static uint32_t run1(uint32_t q, uint32_t j) { return run0(q, j) + 32u; }
    // mb = the f16 pair (32·m_2q, 32·m_2q+1); d, dmin zero for a padding task
    __device__ static void decode(const u32a* win, bool ok, uint32_t q, uint4 (&a)[NM], uint32_t& mb, float& d,
                                  float& dmin) {
        const uint32_t h0 = win[0];
        uint32_t sc[2], mn[2];
        q4k_scale_min_pair(win[1], win[2], win[3], q, sc, mn);
        d = ok ? f16_bits_to_f32(h0) : 0.0f;
        dmin = ok ? f16_bits_to_f32(h0 >> 16) : 0.0f;
        const _Float16 s0 = (_Float16)sc[0], s1 = (_Float16)sc[1];  // exact: < 64
        const h2 s2lo = {s0, s0}, s2hi = {s1, s1};
        mb = __builtin_bit_cast(uint32_t, h2{(_Float16)(32u * mn[0]), (_Float16)(32u * mn[1])});  // exact: <= 2016
#pragma unroll
        for (int j = 0; j < NM; j++) {
            const uint32_t D = win[QS + 8u * q + (uint32_t)j], D8 = D >> 8;
            uint32_t ml = 0x64006400u, mh = 0x54005400u, ml8 = ml, mh8 = mh;
            if constexpr (Q5) {
                const uint32_t H = win[4u + (uint32_t)j] >> (2u * q), H8 = H >> 8;
                ml = and_or(H << 4, 0x00100010u, ml);
                mh = and_or(H << 7, 0x01000100u, mh);
                ml8 = and_or(H8 << 4, 0x00100010u, ml8);
                mh8 = and_or(H8 << 7, 0x01000100u, mh8);
            }
            a[j] = make_uint4(wq(and_or(D, 0x000F000Fu, ml), (_Float16)-1024.0f, s2lo),
                              wq(and_or(D8, 0x000F000Fu, ml8), (_Float16)-1024.0f, s2lo),
                              wq(and_or(D, 0x00F000F0u, mh), (_Float16)-64.0f, s2hi),
                              wq(and_or(D8, 0x00F000F0u, mh8), (_Float16)-64.0f, s2hi));
        }
    }
};
using MfmaQ4K = MfmaQK<false>;
using MfmaQ5K = MfmaQK<true>;

// IQ4_XS (GGML block_iq4_xs, 136 bytes; gguf_block.rs:183-316 "iq4_xs"): a
// task is one super-block; lane quarter q decodes sub-blocks 2q and 2q + 1,
// laid out as Q4_0 blocks (MFMA j: code dword j & 3 of sub-block 2q + (j >> 2),
// low nibbles run0, high nibbles run1), each index looked up in the codebook
// (iq4nl_lookup) and decoded as Q8_0's codes: B = RNE_f16(kv·(ls - 32)), the
// super-block's d multiplied per weight row in f32 (ROWSCALE).  The window:
// pieces 0..7 hold bytes [0, 128), piece 8 bytes [120, 136) at LDS
// [128, 144), so window dwords 32 and 33 sit at LDS dwords 34 and 35.
struct MfmaIQ4XS {
    static constexpr int KT = 256, NM = 8, PF = 4, TPI = 2;
    static constexpr uint32_t UNIT = 256, UPT = 1, UB = 136;
    static constexpr uint32_t TB = UB;
    static constexpr uint32_t NP = 9, WB = 144;
    static constexpr bool ROWSCALE = true, MLX = false, PAIR4 = false, BIAS = false;
    static constexpr uint32_t STAGE = 8;
    __device__ static uint32_t goff(uint32_t piece, uint32_t) { return piece < 8u ? 16u * piece : 120u; }
    __device__ static uint32_t run0(uint32_t q, uint32_t j) { return 64u * q + 32u * (j >> 2) + 4u * (j & 3u); }
    __device__ static uint32_t run1(uint32_t q, uint32_t j) { return run0(q, j) + 16u; }
    __device__ static void decode(const u32a* win, uint32_t, bool ok, uint32_t q, uint4 (&a)[NM], float& d) {
        const uint32_t h0 = win[0], h1 = win[1];
        d = ok ? f16_bits_to_f32(h0) : 0.0f;  // padding task: zero weights
        const h2 o = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t ib = 2u * q + (uint32_t)h;
            const _Float16 sv = (_Float16)((int)iq4xs_scale(h0 >> 16, h1, ib) - 32);  // exact
            const h2 s2 = {sv, sv};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t k = 2u + 4u * ib + (uint32_t)j;  // window dword of the code dword
                const uint32_t Q = win[k < 32u ? k : k + 2u];
                const uint32_t L = iq4nl_lookup(Q & 0x0F0F0F0Fu), H = iq4nl_lookup((Q >> 4) & 0x0F0F0F0Fu);
                a[4 * h + j] = make_uint4(__builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, and_or(L, 0x00FF00FFu, 0x64006400u)) + o) * s2),
                                          __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, and_or(L >> 8, 0x00FF00FFu, 0x64006400u)) + o) * s2),
                                          __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, and_or(H, 0x00FF00FFu, 0x64006400u)) + o) * s2),
                                          __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, and_or(H >> 8, 0x00FF00FFu, 0x64006400u)) + o) * s2));
            }
        }
    }
};

// MLX affine U4 (mlx_affine.rs:557-626, fixture.rs:307-311): a task is 256
// weights of a row, 32 packed words (128 bytes, 16-byte aligned rows, so no
// realignment); lane quarter q decodes words 8q..8q+7 (k 64q..64q+63), MFMA j
// taking word j: nibbles (0,4), (1,5), (2,6), (3,7), i.e. the activation pairs
// (r, r+4) of one run of 8.  w = q·s + b with the group's scale and bias:
// q exact in f16, one fused packed multiply-add rounds once, RNE_f16(q·s + b)
// (bf16 and f16 scales and biases are exact in f16's normal range).
struct MfmaMlxU4 {
    static constexpr int KT = 256, NM = 8, PF = 4, TPI = 2;
    static constexpr uint32_t UNIT = 256, UPT = 1, UB = 128;
    static constexpr uint32_t TB = UB;
    static constexpr uint32_t NP = 8, WB = 144;
    static constexpr bool ROWSCALE = false, MLX = true, PAIR4 = true, BIAS = false;
    static constexpr uint32_t STAGE = 8;
    __device__ static uint32_t goff(uint32_t piece, uint32_t) { return 16u * piece; }
    __device__ static uint32_t run0(uint32_t q, uint32_t j) { return 64u * q + 8u * j; }
    __device__ static uint32_t run1(uint32_t q, uint32_t j) { return run0(q, j) + 4u; }
    // a scale or bias bit pattern (f32, or f16/bf16 in the low half) to f16
    // (all three formed and one selected: the dtype is uniform, and a branch per
    // value put 36 uniform branches in each round of four tasks)
    __device__ static _Float16 sb_f16(uint32_t bits, uint32_t sdtype) {
        const _Float16 f32v = (_Float16)__uint_as_float(bits);
        const _Float16 f16v = __builtin_bit_cast(_Float16, (uint16_t)bits);
        const _Float16 bf16v = (_Float16)__uint_as_float(bits << 16);
        const uint16_t r = sdtype == DT_F32 ? __builtin_bit_cast(uint16_t, f32v)
                         : sdtype == DT_F16 ? __builtin_bit_cast(uint16_t, f16v)
                                            : __builtin_bit_cast(uint16_t, bf16v);
        return __builtin_bit_cast(_Float16, r);
    }
    // aux = (s, b) of the group of words 0..3 and of words 4..7
    __device__ static void decode(const u32a* win, uint32_t q, const uint32_t (&aux)[4], uint32_t sdtype,
                                  uint4 (&a)[NM]) {
        const _Float16 s0 = sb_f16(aux[0], sdtype), b0 = sb_f16(aux[1], sdtype);
        const _Float16 s1 = sb_f16(aux[2], sdtype), b1 = sb_f16(aux[3], sdtype);
        const h2 o1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f}, o64 = {(_Float16)-64.0f, (_Float16)-64.0f};
#pragma unroll
        for (int j = 0; j < NM; j++) {
            const uint32_t w = win[8u * q + (uint32_t)j], w8 = w >> 8;
            const h2 s2 = j < 4 ? h2{s0, s0} : h2{s1, s1}, b2 = j < 4 ? h2{b0, b0} : h2{b1, b1};
            auto wq = [&](uint32_t c, h2 o) {
                return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, c) + o, s2, b2));
            };
            a[j] = make_uint4(wq(and_or(w, 0x000F000Fu, 0x64006400u), o1024),   // nibbles 0, 4
                              wq(and_or(w, 0x00F000F0u, 0x54005400u), o64),     // 1, 5
                              wq(and_or(w8, 0x000F000Fu, 0x64006400u), o1024),  // 2, 6
                              wq(and_or(w8, 0x00F000F0u, 0x54005400u), o64));   // 3, 7
        }
    }
};

// LDS (real tasks only): activations [task][j][64 lanes] x 16 bytes, the
// inverse scales [task][16 rows] f32, for BIAS encodings the activation sums
// [task][16 rows][4 quarters] as f16 pairs, then each wave's window of 16 rows
// x WB bytes.  Tasks
// of a segment are padded to a multiple of PF (the padding tasks have zero
// weights and activations).
// Split mode (few tiles): the ws = 8 (or 4) waves of a group share each tile,
// wave w of the group taking tasks [w·T/ws, (w+1)·T/ws) with a ring of 2, so
// T is a multiple of 2·ws.
template <class M, bool SPLIT>
__host__ __device__ constexpr uint32_t mfma_tasks(uint32_t nunit, uint32_t ws) {
    const uint32_t pad = SPLIT ? 2u * ws : (uint32_t)M::PF;
    return ((nunit + M::UPT - 1u) / M::UPT + pad - 1u) / pad * pad;
}
template <class M>
__host__ __device__ constexpr uint32_t mfma_task_lds() {
    return M::NM * 64u * 16u + 64u + (M::BIAS ? 256u : 0u);
}
// LDS of a segment of nunit units: the real tasks only (padding tasks are
// neither staged nor multiplied), then the windows.
template <class M, bool SPLIT>
__host__ __device__ constexpr uint32_t mfma_lds_bytes(uint32_t nunit) {
    return (nunit + M::UPT - 1u) / M::UPT * mfma_task_lds<M>() + (kMfmaThreads / 64u) * 16u * M::WB;
}

// Slot of A-operand lane l (row b = l % 16, quarter q = l / 16) in the 64
// slots of 16 bytes of one (task, j): l with its low three bits XORed by
// (j + 4·(q & 1)) & 7.  A bijection within each 16-lane quarter, so a
// fragment read (64 lanes, slots l) stays conflict-free, while the staging
// threads of one (task, row) spread their writes over the LDS bank groups.
__device__ __forceinline__ uint32_t xslot(uint32_t l, uint32_t j) { return l ^ ((j + 4u * ((l >> 4) & 1u)) & 7u); }

// The staged form of one unit, the 8 activations v of activation row b for MFMA
// j of lane quarter q of a task: its f16 pairs in the B-operand order, the
// (task, row)'s inverse scale and, for the offset encodings, the quarter's
// scaled sums.  The 32 units of a (task, row) sit on 32 aligned consecutive
// lanes, which all call this together: the maximum (DPP within rows of 16
// lanes, v_permlane16_swap across two) and the quarter sums (8 lanes) are
// cross-lane.
struct Staged {
    uint4 val;
    float inv;
    uint32_t xs;
};
template <class M>
__device__ __forceinline__ Staged stage_unit(const float (&v)[8]) {
    float mv = absmax3(v[0], v[1], v[2]);
    mv = absmax3(mv, v[3], v[4]);
    mv = absmax3(mv, v[5], v[6]);
    mv = absmax3(mv, v[7], v[7]);
    uint32_t mx = __float_as_uint(mv);  // non-negative floats order as integers
    mx = lanes_reduce<8>(mx, [](uint32_t a, uint32_t c) { return a > c ? a : c; });
    mx = max(mx, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x140, 0xF, 0xF, false));  // row_mirror: 16 lanes
    {  // and the neighbouring row of 16
        const auto r = __builtin_amdgcn_permlane16_swap(mx, mx, false, false);
        mx = max(r[0], r[1]);
    }
    int ex = 0;
    (void)frexpf(__uint_as_float(mx), &ex);
    ex = ex < -110 ? -110 : ex;  // keeps the scale a normal f32
    const int sh = 14 - ex;      // largest magnitude / 2^(ex-14) < 2^14
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    auto pk = [&](float a, float c) {
        const f32x2 f = {ldexpf(a, sh), ldexpf(c, sh)};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));  // RNE
    };
    Staged st;
    // pair order: (r, r+2) (r+1, r+3) of each run, or (r, r+4) ... (r+3, r+7)
    // of one run of 8 (MLX words)
    st.val = M::PAIR4 ? make_uint4(pk(v[0], v[4]), pk(v[1], v[5]), pk(v[2], v[6]), pk(v[3], v[7]))
                      : make_uint4(pk(v[0], v[2]), pk(v[1], v[3]), pk(v[4], v[6]), pk(v[5], v[7]));
    st.inv = ldexpf(1.0f, -sh);
    st.xs = 0u;
    if constexpr (M::BIAS) {
        // the unit's two runs summed as stored (f16 values, exact in f32
        // but for the last bits of 32-term sums), over the NM units of
        // its quarter (8 consecutive lanes), stored / 32 as f16 (below
        // 2^14) for the offset MFMA
        const uint32_t one2 = 0x3C003C00u;
        float s0 = dot2(st.val.x, one2, dot2(st.val.y, one2, 0.0f)), s1 = dot2(st.val.z, one2, dot2(st.val.w, one2, 0.0f));
        auto fadd = [](uint32_t a, uint32_t c) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(c)); };
        s0 = __uint_as_float(lanes_reduce<8>(__float_as_uint(s0), fadd));
        s1 = __uint_as_float(lanes_reduce<8>(__float_as_uint(s1), fadd));
        const f32x2 f = {s0 * 0.03125f, s1 * 0.03125f};
        st.xs = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));
    }
    return st;
}

// The staged activations of a whole call in device memory (the caller's
// workspace), laid out as one workgroup's LDS holds a segment: the fragments
// of every task of K, then the inverse scales of every (task, row), then (for
// the offset encodings) the quarter sums; a segment's tasks are a contiguous
// range of each part.
template <class M>
__host__ __device__ constexpr uint64_t mfma_prestage_bytes(uint32_t K) {
    return (uint64_t)(K / M::KT) * mfma_task_lds<M>();
}

}  // namespace

// The kernel arguments the set-up reads, made operands of empty asm statements
// at the kernel's top so the compiler loads them together rather than each
// behind a wait for the one before (as the VALU GEMV's gemv_args_up_front).
template <bool MLX>
__device__ __forceinline__ void mfma_args_up_front(const MfmaParams& p) {
    asm volatile("" ::"s"(p.w[0]), "s"(p.w[1]), "s"(p.w[2]), "s"(p.w[3]), "s"(p.y[0]), "s"(p.y[1]), "s"(p.y[2]),
                 "s"(p.y[3]), "s"(p.x), "s"(p.pre));
    asm volatile("" ::"s"(p.n[0]), "s"(p.n[1]), "s"(p.n[2]), "s"(p.n[3]), "s"(p.tile_begin[0]), "s"(p.tile_begin[1]),
                 "s"(p.tile_begin[2]), "s"(p.tile_begin[3]), "s"(p.total_tiles), "s"(p.grid), "s"(p.K), "s"(p.k0),
                 "s"(p.nunit), "s"(p.seg_units), "s"(p.nseg), "s"(p.nprob), "s"(p.batch), "s"(p.split_ws_log2));
    if constexpr (MLX)
        asm volatile("" ::"s"(p.sc[0]), "s"(p.sc[1]), "s"(p.sc[2]), "s"(p.sc[3]), "s"(p.bi[0]), "s"(p.bi[1]),
                     "s"(p.bi[2]), "s"(p.bi[3]), "s"(p.group), "s"(p.gmagic), "s"(p.sdtype));
}

// How a workgroup gets the segment's activations: it stages them in LDS
// itself, the batch being 3..8 (4 or 8 rows of the A side staged) or 9..16
// (all 16 rows, the staging indices compile-time), or it copies them into LDS
// from the call's workspace, where gemv_mfma_prep_kernel staged them once for
// all workgroups (XS_PRE), or (split mode, eight waves per tile, two tasks per
// wave: XS_REG) each wave loads its own two tasks' operands from the workspace
// into registers, which serve every tile it takes, and LDS holds only the
// weight windows.
enum MfmaStaging { XS_ROWS8 = 0, XS_ROWS16 = 1, XS_PRE = 2, XS_REG = 3 };

template <class M, bool YBF16, bool SPLIT, int XS>
__global__ __launch_bounds__(kMfmaThreads) void gemv_mfma_kernel(const MfmaParams p) {
    constexpr bool ROWS16 = XS == XS_ROWS16, REG = XS == XS_REG;
    static_assert(!REG || SPLIT, "register operands serve the split mode's fixed tasks per wave");
    extern __shared__ __align__(16) uint8_t lds[];
    mfma_args_up_front<M::MLX>(p);
    constexpr uint32_t NM = M::NM, UPR = 4u * NM;  // staging units per (task, row): (q, j)
    constexpr uint32_t NSLOT = 16u * M::NP, NLD = (NSLOT + 63u) / 64u;  // window pieces, loads per lane
    constexpr int PF = SPLIT ? 2 : M::PF;  // tasks of raw loads in flight per wave
    constexpr uint32_t NW = kMfmaThreads / 64u;
    // this workgroup's K segment: units [sidx·seg_units, ...) of the launch's range
    const uint32_t sidx = p.nseg > 1u ? blockIdx.x / p.grid : 0u, bid = blockIdx.x - sidx * p.grid;
    const uint32_t k0 = p.k0 + sidx * p.seg_units * M::UNIT;
    const uint32_t nunit = p.nunit - sidx * p.seg_units < p.seg_units ? p.nunit - sidx * p.seg_units : p.seg_units;
    const uint32_t wsl = SPLIT ? p.split_ws_log2 : 0u, ws = 1u << wsl;  // waves per tile in split mode
    const uint32_t ng = mfma_tasks<M, SPLIT>(nunit, ws), nt = nunit / M::UPT;  // tasks with padding, without
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    if constexpr (XS == XS_PRE) {
        // The segment's staged tasks are one contiguous range of the workspace,
        // laid out as LDS holds them: copied by LDS DMA, 1 KiB per wave
        // instruction (the last one partial), issued before the tile set-up
        // (whose kernel-argument loads then overlap the copies).  Copying only
        // the staged rows' slots of each fragment chunk, half of them at 5..8
        // rows, measured slower: a per-lane test per instruction.
        constexpr uint32_t TL = mfma_task_lds<M>();
        const uint8_t* src = p.pre + (size_t)sidx * (p.seg_units / M::UPT) * TL;
        const uint32_t bytes = nt * TL, nch = (bytes + 1023u) / 1024u;
        for (uint32_t c = wv; c < nch; c += NW)
            if (c * 1024u + 16u * lane < bytes) dma16(src + c * 1024u + 16u * lane, lds + c * 1024u);
        __builtin_amdgcn_sched_barrier(0);
    }
    uint4* xl = reinterpret_cast<uint4*>(lds);
    float* inv = reinterpret_cast<float*>(lds + nt * NM * 64u * 16u);
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds + nt * (NM * 64u * 16u + 64u));  // BIAS: activation sums
    uint8_t* wins = lds + (REG ? 0u : nt * mfma_task_lds<M>());  // the waves' windows
    uint8_t* win = wins + wv * 16u * M::WB;             // this wave's window

    // ---- weight tiles.  Whole tiles per wave: wave wid takes tiles wid,
    // wid + W, ..., waves numbered across workgroups first (wave i of
    // workgroup w is wid = i·grid + w), so a few tiles still spread over all
    // CUs.  Split mode: the workgroup's waves form NW/ws groups of ws; group gi
    // of workgroup w takes tiles w + gi·grid, ... (groups across workgroups
    // first), and its waves split each tile's tasks (wave v of the group:
    // tasks t0 = v·tpw .. t0 + tpw - 1).  Every wave of a workgroup runs the
    // tile count of its group 0 (the most), so all pass the same barriers;
    // a group past its own tiles recomputes its last one and stores nothing.
    const uint32_t gi = SPLIT ? wv >> wsl : 0u, wg = SPLIT ? wv & (ws - 1u) : wv;
    const uint32_t wid = SPLIT ? bid + gi * p.grid : __builtin_amdgcn_readfirstlane(wv * p.grid + bid);
    const uint32_t W = SPLIT ? p.grid * (NW >> wsl) : p.grid * NW;
    const uint32_t tpw = SPLIT ? ng >> wsl : ng, t0 = SPLIT ? wg * tpw : 0u;
    const uint32_t m = lane & 15u, q = lane >> 4;
    const uint32_t ntw = wid < p.total_tiles ? (p.total_tiles - wid + W - 1u) / W : 0u;  // tiles of this wave
    const uint32_t nloop = SPLIT ? (bid < p.total_tiles ? (p.total_tiles - bid + W - 1u) / W : 0u) : ntw;
    const uint32_t rowbytes = (p.K / M::UNIT) * M::UB, seg0 = (k0 / M::UNIT) * M::UB;

    // the wave's i-th tile (past the end: its last, or any tile for a wave
    // without tiles: loaded, never multiplied into a stored result)
    auto tile_at = [&](uint32_t i) {
        const uint32_t ii = i < ntw ? i : (ntw ? ntw - 1u : 0u);
        const uint32_t tile = wid + ii * W;
        return tile < p.total_tiles ? tile : p.total_tiles - 1u;
    };
    struct Where {
        const uint8_t* w;
        const uint8_t* sc;
        const uint8_t* bi;
        void* y;
        uint32_t n, row0;
    };
    auto where = [&](uint32_t tile) {
        uint32_t pi = 0;
#pragma unroll
        for (int i = 1; i < kMaxProblems; i++) pi += ((uint32_t)i < p.nprob && tile >= p.tile_begin[i]) ? 1u : 0u;
        Where r;
        r.w = pick(pi, p.w);
        if constexpr (M::MLX) {
            r.sc = pick(pi, p.sc);
            r.bi = pick(pi, p.bi);
        }
        r.y = pick(pi, p.y);
        r.n = pick(pi, p.n);
        r.row0 = (tile - pick(pi, p.tile_begin)) * 16u;
        return r;
    };
    // Window pieces of this lane: piece slot 64i + lane (the slots past the
    // last re-load it) is piece pc[i] of tile row pr[i], stored at LDS
    // lo[i] of the window.
    uint32_t pr[NLD], pc[NLD], lo[NLD];
#pragma unroll
    for (uint32_t i = 0; i < NLD; i++) {
        const uint32_t sl = 64u * i + lane < NSLOT ? 64u * i + lane : NSLOT - 1u;
        pr[i] = sl / M::NP;
        pc[i] = sl % M::NP;
        lo[i] = pr[i] * M::WB + 16u * pc[i];
    }
    // a tile's 4-byte-aligned weight base and the byte offsets (from it) of
    // the segment's start in this lane's decode row (om) and load rows (oi;
    // for tasks a multiple of 4 bytes long, oi is already the offset of the
    // lane's piece in the segment's first task); rows past the problem
    // re-read its last one: in bounds, never stored
    struct Rows {
        const uint8_t* abase;
        const uint8_t* sc;
        const uint8_t* bi;
        uint32_t om, rowm;
        uint32_t oi[NLD];
    };
    auto rows_of = [&](const Where& wh) {
        const uint32_t bsh = (uint32_t)((uintptr_t)wh.w & 3u);
        auto row = [&](uint32_t r) { return wh.row0 + r < wh.n ? wh.row0 + r : wh.n - 1u; };
        auto off = [&](uint32_t r) { return row(r) * rowbytes + bsh + seg0; };
        Rows r;
        r.abase = wh.w - bsh;
        if constexpr (M::MLX) {
            r.sc = wh.sc;
            r.bi = wh.bi;
            r.rowm = row(m);
        }
        r.om = off(m);
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) {
            const uint32_t o = off(pr[i]);
            // tasks a multiple of 4 bytes long: the piece's offset within its task is the same in every task
            r.oi[i] = M::TB % 4u == 0u ? (o & ~3u) + M::goff(pc[i], o & 3u) : o;
        }
        return r;
    };
    // task t's window start from a row's segment offset (padding tasks
    // re-read the last task)
    auto task_off = [&](uint32_t o, uint32_t t) { return o + (t < nt ? t : nt - 1u) * M::TB; };
    // MLX scales and biases of the lane's row: the dword holding each value
    // (bits shifted down for 16-bit types; it holds a byte of the value, so
    // it stays in the value's page)
    const uint32_t es = p.sdtype == DT_F32 ? 4u : 2u, gpr = p.K / (p.group ? p.group : 1u);
    // (the raw dword: the 16-bit value is shifted out where it is used, so a
    // refill load is not waited for at its issue)
    auto sbload = [&](const uint8_t* base, uint32_t idx) { return *gptr<uint32_t>(base + ((idx * es) & ~3u)); };
    // the scale/bias groups of task t for this lane: k 64q..64q+31 and 64q+32..64q+63
    auto sbgroups = [&](const Rows& r, uint32_t t, uint32_t& g0, uint32_t& g1) {
        const uint32_t kl = k0 + (t < nt ? t : nt - 1u) * M::KT + 64u * q;
        g0 = r.rowm * gpr + div_magic(kl, p.gmagic);
        g1 = r.rowm * gpr + div_magic(kl + 32u, p.gmagic);
    };
    auto load = [&](const Rows& r, uint32_t t, u32x4 (&v)[NLD], uint32_t (&aux)[4]) {
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) {
            // one 32-bit offset from a wave-uniform base (every piece starts
            // inside the tensor, below 4 GiB): no per-lane 64-bit address add
            if constexpr (M::TB % 4u == 0u) {
                v[i] = *gptr<u32x4>(r.abase + (t < nt ? t : nt - 1u) * M::TB + r.oi[i]);
            } else {
                const uint32_t o = task_off(r.oi[i], t);
                v[i] = *gptr<u32x4>(r.abase + ((o & ~3u) + M::goff(pc[i], o & 3u)));
            }
        }
        if constexpr (M::MLX) {
            uint32_t g0, g1;
            sbgroups(r, t, g0, g1);
            aux[0] = sbload(r.sc, g0);
            aux[1] = sbload(r.bi, g0);
            aux[2] = sbload(r.sc, g1);
            aux[3] = sbload(r.bi, g1);
        }
    };
    // ---- stage the activations: unit u = (task g, row b, e = q·NM + j); the
    // 32 units of (g, b) lie on consecutive lanes, their maximum reduced by
    // DPP within rows of 16 lanes and v_permlane16_swap across two.  Chunks
    // of passes: all of a chunk's loads leave before the first is converted.
    // only the segment's real tasks (padding tasks are never multiplied) and
    // the batch's rows rounded up to RB = 4, 8 or 16: rows RB..15 of the
    // MFMA's A side are never staged, and whatever bits their LDS slots hold
    // reach only output rows that are never stored (each output row reads its
    // own activation row).  Per step, the Qwen3-8B GGUF batch 4: 2.29 ->
    // 2.19 ms, batch 8: 3.07 -> 2.73 ms.  Zero-filling those rows first (all
    // slots, then a barrier on the LDS writes) cost more than it saved: 2.23
    // and 2.94 ms.
    const uint32_t rbl = ROWS16 ? 4u : p.batch <= 4u ? 2u : 3u;  // log2 RB
    const uint32_t nunits = nt * (UPR << rbl), npass = (nunits + kMfmaThreads - 1u) / kMfmaThreads;
    // unit u = pass·512 + tid: task g = pass·(16/RB) + tid / (32·RB), row
    // b = (tid / 32) % RB (a constant of the thread), e = tid % 32
    static_assert(kMfmaThreads == 16u * 32u, "a pass is 16 (task, row) pairs of 32 units");
    const uint32_t tg = tid >> (5u + rbl), tb = (tid >> 5u) & ((1u << rbl) - 1u), gstep = 16u >> rbl;
    // A unit's raw activations, loaded unconditionally (a unit past the tasks
    // or the batch reads row 0, in bounds, and stages zeros): a load under a
    // per-lane branch would make its wave wait for it where the branch joins,
    // before the weight loads that follow are issued.
    struct XRaw {
        uint32_t w[8];  // bf16: two runs of 4 in w[0..3]; f32: w[0..7]
        bool ok;
    };
    auto xload = [&](auto xb, uint32_t pass, XRaw& r) {
        constexpr bool XB = decltype(xb)::value;
        const uint32_t u = pass * kMfmaThreads + tid;
        const uint32_t g = ROWS16 ? u / (16u * UPR) : pass * gstep + tg, b = ROWS16 ? (u / UPR) % 16u : tb;
        const uint32_t e = u % UPR, qq = e / NM, j = e % NM;
        r.ok = u < nunits && b < p.batch && g < nt;
        const size_t xk0 = r.ok ? (size_t)b * p.K + k0 + M::KT * g : 0u;
        if constexpr (XB) {  // two runs of 4 bf16: 8 bytes each
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const uint16_t* xr = static_cast<const uint16_t*>(p.x) + xk0;
            const u32x2 lo2 = *gptr<u32x2>(xr + M::run0(qq, j)), hi2 = *gptr<u32x2>(xr + M::run1(qq, j));
            r.w[0] = lo2[0];
            r.w[1] = lo2[1];
            r.w[2] = hi2[0];
            r.w[3] = hi2[1];
        } else {
            const float* xr = static_cast<const float*>(p.x) + xk0;
            const f32x4 lo4 = *gptr<f32x4>(xr + M::run0(qq, j)), hi4 = *gptr<f32x4>(xr + M::run1(qq, j));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                r.w[i] = __float_as_uint(lo4[i]);
                r.w[4 + i] = __float_as_uint(hi4[i]);
            }
        }
    };
    // the unit's 8 activations as f32 (zeros for a unit staged as padding)
    auto xvals = [&](auto xb, const XRaw& r, float (&v)[8]) {
        if constexpr (decltype(xb)::value) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                v[2 * i] = __uint_as_float(r.w[i] << 16);
                v[2 * i + 1] = __uint_as_float(r.w[i] & 0xFFFF0000u);
                v[4 + 2 * i] = __uint_as_float(r.w[2 + i] << 16);
                v[5 + 2 * i] = __uint_as_float(r.w[2 + i] & 0xFFFF0000u);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = __uint_as_float(r.w[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = r.ok ? v[i] : 0.0f;
    };
    auto xstore = [&](uint32_t pass, const float (&v)[8]) {
        const uint32_t u = pass * kMfmaThreads + tid;
        const uint32_t g = ROWS16 ? u / (16u * UPR) : pass * gstep + tg, b = ROWS16 ? (u / UPR) % 16u : tb;
        const uint32_t e = u % UPR, qq = e / NM, j = e % NM;
        const Staged st = stage_unit<M>(v);
        if (u < nunits) {
            xl[(g * NM + j) * 64u + xslot(b + 16u * qq, j)] = st.val;
            if (e == 0) inv[g * 16u + b] = st.inv;
            if (M::BIAS && j == 0) xs[(g * 16u + b) * 4u + qq] = st.xs;
        }
    };
    static_assert(UPR == 32, "a (task, row) spans two rows of 16 lanes");
    // 16 rows: chunks of 4 passes (per step, Qwen3-8B GGUF at 16 rows 3.23 ms
    // with chunks of 8, 3.13 with 4, 3.22 with 2 and 6, 3.41 with 16; the
    // MLX step 1126 -> 1095 us); 4 and 8 rows keep M::STAGE (4 cost 3% at 8)
    constexpr uint32_t kStageChunk = ROWS16 ? 4u : M::STAGE;
    // The first chunk's activation loads leave first, then the first PF
    // tasks' weight loads: loads complete in issue order, so the staging
    // converts while the weights are in flight (weights first made every wave
    // wait for its weights before its first conversion: 1024x2048 MLX at 16
    // rows staged in 4.0 us).
    Where wcur = where(tile_at(0u));
    Rows rcur = rows_of(wcur);
    u32x4 ring[PF][NLD];
    uint32_t rx[PF][4];
    // one copy of the staging per activation dtype (a dtype test per load
    // would join its two arms, and wait for the loads, at every unit)
    auto stage = [&](auto xb) {
        {
            XRaw r[kStageChunk];
#pragma unroll
            for (uint32_t i = 0; i < kStageChunk; i++) xload(xb, i < npass ? i : npass - 1u, r[i]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < PF; s++) load(rcur, t0 + (uint32_t)s, ring[s], rx[s]);  // tpw >= PF: all in tile 0
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (uint32_t i = 0; i < kStageChunk; i++) {
                float v[8];
                xvals(xb, r[i], v);
                if (i < npass) xstore(i, v);
            }
        }
        for (uint32_t c0 = kStageChunk; c0 < npass; c0 += kStageChunk) {
            XRaw r[kStageChunk];
#pragma unroll
            for (uint32_t i = 0; i < kStageChunk; i++) xload(xb, c0 + i < npass ? c0 + i : npass - 1u, r[i]);
#pragma unroll
            for (uint32_t i = 0; i < kStageChunk; i++) {
                float v[8];
                xvals(xb, r[i], v);
                if (c0 + i < npass) xstore(c0 + i, v);
            }
        }
    };
    // XS_REG: the wave's tasks t0, t0 + 1 (every tile's), their fragments in
    // the A layout, inverse scales of rows 4q..4q+3 and (offset encodings)
    // the quarter sums, as the workspace holds them (padding tasks read the
    // last real task: in bounds, never multiplied)
    u32x4 xreg[REG ? PF : 1][NM];
    f32x4 ireg[REG ? PF : 1];
    uint32_t sreg[REG ? PF : 1];
    if constexpr (REG) {
        constexpr uint32_t TL = mfma_task_lds<M>();
        const uint8_t* seg = p.pre + (size_t)sidx * (p.seg_units / M::UPT) * TL;
#pragma unroll
        for (int s = 0; s < PF; s++) {
            const uint32_t t = t0 + (uint32_t)s, tc = t < nt ? t : nt - 1u;
#pragma unroll
            for (uint32_t j = 0; j < NM; j++) xreg[s][j] = *gptr<u32x4>(seg + ((tc * NM + j) * 64u + xslot(lane, j)) * 16u);
            ireg[s] = *gptr<f32x4>(seg + nt * NM * 1024u + (tc * 16u + 4u * q) * 4u);
            if constexpr (M::BIAS) sreg[s] = *gptr<uint32_t>(seg + nt * (NM * 1024u + 64u) + ((tc * 16u + m) * 4u + q) * 4u);
        }
#pragma unroll
        for (int s = 0; s < PF; s++) load(rcur, t0 + (uint32_t)s, ring[s], rx[s]);
    } else if constexpr (XS == XS_PRE) {
        // the copies (issued at the top) and then the first PF tasks' weight
        // loads are in flight; the wait before the barrier covers the copies
        // only (loads complete in issue order), so the weights stay in flight
#pragma unroll
        for (int s = 0; s < PF; s++) load(rcur, t0 + (uint32_t)s, ring[s], rx[s]);
        __builtin_amdgcn_sched_barrier(0);
        ring_barrier<(uint32_t)PF * (NLD + (M::MLX ? 4u : 0u))>();  // (__syncthreads would wait for all loads)
    } else {
        if (p.x_bf16) stage(std::true_type{});
        else stage(std::false_type{});
        __syncthreads();
    }

    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc = zero;
    // One task's product: its pieces into the wave's window (a wave's LDS
    // accesses complete in order, so the reads below see them and the next
    // task's writes wait for these reads), the lane's quarter decoded from
    // its row, and the task's MFMAs into a zeroed tile; rs = the row scale
    // (Q6_K's d).
    auto product = [&](const u32x4 (&v)[NLD], const uint32_t (&aux)[4], const Rows& r, uint32_t t, float& rs,
                       const u32x4 (&xr)[NM], uint32_t xsr) {
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) *reinterpret_cast<u32x4*>(win + lo[i]) = v[i];
        u32x4 xa[NM];
#pragma unroll
        for (uint32_t j = 0; j < NM; j++) {
            if constexpr (REG) xa[j] = xr[j];
            else {
                const uint4 l = xl[(t * NM + j) * 64u + xslot(lane, j)];
                xa[j] = u32x4{l.x, l.y, l.z, l.w};
            }
        }
        uint4 a[NM];
        if constexpr (M::BIAS) {
            uint32_t mb;
            float dd, dm;
            M::decode(reinterpret_cast<const u32a*>(win + m * M::WB), t < nt, q, a, mb, dd, dm);
            f32x4 tmp = zero;
#pragma unroll
            for (uint32_t j = 0; j < NM; j++)
                tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, xa[j]), __builtin_bit_cast(h8, a[j]), tmp, 0, 0, 0);
            // A: the sums of activation row lane % 16 for the lane's quarter's two sub-blocks
            const uint4 xo = make_uint4(REG ? xsr : xs[(t * 16u + m) * 4u + q], 0u, 0u, 0u), wo = make_uint4(mb, 0u, 0u, 0u);
            const f32x4 off = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, xo), __builtin_bit_cast(h8, wo), zero, 0, 0, 0);
#pragma unroll
            for (int c = 0; c < 4; c++) tmp[c] = fmaf(tmp[c], dd, -(off[c] * dm));
            return tmp;
        } else if constexpr (M::MLX) {
            uint32_t g0, g1;
            sbgroups(r, t, g0, g1);
            const uint32_t sh0 = 8u * ((g0 * es) & 3u), sh1 = 8u * ((g1 * es) & 3u);
            auto val = [&](uint32_t raw, uint32_t sh) { return es == 4u ? raw : (raw >> sh) & 0xFFFFu; };
            const uint32_t ax[4] = {val(aux[0], sh0), val(aux[1], sh0), val(aux[2], sh1), val(aux[3], sh1)};
            M::decode(reinterpret_cast<const u32a*>(win + m * M::WB), q, ax, p.sdtype, a);
        } else {
            M::decode(reinterpret_cast<const u32a*>(win + m * M::WB), task_off(r.om, t) & 3u, t < nt, q, a, rs);
        }
        f32x4 tmp = zero;
#pragma unroll
        for (uint32_t j = 0; j < NM; j++)
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, xa[j]), __builtin_bit_cast(h8, a[j]), tmp, 0, 0, 0);
        return tmp;
    };
    // Tiles outer, the wave's tasks inner (tpw is a multiple of PF, so ring
    // slot s of inner step g0 + s is static).  TPI tasks at a time
    // (independent MFMA chains); their slots are refilled, once stored to the
    // window, with the tasks PF later, which cross into the next tile at the
    // end of one.  Each tile's outputs are stored after its last task, outside
    // the loop whose loads stay in flight: no load sits under a branch.
    // One round: the PF tasks from g0 of the current tile (padding tasks, past
    // the segment's last and wave-uniform, are loaded like the others but
    // neither staged nor multiplied), then, with REFILL, their slots reloaded
    // in place (the same registers across rounds: no copies that would wait
    // for the loads) with the tasks PF later, which cross into the next tile
    // at the end of one.  The wave's last round loads nothing: a wave's end
    // waits for its loads in flight, which on launches of one tile per wave
    // were a whole extra round of loads (it is peeled, not branched around,
    // so every wait of the loop keeps its count).
    auto round = [&](uint32_t g0, const Rows& rnxt, auto refill) {
#pragma unroll
        for (int s = 0; s < PF; s += M::TPI) {
            const uint32_t g = t0 + g0 + (uint32_t)s;
            f32x4 prd[M::TPI];
            float rs[M::TPI] = {};
#pragma unroll
            for (int k = 0; k < M::TPI; k++)
                if (g + (uint32_t)k < nt)  // (XS_REG: tpw == PF, so ring slot s + k holds the wave's task s + k)
                    prd[k] = product(ring[s + k], rx[s + k], rcur, g + (uint32_t)k, rs[k], xreg[REG ? s + k : 0],
                                     sreg[REG ? s + k : 0]);
            if constexpr (decltype(refill)::value) {
                const bool wrap = g0 + (uint32_t)s + PF >= tpw;  // the refills belong to the next tile
                const uint32_t gn = wrap ? g + PF - tpw : g + PF;
#pragma unroll
                for (int k = 0; k < M::TPI; k++) load(wrap ? rnxt : rcur, gn + (uint32_t)k, ring[s + k], rx[s + k]);
            }
#pragma unroll
            for (int k = 0; k < M::TPI; k++) {
                if (g + (uint32_t)k >= nt) continue;
                // inverse activation scales of rows 4q..4q+3
                f32x4 sc = REG ? ireg[REG ? s + k : 0] : *reinterpret_cast<const f32x4*>(inv + (g + (uint32_t)k) * 16u + 4u * q);
                if constexpr (M::ROWSCALE) sc *= rs[k];
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] = fmaf(prd[k][c], sc[c], acc[c]);
            }
        }
    };
    for (uint32_t i = 0; i < nloop; i++) {
        const Where wnxt = where(tile_at(i + 1u));
        const Rows rnxt = rows_of(wnxt);
        const bool last = i + 1u == nloop;
        const uint32_t gend = last ? tpw - PF : tpw;  // rounds that reload
        for (uint32_t g0 = 0; g0 < gend; g0 += PF) round(g0, rnxt, std::true_type{});
        if (last) round(tpw - PF, rnxt, std::false_type{});
        if constexpr (SPLIT) {
            // the waves' partial tiles meet in their windows (a wave's last
            // window reads precede these writes: in order); wave 0 of each
            // group adds its group's and stores, then every window may be refilled
            *reinterpret_cast<f32x4*>(win + 16u * lane) = acc;
            __syncthreads();
            auto add_group = [&](auto wsc) {  // the group's other windows, all reads issued together
                constexpr uint32_t G = decltype(wsc)::value;
                f32x4 part[G - 1];
#pragma unroll
                for (uint32_t v = 1; v < G; v++)
                    part[v - 1] = *reinterpret_cast<const f32x4*>(wins + (wv + v) * 16u * M::WB + 16u * lane);
#pragma unroll
                for (uint32_t v = 1; v < G; v++) acc += part[v - 1];
            };
            if (wg == 0u) {
                if (wsl == 3u) add_group(std::integral_constant<uint32_t, 8>{});
                else add_group(std::integral_constant<uint32_t, 4>{});
            }
        }
        // lane l holds weight row l % 16 of activation rows 4q..4q+3
        const uint32_t row = wcur.row0 + m;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t b = 4u * q + (uint32_t)c;
            if ((!SPLIT || wg == 0u) && i < ntw && b < p.batch && row < wcur.n) {
                const size_t idx = (size_t)b * wcur.n + row;
                if constexpr (YBF16) gptr_mut<uint16_t>(wcur.y)[idx] = f32_to_bf16_bits(acc[c]);
                else if (p.accumulate) {  // later K segments
                    // through a global pointer (global_atomic_add_f32): a flat
                    // atomic would make every vmcnt wait of the loop a full drain
                    [[clang::atomic(ignore_denormal_mode)]] {
                        (void)__hip_atomic_fetch_add(gptr_mut<float>(wcur.y) + idx, acc[c], __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                    }
                } else gptr_mut<float>(wcur.y)[idx] = acc[c];
            }
        }
        if constexpr (SPLIT) __syncthreads();
        acc = zero;
        wcur = wnxt;
        rcur = rnxt;
    }
}

namespace {

// Modes (measured on the 8B shapes at batch 16, split / whole tiles / VALU):
// below kMfmaSplitTiles 16-row tiles the eight waves of a workgroup share
// each tile (split mode: 4096x12288 Q6_K 41 / 57 / 80 us, 4096x4096 Q4_0
// 11.7 / 15.3 / 22.7 us, q/k/v 13.9 / 15.9 / 32.8 us) when a segment has at
// least 4 tasks (Qwen3-0.6B MLX q/k/v, K = 1024, at 16 rows: 8.6 us split,
// 11.5 us with one wave per tile running all four); otherwise a wave takes whole tiles, which
// pays from kMfmaMinTiles tiles on (each workgroup stages all activations, a
// few microseconds, before its first product: lm_head 124 us whole tiles,
// 148 us split, 690 us VALU).
constexpr uint32_t kMfmaMinTiles = 384;
// When the VALU GEMV would take two register passes (more rows than one
// holds), whole tiles pay from fewer tiles: MLX q/k/v (4096 x 1024, 256
// tiles) at 16 rows 14.4 us on VALU (two launches), 11.4 us on MFMA.
constexpr uint32_t kMfmaMinTilesTwoPasses = 128;
constexpr uint32_t kMfmaSplitTiles = 1024;

// Units per launch: the fewest segments whose LDS fits, whole tasks each
// except the last.
template <class M, bool SPLIT>
uint32_t mfma_segment(uint32_t units) {
    for (uint32_t nseg = 1; nseg <= units; nseg++) {
        uint32_t seg = (units + nseg - 1u) / nseg;
        seg = nseg > 1 ? (seg + M::UPT - 1u) / M::UPT * M::UPT : seg;
        if (mfma_lds_bytes<M, SPLIT>(seg) <= kLdsBytes) return seg;
    }
    return 0;
}

// Zeroes the f32 outputs [batch, n_i] of every problem (before a launch whose
// K segments all add into them).
__global__ __launch_bounds__(256) void mfma_zero_outputs_kernel(const MfmaParams p) {
    const uint32_t i = blockIdx.y;
    const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < p.nprob && e < (uint64_t)p.batch * pick(i, p.n)) gptr_mut<float>(pick(i, p.y))[e] = 0.0f;
}

// bf16 outputs of a launch whose K segments added into f32 accumulators (the
// caller's workspace): problem blockIdx.y, element e of its [batch, n] rows,
// rounded to nearest even as every GEMV epilogue rounds.
struct MfmaBf16Out {
    const float* src[kMaxProblems];
    uint16_t* dst[kMaxProblems];
    uint32_t count[kMaxProblems];
};
__global__ __launch_bounds__(256) void mfma_bf16_outputs_kernel(const MfmaBf16Out c) {
    const uint32_t i = blockIdx.y;
    const uint32_t e = blockIdx.x * 256u + threadIdx.x;
    if (e < pick(i, c.count)) gptr_mut<uint16_t>(pick(i, c.dst))[e] = f32_to_bf16_bits(gptr<float>(pick(i, c.src))[e]);
}

// Stages a call's activations once, into the workspace, for a launch whose
// workgroups copy them (XS_PRE): unit u = (task g of all of K, row b < RB, e =
// q·NM + j) as the in-kernel staging forms it, with the 32 units of a (task,
// row) on 32 consecutive lanes, stored where segment g / seg_tasks of the
// launch finds it in its contiguous range (laid out as its LDS).  Rows past
// the batch stage zeros; rows RB..15 are not staged (their slots reach only
// output rows that are never stored).  Also clears the f32 outputs of a
// launch whose segments add into them.
constexpr uint32_t kMfmaPrepThreads = 256;
template <class M>
__global__ __launch_bounds__(kMfmaPrepThreads) void gemv_mfma_prep_kernel(const MfmaParams p, uint32_t rbl) {
    constexpr uint32_t NM = M::NM, UPR = 4u * NM, TL = mfma_task_lds<M>();
    static_assert(UPR == 32, "a (task, row) spans 32 lanes");
    const uint32_t tid = threadIdx.x, gid = blockIdx.x * kMfmaPrepThreads + tid;
    const uint32_t tall = p.nunit / M::UPT, seg_tasks = p.seg_units / M::UPT;
    const uint32_t total = tall * (UPR << rbl);
    const uint32_t u = gid < total ? gid : 0u;
    const uint32_t g = u >> (5u + rbl), b = (u >> 5u) & ((1u << rbl) - 1u), e = u % UPR, qq = e / NM, j = e % NM;
    const bool ok = gid < total && b < p.batch;
    const size_t xk0 = ok ? (size_t)b * p.K + M::KT * g : 0u;
    float v[8];
    if (p.x_bf16) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const uint16_t* xr = static_cast<const uint16_t*>(p.x) + xk0;
        const u32x2 lo2 = *gptr<u32x2>(xr + M::run0(qq, j)), hi2 = *gptr<u32x2>(xr + M::run1(qq, j));
        const uint32_t w[4] = {lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    } else {
        const float* xr = static_cast<const float*>(p.x) + xk0;
        const f32x4 lo4 = *gptr<f32x4>(xr + M::run0(qq, j)), hi4 = *gptr<f32x4>(xr + M::run1(qq, j));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = lo4[i];
            v[4 + i] = hi4[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = ok ? v[i] : 0.0f;
    const Staged st = stage_unit<M>(v);  // every lane: the cross-lane steps need whole groups of 32
    if (gid < total) {
        const uint32_t sg = g / seg_tasks, t = g - sg * seg_tasks;
        const uint32_t nts = tall - sg * seg_tasks < seg_tasks ? tall - sg * seg_tasks : seg_tasks;
        uint8_t* base = const_cast<uint8_t*>(p.pre) + (size_t)sg * seg_tasks * TL;
        *gptr_mut<u32x4>(base + ((t * NM + j) * 64u + xslot(b + 16u * qq, j)) * 16u) = u32x4{st.val.x, st.val.y, st.val.z, st.val.w};
        if (e == 0) *gptr_mut<float>(base + nts * NM * 1024u + (t * 16u + b) * 4u) = st.inv;
        if (M::BIAS && j == 0) *gptr_mut<uint32_t>(base + nts * (NM * 1024u + 64u) + ((t * 16u + b) * 4u + qq) * 4u) = st.xs;
    }
    if (p.accumulate) {  // every segment adds into y
        const uint32_t stride = gridDim.x * kMfmaPrepThreads;
        for (uint32_t i = 0; i < p.nprob; i++) {
            const uint32_t elems = p.batch * pick(i, p.n);
            for (uint32_t ei = gid; ei < elems; ei += stride) gptr_mut<float>(pick(i, p.y))[ei] = 0.0f;
        }
    }
}

// Whether a launch stages its activations once per call (when the caller
// gives a workspace) rather than in every workgroup: from K =
// kMfmaPrestageMinK on, at 9..16 rows, or when K takes several LDS segments
// (each staged by its own workgroups, and y cleared by one more launch, which
// the prep kernel replaces).  Per launch, Qwen3-8B Q4_0/Q6_K at 16 rows: q/k/v
// 13.5 -> 11.6 us, o_proj 11.5 -> 9.3, gate/up 23.4 -> 22.6, down_proj (K =
// 12288, three segments) 35.0 -> 26.5, lm_head 123 either way; at 8 rows the
// prep launch costs more than it saves on one segment (q/k/v 11.3 -> 11.5,
// gate/up 21.6 -> 22.6, lm_head 116 -> 120 us) and down_proj still gains,
// 30.3 -> 26.5 us.  From K = 1024 it lost at 12-16 rows on every shape timed
// (bf16 in/out, per launch: MLX 4096 x 1024 8.9 -> 10.2 us, 12288 x 1024
// 13.6 -> 15.1; Q4_0 4096 x 1024 7.4 -> 8.5, 12288 x 1024 11.2 -> 12.0).
constexpr uint32_t kMfmaPrestageMinK = 2048;
template <class M>
bool mfma_prestages(uint32_t K, uint32_t batch, int mode) {
    if (K < kMfmaPrestageMinK || mode == 0) return false;
    const uint32_t units = K / M::UNIT;
    const uint32_t seg = mode == 2 ? mfma_segment<M, true>(units) : mfma_segment<M, false>(units);
    return batch > 8u || seg < units;
}

template <class M, bool SPLIT>
hipError_t launch_mode(MfmaParams p, uint32_t units, bool y_bf16, uint8_t* pre, hipStream_t st) {
    uint32_t seg = mfma_segment<M, SPLIT>(units);
    if (seg == 0 || (y_bf16 && seg < units)) return hipErrorInvalidValue;
    // (a kernel whose row count is a run-time value stages 4 and 8 rows in a
    // quarter and half of the passes, but runs 16 rows ~1% slower than one
    // whose staging indices are constants: two instantiations)
    const bool r16 = p.batch > 8u;
    auto kernel = pre ? (y_bf16 ? gemv_mfma_kernel<M, true, SPLIT, XS_PRE> : gemv_mfma_kernel<M, false, SPLIT, XS_PRE>)
                : y_bf16 ? (r16 ? gemv_mfma_kernel<M, true, SPLIT, XS_ROWS16> : gemv_mfma_kernel<M, true, SPLIT, XS_ROWS8>)
                         : (r16 ? gemv_mfma_kernel<M, false, SPLIT, XS_ROWS16> : gemv_mfma_kernel<M, false, SPLIT, XS_ROWS8>);
    int cus = 0, per_cu = 0;
    hipError_t e = cached_occupancy(reinterpret_cast<const void*>(kernel), mfma_lds_bytes<M, SPLIT>(seg), kMfmaThreads,
                                    &per_cu, &cus);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || cus < 1) return hipErrorInvalidConfiguration;
    // K too long for LDS on a launch of at most one 16-row tile per CU: each
    // workgroup takes nseg tiles of one segment (segments of whole rounds of
    // tasks, a task per wave in split mode), so it stages a segment's
    // activations once for nseg tiles instead of once per tile (8B down_proj,
    // 4096 x 12288 Q6_K at 16 rows: 38.8 -> 35.2 us; cutting K where LDS does
    // not force it measured slower: o_proj 4096 x 4096 Q4_0 11.3 -> 14.6 us).
    bool shared_tiles = false;
    if (!y_bf16 && seg < units && p.total_tiles <= (uint32_t)cus) {
        const uint32_t step = SPLIT ? 8u * M::UPT : M::UPT;
        if (seg / step * step >= step) {
            seg = seg / step * step;
            shared_tiles = true;
        }
    }
    const uint32_t nseg = (units + seg - 1u) / seg;
    const size_t lds = mfma_lds_bytes<M, SPLIT>(seg);
    e = cached_occupancy(reinterpret_cast<const void*>(kernel), lds, kMfmaThreads, &per_cu, &cus);
    if (e != hipSuccess) return e;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    // every CU gets a workgroup while there are tiles: the tiles spread over
    // the workgroups first
    const uint64_t cap = (uint64_t)per_cu * cus;
    p.grid = (uint32_t)(p.total_tiles < cap ? p.total_tiles : cap);
    if (shared_tiles) {
        // about nseg tiles per workgroup, all nseg segments' workgroups resident
        // at once: a workgroup more than the CUs hold runs after the others
        // (8B down_proj at 16 rows, 256 tiles in three segments: 86 workgroups
        // a segment left two for a second round, 25.5 us; 85, one of them
        // taking a fourth tile, ~19 us)
        p.grid = (p.total_tiles + nseg - 1u) / nseg;
        const uint32_t fit = (uint32_t)(cap / nseg);
        p.grid = p.grid < fit ? p.grid : (fit ? fit : 1u);
    }
    // Split mode with more tiles than resident workgroups (one segment): two
    // groups of 4 waves per workgroup, each on its own tile, so the tiles take
    // one round instead of two (Qwen3-0.6B MLX gate/up, 384 tiles at ~161
    // VGPRs: one 8-wave workgroup per CU).
    p.split_ws_log2 = 3u;
    if (SPLIT && nseg == 1u && p.total_tiles > cap && p.total_tiles <= 2u * cap) {
        p.split_ws_log2 = 2u;
        p.grid = (p.total_tiles + 1u) / 2u;
    }
    p.k0 = 0;
    p.nunit = units;
    p.seg_units = seg;
    p.nseg = nseg;
    p.accumulate = nseg > 1u ? 1u : 0u;
    // split mode with eight waves per tile and two tasks per wave: each wave's
    // operands in registers (XS_REG), no copy into LDS
    size_t lds_launch = lds;
    if constexpr (SPLIT) {
        if (pre && p.split_ws_log2 == 3u && mfma_tasks<M, true>(seg, 8u) == 16u) {
            auto kreg = y_bf16 ? gemv_mfma_kernel<M, true, true, XS_REG> : gemv_mfma_kernel<M, false, true, XS_REG>;
            const size_t lreg = (kMfmaThreads / 64u) * 16u * M::WB;  // the windows only
            int rcus = 0, rper = 0;
            e = cached_occupancy(reinterpret_cast<const void*>(kreg), lreg, kMfmaThreads, &rper, &rcus);
            if (e != hipSuccess) return e;
            if ((uint64_t)rper * rcus >= (uint64_t)p.grid * nseg) {  // all workgroups resident, as planned
                kernel = kreg;
                lds_launch = lreg;
            }
        }
    }
    if (pre) {  // stage once (and clear y when the segments add into it)
        p.pre = pre;
        const uint32_t rbl = p.batch <= 4u ? 2u : p.batch <= 8u ? 3u : 4u;
        const uint64_t total = (uint64_t)(units / M::UPT) * (32u << rbl);
        hipLaunchKernelGGL(gemv_mfma_prep_kernel<M>, dim3((unsigned)((total + kMfmaPrepThreads - 1u) / kMfmaPrepThreads)),
                           dim3(kMfmaPrepThreads), 0, st, p, rbl);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    } else if (nseg > 1u) {  // every segment adds into y (f32): clear it first
        uint32_t nmax = 0;
        for (uint32_t i = 0; i < p.nprob; i++) nmax = p.n[i] > nmax ? p.n[i] : nmax;
        const uint64_t elems = (uint64_t)p.batch * nmax;
        hipLaunchKernelGGL(mfma_zero_outputs_kernel, dim3((unsigned)((elems + 255u) / 256u), p.nprob), dim3(256), 0, st,
                           p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(p.grid * nseg), dim3(kMfmaThreads), lds_launch, st, p);
    return hipGetLastError();
}

template <class M>
int mfma_mode(uint32_t K, uint32_t tiles, bool y_bf16, uint32_t min_tiles);

uint32_t mfma_min_tiles(uint32_t enc, uint32_t batch) {
    return batch > max_register_batch(enc) ? kMfmaMinTilesTwoPasses : kMfmaMinTiles;
}

template <class M>
hipError_t launch_mfma(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x, bool x_bf16,
                       uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, void* work, uint64_t work_bytes,
                       hipStream_t st) {
    const uint32_t min_tiles = mfma_min_tiles(enc, batch);
    MfmaParams p = {};
    uint32_t tiles = 0;
    for (int i = 0; i < kMaxProblems; i++) {
        const GemvProblem& g = probs[i < nprob ? i : nprob - 1];
        p.w[i] = g.w;
        p.sc[i] = g.sc;
        p.bi[i] = g.bi;
        p.y[i] = g.y;
        p.n[i] = i < nprob ? g.n : 0u;
        p.tile_begin[i] = tiles;
        if (i < nprob) tiles += (g.n + 15u) / 16u;
    }
    p.total_tiles = tiles;
    p.nprob = (uint32_t)nprob;
    p.K = K;
    p.batch = batch;
    p.x = x;
    p.x_bf16 = x_bf16 ? 1u : 0u;
    p.group = group;
    p.gmagic = group_magic(group);
    p.sdtype = sdtype;
    const uint32_t units = K / M::UNIT;
    const int mode = mfma_mode<M>(K, tiles, y_bf16, min_tiles);
    uint8_t* pre = work && work_bytes >= mfma_prestage_bytes<M>(K) && mfma_prestages<M>(K, batch, mode)
                       ? static_cast<uint8_t*>(work)
                       : nullptr;
    return mode == 2 ? launch_mode<M, true>(p, units, y_bf16, pre, st) : launch_mode<M, false>(p, units, y_bf16, pre, st);
}

// 2: split mode, 1: whole tiles per wave, 0: not on MFMA (with bf16 outputs
// only a single segment)
template <class M>
int mfma_mode(uint32_t K, uint32_t tiles, bool y_bf16, uint32_t min_tiles) {
    const uint32_t units = K / M::UNIT;
    if (tiles < kMfmaSplitTiles) {
        const uint32_t seg = mfma_segment<M, true>(units);
        if (seg / M::UPT >= 4u && (!y_bf16 || seg == units)) return 2;
    }
    const uint32_t seg = mfma_segment<M, false>(units);
    return tiles >= min_tiles && seg > 0 && (!y_bf16 || seg == units) ? 1 : 0;
}

}  // namespace

bool gemv_mfma_applies(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K, bool y_bf16,
                       uint32_t group) {
    if ((enc != ENC_Q4_0 && enc != ENC_Q6_K && enc != ENC_Q4_K && enc != ENC_Q5_K && enc != ENC_IQ4_XS &&
         enc != ENC_MLX_U4) ||
        batch < 3 || batch > 16 || K % 256u)
        return false;
    if (enc == ENC_MLX_U4 && (group == 0 || group % 32u)) return false;
    uint32_t tiles = 0;
    uint64_t rows = 0;
    for (int i = 0; i < nprob; i++) {
        tiles += (probs[i].n + 15u) / 16u;
        rows += probs[i].n;
    }
    // The MFMA path's fixed costs (staging every activation row per
    // workgroup, a wave's first products) outweigh the VALU GEMV's per-row
    // work on small launches that the VALU GEMV serves in one register pass:
    // it takes launches with more rows than one pass holds, launches of at
    // least 8 MB of weights, or at least kMfmaSplitTiles tiles (measured at
    // the Qwen3-0.6B MLX shapes: 1-4 MB launches take ~13 us on MFMA against
    // 7-9 us on VALU at 5-8 rows, 13-15 against 14-18 us at 16 rows).
    // At 3-4 rows only the largest launches gain (8B lm_head at 4 rows: 114 us on MFMA against 181 us;
    // at 2 rows both take ~111 us).
    const uint64_t bytes = rows * (enc == ENC_Q4_0   ? K / 32u * 18u
                                   : enc == ENC_Q6_K ? K / 256u * 210u
                                   : enc == ENC_Q4_K ? K / 256u * 144u
                                   : enc == ENC_Q5_K ? K / 256u * 176u
                                   : enc == ENC_IQ4_XS ? K / 256u * 136u
                                                     : K / 2u);
    // At 3-4 rows the VALU GEMV's per-row dot products are cheap enough that
    // only the largest launches gain, and Q4_0 (the cheapest MFMA decode) with
    // K = 4096 on 384-512 tiles: per launch at 4 rows, the 8B q/k/v (384 tiles)
    // 10.58 -> 9.82 us, 8192 x 4096 11.6 -> 11.3; o_proj (256 tiles) 7.5 -> 7.9,
    // the Q6_K down_proj 17.9 -> 20.2 and the Q4_K q/k 10.0 -> 10.5 stay on
    // VALU, and so do other Q4_0 shapes (10240 x 4096 12.9 -> 14.5, 14336 x
    // 4096 17.0 -> 17.5, 6144 x 5120 14.3 -> 17.6, 13824 x 5120 23.0 -> 29.1,
    // 6144 x 8192 15.8 -> 19.6 on MFMA).
    const bool q4_0_few = enc == ENC_Q4_0 && K == 4096u && tiles >= kMfmaMinTiles && tiles <= 512u;
    if (batch < 5 && tiles < kMfmaSplitTiles && !q4_0_few) return false;
    if (batch <= max_register_batch(enc) && bytes < (8ull << 20) && tiles < kMfmaSplitTiles) return false;
    const uint32_t min_tiles = mfma_min_tiles(enc, batch);
    const int mode = enc == ENC_Q4_0   ? mfma_mode<MfmaQ40>(K, tiles, y_bf16, min_tiles)
                   : enc == ENC_Q6_K   ? mfma_mode<MfmaQ6K>(K, tiles, y_bf16, min_tiles)
                   : enc == ENC_Q4_K   ? mfma_mode<MfmaQ4K>(K, tiles, y_bf16, min_tiles)
                   : enc == ENC_Q5_K   ? mfma_mode<MfmaQ5K>(K, tiles, y_bf16, min_tiles)
                   : enc == ENC_IQ4_XS ? mfma_mode<MfmaIQ4XS>(K, tiles, y_bf16, min_tiles)
                                       : mfma_mode<MfmaMlxU4>(K, tiles, y_bf16, min_tiles);
    return mode != 0;
}

uint64_t gemv_mfma_workspace_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                                   bool y_bf16, uint32_t group) {
    if (!gemv_mfma_applies(enc, probs, nprob, batch, K, y_bf16, group))
        return y_bf16 ? gemv_mfma_bf16_acc_bytes(enc, probs, nprob, batch, K, group) : 0;
    uint32_t tiles = 0;
    for (int i = 0; i < nprob; i++) tiles += (probs[i].n + 15u) / 16u;
    const uint32_t min_tiles = mfma_min_tiles(enc, batch);
    auto size = [&](auto pol) -> uint64_t {
        using M = decltype(pol);
        if (!mfma_prestages<M>(K, batch, mfma_mode<M>(K, tiles, y_bf16, min_tiles))) return 0;
        return (mfma_prestage_bytes<M>(K) + 255u) & ~(uint64_t)255u;
    };
    return enc == ENC_Q4_0   ? size(MfmaQ40{})
         : enc == ENC_Q6_K   ? size(MfmaQ6K{})
         : enc == ENC_Q4_K   ? size(MfmaQ4K{})
         : enc == ENC_Q5_K   ? size(MfmaQ5K{})
         : enc == ENC_IQ4_XS ? size(MfmaIQ4XS{})
                             : size(MfmaMlxU4{});
}

hipError_t gemv_mfma_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x, bool x_bf16,
                            uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, void* work,
                            uint64_t work_bytes, hipStream_t st) {
    if (nprob < 1 || nprob > kMaxProblems) return hipErrorInvalidValue;
    auto go = [&](auto pol) {
        return launch_mfma<decltype(pol)>(enc, probs, nprob, K, x, x_bf16, batch, y_bf16, group, sdtype, work,
                                          work_bytes, st);
    };
    if (enc == ENC_Q4_0) return go(MfmaQ40{});
    if (enc == ENC_Q6_K) return go(MfmaQ6K{});
    if (enc == ENC_Q4_K) return go(MfmaQ4K{});
    if (enc == ENC_Q5_K) return go(MfmaQ5K{});
    if (enc == ENC_IQ4_XS) return go(MfmaIQ4XS{});
    if (enc == ENC_MLX_U4) return go(MfmaMlxU4{});
    return hipErrorInvalidValue;
}

// bf16 outputs: K segments cannot add into them, so a launch with K too long
// for one LDS segment leaves the MFMA GEMV (onto the VALU GEMV's two register
// passes at 9..16 rows: 4096 x 12288 at 16 rows 63-74 us against 17-23 us with
// f32 outputs).  Given a workspace, the segments add into f32 accumulators in
// it (after the staged activations) and one more launch rounds them to bf16.
namespace {
uint64_t bf16_acc_bytes(const GemvProblem* probs, int nprob, uint32_t batch) {
    uint64_t s = 0;
    for (int i = 0; i < nprob; i++) s += ((uint64_t)batch * probs[i].n * 4u + 255u) & ~(uint64_t)255u;
    return s;
}
}  // namespace

uint64_t gemv_mfma_bf16_acc_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                                  uint32_t group) {
    if (gemv_mfma_applies(enc, probs, nprob, batch, K, true, group) ||
        !gemv_mfma_applies(enc, probs, nprob, batch, K, false, group))
        return 0;
    const uint64_t pre = gemv_mfma_workspace_bytes(enc, probs, nprob, batch, K, false, group);
    return pre ? pre + bf16_acc_bytes(probs, nprob, batch) : 0;  // (a segmented launch always prestages)
}

hipError_t gemv_mfma_launch_bf16_acc(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x,
                                     bool x_bf16, uint32_t batch, uint32_t group, uint32_t sdtype, void* work,
                                     uint64_t work_bytes, hipStream_t st) {
    if (nprob < 1 || nprob > kMaxProblems) return hipErrorInvalidValue;
    const uint64_t need = gemv_mfma_bf16_acc_bytes(enc, probs, nprob, batch, K, group);
    if (!need || !work || work_bytes < need || ((uintptr_t)work & 255u)) return hipErrorInvalidValue;
    const uint64_t pre = gemv_mfma_workspace_bytes(enc, probs, nprob, batch, K, false, group);
    GemvProblem acc[kMaxProblems];
    MfmaBf16Out c{};
    uint8_t* a = static_cast<uint8_t*>(work) + pre;
    uint32_t most = 0;
    for (int i = 0; i < kMaxProblems; i++) {
        const int k = i < nprob ? i : nprob - 1;
        acc[i] = probs[k];
        c.count[i] = i < nprob ? batch * probs[i].n : 0u;
        if (i < nprob) {
            acc[i].y = a;
            c.src[i] = reinterpret_cast<const float*>(a);
            c.dst[i] = static_cast<uint16_t*>(probs[i].y);
            a += ((uint64_t)c.count[i] * 4u + 255u) & ~(uint64_t)255u;
            most = c.count[i] > most ? c.count[i] : most;
        } else {
            c.src[i] = c.src[0];
            c.dst[i] = c.dst[0];
        }
    }
    hipError_t e = gemv_mfma_launch(enc, acc, nprob, K, x, x_bf16, batch, false, group, sdtype, work, pre, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mfma_bf16_outputs_kernel, dim3((most + 255u) / 256u, (unsigned)nprob), dim3(256), 0, st, c);
    return hipGetLastError();
}

}  // namespace dmx
