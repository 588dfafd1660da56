// Decode GEMV on MFMA for 5..16 activation rows, GGUF Q4_0 (y[b, o] =
// Σ_k x[b, k]·w[o, k], f32 accumulation; gguf_codegen.rs:268-314 `emit_linear`
// with the Q4_0 dequantisation of :412-472).
//
// The VALU GEMV multiplies every decoded weight once per activation row (a
// v_dot2 per pair per row), so above ~4 rows its VALU and LDS work grows with
// the batch while the weight stream does not.  Here the activation rows are
// the N side of v_mfma_f32_16x16x32_f16 (16 columns, zero-padded) and each
// weight is decoded once, whatever the batch:
//   * a wave owns tiles of 16 weight rows (the A side: lane l holds row l % 16
//     and 8 k of the instruction's 32); per instruction, lane quarter
//     q = l / 16 contributes 8 weights of its own block 4g + q of the row (the
//     k slots of one MFMA may hold any k as long as the activation side holds
//     the same ones, and the block scale is folded into each f16 weight), so
//     the four lanes of a row read 72 contiguous bytes, and the four MFMAs of
//     a 4-block group j = 0..3 take code dword j of every block: its 8 weights
//     (4j, 4j+2), (4j+1, 4j+3), (16+4j, 18+4j), (17+4j, 19+4j), one
//     v_and_or_b32 per pair (a low nibble under the f16 exponent of 1024 is
//     1024+q, a high nibble under that of 64 is 64+q, both exact), a packed
//     add giving q-8 (exact) and a packed multiply RNE_f16((q-8)·d), the only
//     rounding of the weight (relative 2^-11);
//   * the activations are staged once per workgroup in LDS as f16 in the B
//     layout of each (group, j): lane (b, q) the 8 matching activations of
//     row b, scaled by a power of two per (row, 128-k group) whose largest
//     magnitude lands in [2^13, 2^14) (no overflow, no flush of the group's
//     large values), rounded once to f16; the group's four MFMAs accumulate
//     into a zeroed tile that is then added to the f32 total times the
//     group's inverse scale;
//   * weights stream through a ring of PF groups of raw block loads per
//     wave (the next groups' loads in flight while one is multiplied);
//   * a K range too long for LDS runs as segments in consecutive launches,
//     the later ones adding to the f32 outputs.
// Accuracy: |y - y_exact| <= (2^-11 + 2^-11 + 2^-22)·Σ|w||x| + f32 accumulation
// error (weight and activation roundings), inside the 2e-3 normalised tolerance.
#include "gemv_kernels.hpp"

namespace dmx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef half2_t h2;
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kMfmaThreads = 512;
constexpr int kMfmaPF = 8;  // tasks of raw loads in flight per wave (a multiple of 4)

struct MfmaParams {
    const uint8_t* w[kMaxProblems];
    uint32_t n[kMaxProblems];
    uint32_t tile_begin[kMaxProblems];  // first 16-row tile of each problem
    uint32_t total_tiles;
    uint32_t grid;
    uint32_t K;        // full reduction length (row bytes)
    uint32_t k0;       // first k of this launch's segment
    uint32_t nblk;     // Q4_0 blocks in the segment
    uint32_t nprob;
    uint32_t batch;
    uint32_t y_bf16;
    uint32_t accumulate;  // add to y (later segments; f32 outputs only)
    const float* x;
    void* y[kMaxProblems];
};

// LDS: activations [group][j][64 lanes] x 16 bytes, then the inverse scales
// [group][16 rows] f32.
// 4-block groups of a segment, padded to a multiple of kMfmaPF (the padding
// groups have zero weights and activations)
__host__ __device__ constexpr uint32_t mfma_groups(uint32_t nblk) {
    return ((nblk + 3u) / 4u + kMfmaPF - 1u) / kMfmaPF * kMfmaPF;
}
__host__ __device__ constexpr uint32_t mfma_lds_bytes(uint32_t nblk) { return mfma_groups(nblk) * (4u * 64u * 16u + 64u); }

// Slot of B-operand lane l (row b = l % 16, quarter q = l / 16) in the 64
// slots of 16 bytes of one (group, j): l with its low three bits XORed by
// (j + 4·(q & 1)) & 7.  A bijection within each 16-lane quarter, so a
// fragment read (64 lanes, slots l) stays conflict-free, while the 16
// staging threads of one (group, row) (j, q = 0..3) spread their writes over
// all 8 16-byte bank groups instead of one.
__device__ __forceinline__ uint32_t xslot(uint32_t l, uint32_t j) { return l ^ ((j + 4u * ((l >> 4) & 1u)) & 7u); }

__device__ __forceinline__ uint32_t wq(uint32_t c, _Float16 off, h2 d2) {
    const h2 o = {off, off};
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, c) + o) * d2);
}

}  // namespace

template <bool YBF16>
__global__ __launch_bounds__(kMfmaThreads) void gemv_mfma_q4_0_kernel(const MfmaParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t ng = mfma_groups(p.nblk);
    uint4* xl = reinterpret_cast<uint4*>(lds);
    float* inv = reinterpret_cast<float*>(lds + ng * 4u * 64u * 16u);
    const uint32_t tid = threadIdx.x, lane = tid & 63u;

    // ---- weight tiles: wave wid takes tiles wid, wid + W, ..., waves numbered
    // across workgroups first (wave i of workgroup w is wid = i·grid + w), so
    // a few tiles still spread over all CUs; task = (tile, group), PF tasks of
    // raw loads in flight
    const uint32_t wid = __builtin_amdgcn_readfirstlane((tid >> 6) * p.grid + blockIdx.x);
    const uint32_t W = p.grid * (kMfmaThreads / 64u);
    const uint32_t m = lane & 15u, q = lane >> 4;
    const uint32_t ntw = wid < p.total_tiles ? (p.total_tiles - wid + W - 1u) / W : 0u;  // tiles of this wave
    const uint32_t rowbytes = (p.K / 32u) * 18u, kb0 = p.k0 / 32u;

    // the wave's i-th tile (past the end: its last, or any tile for a wave
    // without tiles: loaded, never multiplied into a stored result)
    auto tile_at = [&](uint32_t i) {
        const uint32_t ii = i < ntw ? i : (ntw ? ntw - 1u : 0u);
        const uint32_t tile = wid + ii * W;
        return tile < p.total_tiles ? tile : p.total_tiles - 1u;
    };
    struct Where {
        const uint8_t* w;
        void* y;
        uint32_t n, row0;
    };
    auto where = [&](uint32_t tile) {
        uint32_t pi = 0;
#pragma unroll
        for (int i = 1; i < kMaxProblems; i++) pi += ((uint32_t)i < p.nprob && tile >= p.tile_begin[i]) ? 1u : 0u;
        Where r;
        r.w = pick(pi, p.w);
        r.y = pick(pi, p.y);
        r.n = pick(pi, p.n);
        r.row0 = (tile - pick(pi, p.tile_begin)) * 16u;
        return r;
    };
    // a tile's weight base and the byte offset of this lane's row (rows past
    // the problem re-read its last one: in bounds, never stored)
    struct Rows {
        const uint8_t* w;
        uint32_t off;
    };
    auto rows_of = [&](const Where& wh) {
        const uint32_t row = wh.row0 + m < wh.n ? wh.row0 + m : wh.n - 1u;
        return Rows{wh.w, row * rowbytes};
    };
    // raw loads of group g of a tile: block 4g + q of the lane's row
    auto load = [&](const Rows& r, uint32_t g) {
        const uint32_t blk = 4u * g + q;
        const uint32_t kb = kb0 + (blk < p.nblk ? blk : p.nblk - 1u);  // past the segment: zeroed d
        return load_raw_block<5>(r.w, r.off + kb * 18u);
    };
    // the first PF tasks' weight loads leave before the activations are staged
    Where wcur = where(tile_at(0u));
    Rows rcur = rows_of(wcur);
    RawBlock<5> ring[kMfmaPF];
#pragma unroll
    for (int s = 0; s < kMfmaPF; s++) ring[s] = load(rcur, (uint32_t)s);  // ng >= PF: all in tile 0

    // ---- stage the activations: unit u = (group g, row b, e = 4q + j), the 16
    // units of (g, b) on one DPP row of 16 lanes.  Pass i + 1's loads are
    // issued before pass i is converted, so the passes share one latency.
    const uint32_t nunits = ng * 256u, npass = (nunits + kMfmaThreads - 1u) / kMfmaThreads;
    auto xload = [&](uint32_t pass, float (&v)[8]) {
        const uint32_t u = pass * kMfmaThreads + tid;
        const uint32_t g = u >> 8, b = (u >> 4) & 15u, e = u & 15u, q = e >> 2, j = e & 3u;
        const uint32_t blk = 4u * g + q;
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.0f;
        if (u < nunits && b < p.batch && blk < p.nblk) {
            const float* xr = p.x + (size_t)b * p.K + p.k0 + 32u * blk + 4u * j;
            const f32x4 lo = *gptr<f32x4>(xr), hi = *gptr<f32x4>(xr + 16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = lo[i];
                v[4 + i] = hi[i];
            }
        }
    };
    auto xstore = [&](uint32_t pass, const float (&v)[8]) {
        const uint32_t u = pass * kMfmaThreads + tid;
        const uint32_t g = u >> 8, b = (u >> 4) & 15u, e = u & 15u, q = e >> 2, j = e & 3u;
        float m = absmax3(v[0], v[1], v[2]);
        m = absmax3(m, v[3], v[4]);
        m = absmax3(m, v[5], v[6]);
        m = absmax3(m, v[7], v[7]);
        uint32_t mx = __float_as_uint(m);  // non-negative floats order as integers
        mx = lanes_reduce<8>(mx, [](uint32_t a, uint32_t c) { return a > c ? a : c; });
        mx = max(mx, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x140, 0xF, 0xF, false));  // row_mirror: all 16
        int ex = 0;
        (void)frexpf(__uint_as_float(mx), &ex);
        ex = ex < -110 ? -110 : ex;  // keeps the scale a normal f32
        const int sh = 14 - ex;      // largest magnitude / 2^(ex-14) < 2^14
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        auto pk = [&](float a, float c) {
            const f32x2 f = {ldexpf(a, sh), ldexpf(c, sh)};
            return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));  // RNE
        };
        // block-relative k: (4j, 4j+2) (4j+1, 4j+3) (16+4j, 18+4j) (17+4j, 19+4j)
        const uint4 val = make_uint4(pk(v[0], v[2]), pk(v[1], v[3]), pk(v[4], v[6]), pk(v[5], v[7]));
        if (u < nunits) {
            xl[(g * 4u + j) * 64u + xslot(b + 16u * q, j)] = val;
            if (e == 0) inv[g * 16u + b] = ldexpf(1.0f, -sh);
        }
    };
    // chunks of kStageChunk passes (K = 4096 at batch 16: one chunk): all of a
    // chunk's loads leave before the first is converted
    constexpr uint32_t kStageChunk = 16;
    for (uint32_t c0 = 0; c0 < npass; c0 += kStageChunk) {
        float v[kStageChunk][8];
#pragma unroll
        for (uint32_t i = 0; i < kStageChunk; i++) xload(c0 + i < npass ? c0 + i : npass - 1u, v[i]);
#pragma unroll
        for (uint32_t i = 0; i < kStageChunk; i++)
            if (c0 + i < npass) xstore(c0 + i, v[i]);
    }
    __syncthreads();

    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc = zero;
    // one task's product: decode block 4g + q's four code dwords and run the
    // group's four MFMAs into a zeroed tile
    auto product = [&](const RawBlock<5>& r, uint32_t g) {
        const bool ok = 4u * g + q < p.nblk;
        const uint32_t sel = realign_sel(r.sh, 2);
        uint32_t cd[4];
#pragma unroll
        for (int c = 0; c < 4; c++) cd[c] = __builtin_amdgcn_perm(r.d[c + 1], r.d[c], sel);
        const uint32_t db = ok ? (r.d[0] >> (8u * r.sh)) & 0xFFFFu : 0u;  // past the segment: zero weights
        const h2 d2 = __builtin_bit_cast(h2, db * 0x00010001u);
        f32x4 tmp = zero;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const uint32_t D = cd[jj], D8 = D >> 8;
            const uint4 a = make_uint4(wq(and_or(D, 0x000F000Fu, 0x64006400u), (_Float16)-1032.0f, d2),
                                       wq(and_or(D8, 0x000F000Fu, 0x64006400u), (_Float16)-1032.0f, d2),
                                       wq(and_or(D, 0x00F000F0u, 0x54005400u), (_Float16)-72.0f, d2),
                                       wq(and_or(D8, 0x00F000F0u, 0x54005400u), (_Float16)-72.0f, d2));
            const uint4 xb = xl[(g * 4u + (uint32_t)jj) * 64u + xslot(lane, (uint32_t)jj)];
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, xb), tmp, 0, 0, 0);
        }
        return tmp;
    };
    // Tiles outer, groups inner (ng is a multiple of PF, so ring slot s of
    // inner step g0 + s is static).  Four tasks at a time (four independent
    // MFMA chains); their slots are refilled, once decoded, with the tasks PF
    // later, which cross into the next tile at the end of one.  Each tile's outputs are
    // stored after its last group, outside the loop whose loads stay in
    // flight: no load sits under a branch.
    for (uint32_t i = 0; i < ntw; i++) {
        const Where wnxt = where(tile_at(i + 1u));
        const Rows rnxt = rows_of(wnxt);
        for (uint32_t g0 = 0; g0 < ng; g0 += kMfmaPF) {
#pragma unroll
            for (int s = 0; s < kMfmaPF; s += 4) {
                const uint32_t g = g0 + (uint32_t)s;
                f32x4 pr[4];
#pragma unroll
                for (int u = 0; u < 4; u++) pr[u] = product(ring[s + u], g + (uint32_t)u);
                // refill the slots in place once decoded (the same registers
                // across iterations: no copies that would wait for the loads)
                const bool wrap = g + kMfmaPF >= ng;  // the refills belong to the next tile
                const Rows rr = wrap ? rnxt : rcur;
                const uint32_t ng0 = wrap ? g + kMfmaPF - ng : g + kMfmaPF;
#pragma unroll
                for (int u = 0; u < 4; u++) ring[s + u] = load(rr, ng0 + (uint32_t)u);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float sc = inv[(g + (uint32_t)u) * 16u + (lane & 15u)];
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[k] = fmaf(pr[u][k], sc, acc[k]);
                }
            }
        }
        // lane l holds activation row b = l % 16 and weight rows 4q..4q+3
        const Where wh = wcur;
        const uint32_t b = lane & 15u;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t row = wh.row0 + 4u * q + (uint32_t)k;
            if (b < p.batch && row < wh.n) {
                const size_t idx = (size_t)b * wh.n + row;
                if constexpr (YBF16) gptr_mut<uint16_t>(wh.y)[idx] = f32_to_bf16_bits(acc[k]);
                else if (p.accumulate) unsafeAtomicAdd(&static_cast<float*>(wh.y)[idx], acc[k]);  // later K segments
                else gptr_mut<float>(wh.y)[idx] = acc[k];
            }
        }
        acc = zero;
        wcur = wnxt;
        rcur = rnxt;
    }
}

// Launches with fewer than kMfmaMinTiles 16-row tiles stay on the VALU GEMV:
// each workgroup stages all activations (~6-8 us at K = 4096, batch 16)
// and a wave multiplies its tile's groups in sequence, which only pays off
// when the weights are many (measured on the 8B shapes at batch 16: 4096
// rows 28 us on MFMA against 22 us on VALU, 6144 rows 28 against 32,
// 24576 rows 31 against 76).
constexpr uint32_t kMfmaMinTiles = 384;

bool gemv_mfma_applies(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K, bool x_bf16,
                       bool y_bf16) {
    if (enc != ENC_Q4_0 || x_bf16 || batch < 5 || batch > 16) return false;
    uint32_t tiles = 0;
    for (int i = 0; i < nprob; i++) tiles += (probs[i].n + 15u) / 16u;
    if (tiles < kMfmaMinTiles) return false;
    return !y_bf16 || mfma_lds_bytes(K / 32u) <= kLdsBytes;  // bf16 outputs cannot add up segments
}

hipError_t gemv_mfma_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x,
                            uint32_t batch, bool y_bf16, hipStream_t st) {
    if (enc != ENC_Q4_0 || nprob < 1 || nprob > kMaxProblems) return hipErrorInvalidValue;
    MfmaParams p = {};
    uint32_t tiles = 0;
    for (int i = 0; i < kMaxProblems; i++) {
        const GemvProblem& g = probs[i < nprob ? i : nprob - 1];
        p.w[i] = g.w;
        p.y[i] = g.y;
        p.n[i] = i < nprob ? g.n : 0u;
        p.tile_begin[i] = tiles;
        if (i < nprob) tiles += (g.n + 15u) / 16u;
    }
    p.total_tiles = tiles;
    p.nprob = (uint32_t)nprob;
    p.K = K;
    p.batch = batch;
    p.y_bf16 = y_bf16 ? 1u : 0u;
    p.x = static_cast<const float*>(x);
    // segments of at most kSegBlocks blocks (a multiple of 4: whole groups)
    uint32_t seg = K / 32u;
    while (mfma_lds_bytes(seg) > kLdsBytes) seg = (seg + 1u) / 2u;
    seg = seg < K / 32u ? (seg + 3u) / 4u * 4u : seg;
    while (mfma_lds_bytes(seg) > kLdsBytes) seg -= 4u;
    if (seg == 0) return hipErrorInvalidValue;
    if (y_bf16 && seg < K / 32u) return hipErrorInvalidValue;
    auto kernel = y_bf16 ? gemv_mfma_q4_0_kernel<true> : gemv_mfma_q4_0_kernel<false>;
    for (uint32_t b0 = 0; b0 < K / 32u; b0 += seg) {
        const uint32_t nb = K / 32u - b0 < seg ? K / 32u - b0 : seg;
        const size_t lds = mfma_lds_bytes(nb);
        int cus = 0, per_cu = 0;
        hipError_t e = cached_occupancy(reinterpret_cast<const void*>(kernel), lds, kMfmaThreads, &per_cu, &cus);
        if (e != hipSuccess) return e;
        if (per_cu < 1) return hipErrorInvalidConfiguration;
        // every CU gets a workgroup while there are tiles: the tiles spread over
        // the workgroups first (wave numbering in the kernel)
        const uint64_t cap = (uint64_t)per_cu * cus;
        p.grid = (uint32_t)(tiles < cap ? tiles : cap);
        p.k0 = b0 * 32u;
        p.nblk = nb;
        p.accumulate = b0 > 0 ? 1u : 0u;
        hipLaunchKernelGGL(kernel, dim3(p.grid), dim3(kMfmaThreads), lds, st, p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace dmx
