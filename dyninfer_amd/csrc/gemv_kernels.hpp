// Decode GEMV kernel templates (activation rows 1..16) for GGUF Q4_0/Q4_1/Q8_0/
// Q6_K and MLX affine U4.
//
// Semantics: y[b, o] = Σ_k x[b, k] · w[o, k] with f32 accumulation, w the
// reference's dequantised weight (gguf_codegen.rs:268-314 `emit_linear`,
// mlx_affine.rs:557-626 `emit_linear_u4`).  IREE's reduction order is itself
// unspecified, so results agree within f32 reassociation and the f16 rounding
// of activations (encodings.hpp), not bitwise.
//
// Mapping (wave64, 512-thread workgroups; packed weights stream once from HBM):
//   * the activations are staged once per workgroup in LDS as f16 pairs in
//     each encoding's decode order, with per-(row, chunk, group) constants
//     (-C, power-of-two scale, Σx) — encodings.hpp gives the contract;
//   * the weight rows are cut into row blocks of G·R rows (G = 64/L lane
//     groups per wave, R rows per group); the L lanes of a group split K:
//     lane j takes chunks j, j+L, ... (cpl = ceil(chunks/L) of them per row
//     block; a lane past the last chunk re-reads the last one and adds zero),
//     so neighbouring lanes read neighbouring blocks (coalesced) and
//     neighbouring activation chunks (distinct LDS banks, 16-byte padding);
//   * the grid is persistent (occupancy x CUs workgroups): wave w walks row
//     blocks w, w+W, ... and the lane's (row block, chunk) tasks run as one
//     software pipeline — the next task's weight bytes are loaded before the
//     current task is computed, and the first task's before the activation
//     staging, so HBM latency overlaps staging and arithmetic;
//   * per weight: half a v_and_or_b32 and half a v_dot2_f32_f16 per
//     activation row; per group and row: two or three f32 ops;
//   * at the end of a row block the L lanes combine their R·B partial sums
//     with cross-lane shuffles and lane 0 of the group stores.
// Several weights that share one activation (q/k/v, gate/up) are served by one
// launch: row blocks are numbered across the problems.
#pragma once
#include <type_traits>

#include "encodings.hpp"
#include "kernels.hpp"

namespace dmx {

constexpr int kGemvThreads = 512;

// a[i] for a wave-uniform i, branch-free.  The four values are pinned in
// scalar registers first (otherwise the optimiser folds the selection back
// into a dynamic index of the kernel-argument array, which it can only serve
// from a private scratch copy), then combined with masks (a select chain is
// turned into branches, and branches between a load and its use cost the
// wait counters their precision).
template <class T>
__device__ __forceinline__ T pick(uint32_t i, const T (&a)[kMaxProblems]) {
    static_assert(kMaxProblems == 4, "pick() assumes 4 problems");
    static_assert(sizeof(T) == 8 || sizeof(T) == 4, "pick() takes pointers and 32-bit values");
    typedef typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type U;
    U v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = __builtin_bit_cast(U, a[k]);
    asm("" : "+s"(v[0]), "+s"(v[1]), "+s"(v[2]), "+s"(v[3]));
    U r = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) r |= v[k] & ((U)0 - (U)(i == (uint32_t)k));
    return __builtin_bit_cast(T, r);
}

// ---------------------------------------------------------------- activation tile
// LDS layout: pairs u32 [B][nch][XPW] (XPW = NT·PPT + 4: the chunk's decode-
// ordered f16 pairs and 16 bytes of bank padding), then constants
// f32 [B][nch][NG][NCF] = (-C, s, s·Σx, 0) (NCF = 2 without the Σx term).
template <class E>
struct XTile {
    static constexpr int XPW = E::NT * E::PPT + 4;
    static constexpr int NCF = E::AFFINE ? 4 : 2;
    static constexpr uint32_t chunk_bytes = XPW * 4 + E::NG * NCF * 4;
    static_assert(chunk_bytes == xtile_chunk_bytes(E::ENC), "host/device activation tile layouts differ");
};

// f32 [n] of activation row b at element k (f32 or bf16 source), 16-byte loads.
template <bool XBF16, int N>
__device__ __forceinline__ void load_xrun(const void* __restrict__ x, size_t off, float (&v)[N]) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    if constexpr (XBF16) {
        static_assert(N % 8 == 0, "bf16 runs are read 8 at a time");
        const uint16_t* xp = static_cast<const uint16_t*>(x) + off;
#pragma unroll
        for (int i = 0; i < N; i += 8) {
            const u32x4 q = *gptr<u32x4>(xp + i);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[i + 2 * j] = __uint_as_float(q[j] << 16);
                v[i + 2 * j + 1] = __uint_as_float(q[j] & 0xFFFF0000u);
            }
        }
    } else {
        static_assert(N % 4 == 0, "f32 runs are read 4 at a time");
        const float* xp = static_cast<const float*>(x) + off;
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const f32x4 q = *gptr<f32x4>(xp + i);
#pragma unroll
            for (int j = 0; j < 4; j++) v[i + j] = q[j];
        }
    }
}

// Stages activation rows [0, batch) (rows up to B zero-filled) into the tile.
// One thread per (row, chunk): it reads the chunk's activations, picks each
// scale group's power of two s = 2^(e-14) from the group's largest magnitude
// (frexp exponent e, so |x|/s < 2^14), writes the f16 pairs in decode order
// (pairs meeting x16 codes divided by 16), and the group constants
// -C = -Σ coef·v and s·Σx over the stored values v.  All threads of the
// workgroup take part; ends with a barrier.
template <class E, int B, bool XBF16>
__device__ __forceinline__ void stage_x(uint8_t* lds, const void* __restrict__ x, uint32_t K, uint32_t ldx,
                                        uint32_t batch) {
    using XT = XTile<E>;
    const uint32_t nch = K / (uint32_t)E::CW;
    uint32_t* xp = reinterpret_cast<uint32_t*>(lds);
    float* xc = reinterpret_cast<float*>(lds + (size_t)B * nch * XT::XPW * 4u);
    for (uint32_t item = threadIdx.x; item < (uint32_t)B * nch; item += (uint32_t)kGemvThreads) {
        const uint32_t b = item / nch, u = item - b * nch;
        float v[E::NRUN][E::RUNLEN];
        if (b < batch) {
#pragma unroll
            for (int r = 0; r < E::NRUN; r++)
                load_xrun<XBF16>(x, (size_t)b * ldx + E::xbase(u) + (uint32_t)(r * E::RUNSTRIDE), v[r]);
        } else {
#pragma unroll
            for (int r = 0; r < E::NRUN; r++)
#pragma unroll
                for (int i = 0; i < E::RUNLEN; i++) v[r][i] = 0.0f;
        }
        auto val = [&](int t, int h, int e) -> float {
            const int o = E::xoff(t, h, e);
            const int r = E::NRUN > 1 ? o / (E::NRUN > 1 ? E::RUNSTRIDE : 1) : 0;
            return v[r][o - r * E::RUNSTRIDE];
        };
        int ex[E::NG];
#pragma unroll
        for (int g = 0; g < E::NG; g++) {
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < E::NT; t++)
#pragma unroll
                for (int h = 0; h < E::PPT; h++)
                    if (E::grp(t, h) == g) m = fmaxf(m, fmaxf(fabsf(val(t, h, 0)), fabsf(val(t, h, 1))));
            int e = 0;
            (void)frexpf(m, &e);
            ex[g] = e < -110 ? -110 : e;  // keeps s = 2^(e-14) a normal f32
        }
        float C[E::NG], S[E::NG];
#pragma unroll
        for (int g = 0; g < E::NG; g++) C[g] = S[g] = 0.0f;
        uint32_t pr[E::NT * E::PPT];
#pragma unroll
        for (int t = 0; t < E::NT; t++)
#pragma unroll
            for (int h = 0; h < E::PPT; h++) {
                const int g = E::grp(t, h);
                const bool dv = E::dv(t, h);
                _Float16 lo = (_Float16)ldexpf(val(t, h, 0), 14 - ex[g]);
                _Float16 hi = (_Float16)ldexpf(val(t, h, 1), 14 - ex[g]);
                if (dv) {
                    lo = lo * (_Float16)0.0625f;
                    hi = hi * (_Float16)0.0625f;
                }
                pr[t * E::PPT + h] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                                     ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
                const float fl = (float)lo, fh = (float)hi;
                C[g] = fmaf(E::coef(dv), fh, fmaf(E::coef(dv), fl, C[g]));
                S[g] = fmaf(dv ? 16.0f : 1.0f, fh, fmaf(dv ? 16.0f : 1.0f, fl, S[g]));
            }
        uint4* dst = reinterpret_cast<uint4*>(xp + (size_t)item * XT::XPW);
#pragma unroll
        for (int i = 0; i < E::NT * E::PPT; i += 4) dst[i / 4] = make_uint4(pr[i], pr[i + 1], pr[i + 2], pr[i + 3]);
#pragma unroll
        for (int g = 0; g < E::NG; g++) {
            const float s = ldexpf(1.0f, ex[g] - 14);
            float* c = xc + ((size_t)item * E::NG + g) * XT::NCF;
            if constexpr (XT::NCF == 4) {
                *reinterpret_cast<float4*>(c) = make_float4(-C[g], s, s * S[g], 0.0f);
            } else {
                *reinterpret_cast<float2*>(c) = make_float2(-C[g], s);
            }
        }
    }
    __syncthreads();
}

// Reduction over the GP (8 or 16) adjacent lanes of a scale group, all lanes
// receiving the result: xor-1, xor-2 quad permutes, then the half-row and row
// mirrors (each lane meets the other half of its 8, then of its 16).
template <int GP, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
    static_assert(GP == 8 || GP == 16, "scale groups span 8 or 16 lanes");
#define DMX_STEP(ctrl)                                                                                 \
    {                                                                                                  \
        const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false)); \
        v = MAX ? fmaxf(v, o) : v + o;                                                                 \
    }
    DMX_STEP(0xB1)   // quad_perm [1,0,3,2]
    DMX_STEP(0x4E)   // quad_perm [2,3,0,1]
    DMX_STEP(0x141)  // row_half_mirror
    if constexpr (GP == 16) DMX_STEP(0x140)  // row_mirror
#undef DMX_STEP
    return v;
}

// Same tile as stage_x, staged with one thread per f16 pair (NT·PPT threads
// per (row, chunk), PASSES rounds of the workgroup): for tiles of few chunks,
// where one thread per chunk would leave most of the workgroup idle behind a
// long serial chain.  A scale group's pairs sit on adjacent lanes inside one
// DPP row, so its largest magnitude and its constants reduce across lanes.
// The constants equal stage_x's up to the order of their f32 sums.
template <class E, int B, bool XBF16, int PASSES>
__device__ __forceinline__ void stage_x_pairs(uint8_t* lds, const void* __restrict__ x, uint32_t K, uint32_t ldx,
                                              uint32_t batch) {
    using XT = XTile<E>;
    constexpr int NP = E::NT * E::PPT;  // pairs per chunk
    constexpr int GP = NP / E::NG;      // pairs per scale group
    const uint32_t nch = K / (uint32_t)E::CW;
    const uint32_t items = (uint32_t)B * nch;
    uint32_t* xp = reinterpret_cast<uint32_t*>(lds);
    float* xc = reinterpret_cast<float*>(lds + (size_t)B * nch * XT::XPW * 4u);
    // Pair (t, h) of lane j: the GP pairs of scale group g = j / GP.
    const uint32_t j = threadIdx.x % (uint32_t)NP;  // the workgroup size is a multiple of NP
    const uint32_t g = j / (uint32_t)GP, k = j % (uint32_t)GP;
    uint32_t t, h;
    if constexpr (E::NG == 1) {
        t = j / (uint32_t)E::PPT;
        h = j % (uint32_t)E::PPT;
    } else {
        static_assert(E::NG == 4 && E::NT == 4 && E::PPT == 8, "Q6_K groups: h in {g, g + 4}, t = 0..3");
        t = k >> 1;
        h = g + 4u * (k & 1u);
    }
    const uint32_t o0 = (uint32_t)E::xoff((int)t, (int)h, 0), o1 = (uint32_t)E::xoff((int)t, (int)h, 1);
    const bool dv = E::dv((int)t, (int)h);
    // All rounds' activations are loaded before any is used, so the rounds
    // share one memory latency.
    uint32_t item[PASSES];
    bool live[PASSES];
    float v0[PASSES], v1[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ps++) {
        const uint32_t it = (threadIdx.x + (uint32_t)ps * (uint32_t)kGemvThreads) / (uint32_t)NP;
        live[ps] = it < items;
        item[ps] = live[ps] ? it : items - 1u;  // spare lanes redo the last chunk, unstored
        const uint32_t b = B == 1 ? 0u : item[ps] / nch, u = item[ps] - b * nch;
        const uint32_t base = (b < batch ? b : 0u) * ldx + E::xbase(u);  // the activations are < 4 GiB
        if constexpr (XBF16) {
            const uint16_t* xs = static_cast<const uint16_t*>(x);
            v0[ps] = __uint_as_float((uint32_t)*gptr<uint16_t>(xs + (base + o0)) << 16);
            v1[ps] = __uint_as_float((uint32_t)*gptr<uint16_t>(xs + (base + o1)) << 16);
        } else {
            const float* xs = static_cast<const float*>(x);
            v0[ps] = *gptr<float>(xs + (base + o0));
            v1[ps] = *gptr<float>(xs + (base + o1));
        }
        if (b >= batch) v0[ps] = v1[ps] = 0.0f;  // rows past the batch stage as zeros
    }
#pragma unroll
    for (int ps = 0; ps < PASSES; ps++) {
        const float m = group_reduce<GP, true>(fmaxf(fabsf(v0[ps]), fabsf(v1[ps])));
        int e = 0;
        (void)frexpf(m, &e);
        e = e < -110 ? -110 : e;  // keeps s = 2^(e-14) a normal f32
        _Float16 lo = (_Float16)ldexpf(v0[ps], 14 - e);
        _Float16 hi = (_Float16)ldexpf(v1[ps], 14 - e);
        if (dv) {
            lo = lo * (_Float16)0.0625f;
            hi = hi * (_Float16)0.0625f;
        }
        const float fl = (float)lo, fh = (float)hi;
        const float coef = dv ? E::coef(true) : E::coef(false);
        const float C = group_reduce<GP, false>(fmaf(coef, fh, coef * fl));
        const float S = group_reduce<GP, false>(dv ? 16.0f * (fl + fh) : fl + fh);
        if (live[ps]) {
            xp[(size_t)item[ps] * XT::XPW + t * (uint32_t)E::PPT + h] =
                (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            if (k == 0) {
                const float s = ldexpf(1.0f, e - 14);
                float* c = xc + ((size_t)item[ps] * E::NG + g) * XT::NCF;
                if constexpr (XT::NCF == 4) {
                    *reinterpret_cast<float4*>(c) = make_float4(-C, s, s * S, 0.0f);
                } else {
                    *reinterpret_cast<float2*>(c) = make_float2(-C, s);
                }
            }
        }
    }
    __syncthreads();
}

// Stages the activation tile.  When every wave of the grid has at most one
// row block the launch is latency-bound and the tile is staged one thread per
// pair (up to four rounds of the workgroup); otherwise the weight stream is
// long and the one-thread-per-chunk stager, which spends a fraction of the
// instructions, is used.
template <class E, int B, bool XBF16>
__device__ __forceinline__ void stage_x_auto(uint8_t* lds, const GemvParams& p) {
    const void* x = p.x;
    const uint32_t K = p.K, ldx = p.ldx, batch = p.batch;
    const uint32_t pairs = (uint32_t)B * (K / (uint32_t)E::CW) * (uint32_t)(E::NT * E::PPT);
    const bool latency_bound = p.total_rb <= p.grid * (uint32_t)(kGemvThreads / 64);
    if (!latency_bound) stage_x<E, B, XBF16>(lds, x, K, ldx, batch);
    else if (pairs <= 1u * kGemvThreads) stage_x_pairs<E, B, XBF16, 1>(lds, x, K, ldx, batch);
    else if (pairs <= 2u * kGemvThreads) stage_x_pairs<E, B, XBF16, 2>(lds, x, K, ldx, batch);
    else if (pairs <= 4u * kGemvThreads) stage_x_pairs<E, B, XBF16, 4>(lds, x, K, ldx, batch);
    else stage_x<E, B, XBF16>(lds, x, K, ldx, batch);
}

// ---------------------------------------------------------------- chunk dot product
// Reads the (-C, s, s·Σx) constants of group g of chunk u for activation row b.
template <class E>
__device__ __forceinline__ void load_consts(const float* xc, uint32_t idx, float& negc, float& s, float& sm) {
    using XT = XTile<E>;
    const float* cp = xc + (size_t)idx * XT::NCF;
    if constexpr (XT::NCF == 4) {
        const float4 q = *reinterpret_cast<const float4*>(cp);
        negc = q.x;
        s = q.y;
        sm = q.z;
    } else {
        const float2 q = *reinterpret_cast<const float2*>(cp);
        negc = q.x;
        s = q.y;
        sm = 0.0f;
    }
}

// The PPT activation pairs of code dword t of chunk u, activation row b.
template <class E>
__device__ __forceinline__ void load_xpairs(const uint32_t* xp, uint32_t idx, int t, uint32_t (&xv)[E::PPT]) {
    const uint32_t* xq = xp + (size_t)idx * XTile<E>::XPW + t * E::PPT;
    if constexpr (E::PPT % 4 == 0) {
#pragma unroll
        for (int h = 0; h < E::PPT; h += 4) {
            const uint4 q = *reinterpret_cast<const uint4*>(xq + h);
            xv[h] = q.x; xv[h + 1] = q.y; xv[h + 2] = q.z; xv[h + 3] = q.w;
        }
    } else {
        static_assert(E::PPT == 2, "pairs per code dword: 2, 4 or 8");
        const uint2 q = *reinterpret_cast<const uint2*>(xq);
        xv[0] = q.x; xv[1] = q.y;
    }
}

// y[i][b] += Σ over chunk u of row i: w·x, for R rows and B activation rows.
// Up to 4 activation rows: code dword outer (each dword's pairs are decoded
// and used at once, R·B·NG accumulators).  More rows: activation row outer
// (the chunk's pairs are decoded once and kept, R·NG accumulators), which
// keeps the registers of the wide batches in check.
template <class E, int R, int B>
__device__ __forceinline__ void chunk_dot(const typename E::Chunk (&c)[R], const uint8_t* lds, uint32_t nch,
                                          uint32_t u, float (&y)[R][B]) {
    using XT = XTile<E>;
    const uint32_t* xp = reinterpret_cast<const uint32_t*>(lds);
    const float* xc = reinterpret_cast<const float*>(lds + (size_t)B * nch * XT::XPW * 4u);
    if constexpr (B <= 4) {
        float acc[R][B][E::NG];
        float sc[B][E::NG], sm[B][E::NG];
#pragma unroll
        for (int b = 0; b < B; b++)
#pragma unroll
            for (int g = 0; g < E::NG; g++) {
                float negc;
                load_consts<E>(xc, ((uint32_t)b * nch + u) * E::NG + g, negc, sc[b][g], sm[b][g]);
#pragma unroll
                for (int i = 0; i < R; i++) acc[i][b][g] = negc;
            }
#pragma unroll
        for (int t = 0; t < E::NT; t++) {
            uint32_t pr[R][E::PPT];
#pragma unroll
            for (int i = 0; i < R; i++) E::pairs(c[i], t, pr[i]);
#pragma unroll
            for (int b = 0; b < B; b++) {
                uint32_t xv[E::PPT];
                load_xpairs<E>(xp, (uint32_t)b * nch + u, t, xv);
#pragma unroll
                for (int i = 0; i < R; i++)
#pragma unroll
                    for (int h = 0; h < E::PPT; h++) {
                        float& a = acc[i][b][E::grp(t, h)];
                        a = dot2(pr[i][h], xv[h], a);
                    }
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int b = 0; b < B; b++)
#pragma unroll
                for (int g = 0; g < E::NG; g++) {
                    // weight scale first: d·acc·s is the group's true contribution,
                    // while acc·s alone (Σ q·x) can overflow f32 for huge activations
                    y[i][b] = fmaf(E::gscale(c[i], g) * acc[i][b][g], sc[b][g], y[i][b]);
                    if constexpr (E::AFFINE) y[i][b] = fmaf(E::goffset(c[i], g), sm[b][g], y[i][b]);
                }
    } else {
        uint32_t pr[R][E::NT][E::PPT];
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int t = 0; t < E::NT; t++) E::pairs(c[i], t, pr[i][t]);
#pragma unroll
        for (int b = 0; b < B; b++) {
            float acc[R][E::NG], sc[E::NG], sm[E::NG];
#pragma unroll
            for (int g = 0; g < E::NG; g++) {
                float negc;
                load_consts<E>(xc, ((uint32_t)b * nch + u) * E::NG + g, negc, sc[g], sm[g]);
#pragma unroll
                for (int i = 0; i < R; i++) acc[i][g] = negc;
            }
#pragma unroll
            for (int t = 0; t < E::NT; t++) {
                uint32_t xv[E::PPT];
                load_xpairs<E>(xp, (uint32_t)b * nch + u, t, xv);
#pragma unroll
                for (int i = 0; i < R; i++)
#pragma unroll
                    for (int h = 0; h < E::PPT; h++) {
                        float& a = acc[i][E::grp(t, h)];
                        a = dot2(pr[i][t][h], xv[h], a);
                    }
            }
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int g = 0; g < E::NG; g++) {
                    y[i][b] = fmaf(E::gscale(c[i], g) * acc[i][g], sc[g], y[i][b]);
                    if constexpr (E::AFFINE) y[i][b] = fmaf(E::goffset(c[i], g), sm[g], y[i][b]);
                }
            // one activation row's LDS reads in flight at a time: hoisting all of
            // them (which the optimiser does before scheduling) would spill
            asm volatile("" ::: "memory");
        }
    }
}

// Row block -> its problem's pointers, row count and first row (all wave-
// uniform, computed once per task in scalar registers).
struct RowBlock {
    const uint8_t* w;
    const uint8_t* sc;
    const uint8_t* bi;
    void* y;
    uint32_t n, base;
};

__device__ __forceinline__ RowBlock row_block(const GemvParams& p, uint32_t rb, uint32_t rows_per_rb) {
    uint32_t pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; i++) pi += (i < (int)p.nprob && rb >= p.rb_begin[i]) ? 1u : 0u;
    RowBlock r;
    r.w = pick(pi, p.w);
    r.sc = pick(pi, p.sc);
    r.bi = pick(pi, p.bi);
    r.y = pick(pi, p.y);
    r.n = pick(pi, p.n);
    r.base = (rb - pick(pi, p.rb_begin)) * rows_per_rb;
    return r;
}

// Sum over each aligned group of L lanes (L a power of two <= 64, wave-
// uniform), left in every lane of the group: DPP butterflies within rows of
// 16 lanes (quad permutes, then the half-row and row mirrors, which pair every
// lane with one of the other half once the halves are uniform), then the
// gfx950 row-pair and half-wave swaps.  All VALU, no LDS round trips.
__device__ __forceinline__ float group_sum(float v, uint32_t L) {
#define DMX_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false))
    if (L >= 2) v += DMX_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    if (L >= 4) v += DMX_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    if (L >= 8) v += DMX_DPP(v, 0x141);  // row_half_mirror
    if (L >= 16) v += DMX_DPP(v, 0x140); // row_mirror
#undef DMX_DPP
    if (L >= 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if (L >= 64) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

template <int R, int B>
__device__ __forceinline__ void reduce_store(float (&acc)[R][B], const RowBlock& rb, uint32_t row0, uint32_t j,
                                             uint32_t L, const GemvParams& p) {
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[i][b] = group_sum(acc[i][b], L);
    if (j == 0) {
        void* y = rb.y;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t row = row0 + (uint32_t)i;
            if (row >= rb.n) continue;
#pragma unroll
            for (int b = 0; b < B; b++) {
                if ((uint32_t)b < p.batch) {
                    const size_t idx = (size_t)b * rb.n + row;
                    // global (not flat) stores: a flat store makes the wait counters
                    // drain every load in flight
                    if (p.y_bf16) gptr_mut<uint16_t>(y)[idx] = f32_to_bf16_bits(acc[i][b]);
                    else gptr_mut<float>(y)[idx] = acc[i][b];
                }
            }
        }
    }
}

// The persistent task pipeline shared by all encodings.  load(rb, row, u)
// returns the raw bytes of chunk u of a row (rows past the end are clamped to
// the last row: in bounds, their sums are never stored).  Every load is
// unconditional — a wave without row blocks loads the last row block's first
// task, and at the end of the sequence the current task is loaded again — so
// the compiler's wait counters can keep a lane's loads in flight across one
// task of compute.  stage() stages the activations (with a barrier); it runs
// after the first task's loads are issued, in every wave.
template <class E, int R, int B, class LOAD, class STAGE>
__device__ __forceinline__ void gemv_pipeline(const GemvParams& p, const uint8_t* lds, LOAD&& load, STAGE&& stage) {
    const uint32_t lane = threadIdx.x & 63u;
    // The launch shape comes from compile-time constants and the parameters:
    // reading blockDim/gridDim costs a load from the dispatch packet that the
    // first weight loads would wait behind.
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)(kGemvThreads / 64) + (threadIdx.x >> 6));
    const uint32_t W = p.grid * (uint32_t)(kGemvThreads / 64);
    const uint32_t L = 1u << p.lanes_log2;
    const uint32_t j = lane & (L - 1u), g = lane >> p.lanes_log2;
    const uint32_t rows_per_rb = (64u >> p.lanes_log2) * (uint32_t)R;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const uint32_t cpl = (nch + L - 1u) >> p.lanes_log2;  // chunks per lane per row block
    const uint32_t T = wid < p.total_rb ? (p.total_rb - wid + W - 1) / W * cpl : 0u;  // tasks of this wave

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[i][b] = 0.0f;

    auto load_task = [&](typename E::Raw (&dst)[R], const RowBlock& rb, uint32_t c) {
        const uint32_t row0 = rb.base + g * (uint32_t)R;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t row = row0 + (uint32_t)i < rb.n ? row0 + (uint32_t)i : rb.n - 1u;
            const uint32_t u = j + c * L;
            dst[i] = load(rb, row, u < nch ? u : nch - 1u);
        }
    };

    // Two register buffers in ping-pong (no copies between them, so waiting
    // for one buffer never waits for the loads in flight into the other).
    typename E::Raw ba[R], bb[R];
    uint32_t nrb = wid < p.total_rb ? wid : p.total_rb - 1u, nc = 0;  // the task loaded next
    RowBlock nblk = row_block(p, nrb, rows_per_rb);
    // wave-uniform and branch-free; past the end the last task is loaded again
    auto advance = [&](uint32_t t) {
        const bool more = t + 1 < T;
        const bool wrap = more && nc + 1 == cpl;
        nc = wrap ? 0u : (more ? nc + 1 : nc);
        nrb = wrap ? nrb + W : nrb;
        nblk = row_block(p, nrb, rows_per_rb);
    };
    auto compute = [&](const typename E::Raw (&buf)[R], const RowBlock& blk, uint32_t c) {
        const uint32_t u0 = j + c * L;
        const bool past = u0 >= nch;  // a lane past the last chunk: adds zero
        const uint32_t u = past ? nch - 1u : u0;
        typename E::Chunk ch[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            ch[i] = E::unpack(buf[i], u);
            E::zero_if(ch[i], past);
        }
        chunk_dot<E, R, B>(ch, lds, nch, u, acc);
        if (c + 1 == cpl) {
            reduce_store<R, B>(acc, blk, blk.base + g * (uint32_t)R, j, L, p);
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int b = 0; b < B; b++) acc[i][b] = 0.0f;
        }
    };
    load_task(ba, nblk, nc);
    stage();
    if (T == 0) return;
    uint32_t t = 0;
    for (; t + 2 <= T; t += 2) {
        // task t is in ba: load task t+1 into bb, compute ba
        RowBlock blk = nblk;
        uint32_t c = nc;
        advance(t);
        load_task(bb, nblk, nc);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the compute
        compute(ba, blk, c);
        // task t+1 is in bb: load task t+2 into ba, compute bb
        blk = nblk;
        c = nc;
        advance(t + 1);
        load_task(ba, nblk, nc);
        __builtin_amdgcn_sched_barrier(0);
        compute(bb, blk, c);
    }
    if (t < T) compute(ba, nblk, nc);  // odd task count: the last task is in ba
}

// Latency mode: every wave owns at most one row block of one row per lane
// group (total row blocks <= waves launched), so there is no task loop.  A
// lane issues the loads of all CPL of its chunks before the activations are
// staged, so the whole launch waits on one memory latency; then it
// multiplies them for the B activation rows, the L lanes reduce, and lane 0
// stores.
template <class E, int CPL, int B, class LOAD, class STAGE>
__device__ __forceinline__ void gemv_oneshot(const GemvParams& p, const uint8_t* lds, LOAD&& load, STAGE&& stage) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)(kGemvThreads / 64) + (threadIdx.x >> 6));
    const uint32_t L = 1u << p.lanes_log2;
    const uint32_t j = lane & (L - 1u), g = lane >> p.lanes_log2;
    const uint32_t rows_per_rb = 64u >> p.lanes_log2;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const bool active = wid < p.total_rb;
    const RowBlock blk = row_block(p, active ? wid : p.total_rb - 1u, rows_per_rb);
    const uint32_t row = blk.base + g < blk.n ? blk.base + g : blk.n - 1u;
    typename E::Raw buf[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const uint32_t u = j + (uint32_t)c * L;
        buf[c] = load(blk, row, u < nch ? u : nch - 1u);
    }
    stage();
    if (!active) return;
    float acc[1][B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[0][b] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const uint32_t u0 = j + (uint32_t)c * L;
        const bool past = u0 >= nch;  // a lane past the last chunk: adds zero
        const uint32_t u = past ? nch - 1u : u0;
        typename E::Chunk ch[1];
        ch[0] = E::unpack(buf[c], u);
        E::zero_if(ch[0], past);
        chunk_dot<E, 1, B>(ch, lds, nch, u, acc);
    }
    reduce_store<1, B>(acc, blk, blk.base + g, j, L, p);
}

// ---------------------------------------------------------------- GGUF
// Weight offsets are 32-bit (the C ABI limits one weight to 4 GiB), so loads
// use a uniform 64-bit base plus a per-lane 32-bit offset.
template <class E, int B, int R, bool XBF16>
__global__ __launch_bounds__(kGemvThreads) void gguf_gemv_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    const uint32_t rowbytes = (p.K / (uint32_t)E::QK) * (uint32_t)E::BB;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) { return E::load(rb.w, row * rowbytes, u); };
    gemv_pipeline<E, R, B>(p, xlds, load, [&] { stage_x_auto<E, B, XBF16>(xlds, p); });
}

template <class E, int CPL, int B, bool XBF16>
__global__ __launch_bounds__(kGemvThreads) void gguf_gemv_oneshot_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    const uint32_t rowbytes = (p.K / (uint32_t)E::QK) * (uint32_t)E::BB;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) { return E::load(rb.w, row * rowbytes, u); };
    gemv_oneshot<E, CPL, B>(p, xlds, load, [&] { stage_x_auto<E, B, XBF16>(xlds, p); });
}

// ---------------------------------------------------------------- MLX affine U4
// Raw bytes of chunk u of a row: 16 bytes of packed words plus the group's
// scale and bias (f32, or f16/bf16 bits).
struct MlxLoad {
    const GemvParams& p;
    uint32_t ngroups, chunks_per_group;
    bool f32s;
    __device__ __forceinline__ explicit MlxLoad(const GemvParams& q)
        : p(q), ngroups(q.K / q.group), chunks_per_group(q.group / 32u), f32s(q.sdtype == DT_F32) {}
    __device__ __forceinline__ EncMlxU4::Raw operator()(const RowBlock& rb, uint32_t row, uint32_t u) const {
        EncMlxU4::Raw r;
        const uint8_t* wb = rb.w;
        load_dwords<4>(reinterpret_cast<const uint32_t*>(wb + (row * (p.K / 2u) + u * 16u)), r.w);
        const uint32_t gi = row * ngroups + u / chunks_per_group;
        const uint8_t* scb = rb.sc;
        const uint8_t* bib = rb.bi;
        if (f32s) {
            r.s = *gptr<uint32_t>(scb + gi * 4u);
            r.b = *gptr<uint32_t>(bib + gi * 4u);
        } else {
            r.s = *gptr<uint16_t>(scb + gi * 2u);
            r.b = *gptr<uint16_t>(bib + gi * 2u);
        }
        r.kind = p.sdtype;
        return r;
    }
};

template <int B, int R, bool XBF16>
__global__ __launch_bounds__(kGemvThreads) void mlx_u4_gemv_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    gemv_pipeline<EncMlxU4, R, B>(p, xlds, MlxLoad(p), [&] { stage_x_auto<EncMlxU4, B, XBF16>(xlds, p); });
}

template <int CPL, int B, bool XBF16>
__global__ __launch_bounds__(kGemvThreads) void mlx_u4_gemv_oneshot_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    gemv_oneshot<EncMlxU4, CPL, B>(p, xlds, MlxLoad(p), [&] { stage_x_auto<EncMlxU4, B, XBF16>(xlds, p); });
}

// Rows per lane group for a register batch B: more rows amortise each
// activation read from LDS and the per-task overhead, fewer keep the
// accumulators in registers.  (With one activation row the host may pick a
// single row per group instead, for matrices too small to fill the GPU.)
template <class E, int B>
constexpr int rows_per_group() {
    if constexpr (E::ENC == ENC_Q6_K) return B <= 2 ? 2 : 1;
    else return B <= 2 ? 4 : 2;
}

// The narrower tile instantiated beside it for activation rows > 1, taken by
// the host when the wider one would leave too few row blocks for the GPU
// (halving the rows gives twice the waves at fewer registers each).
template <class E, int B>
constexpr int rows_per_group_narrow() {
    return rows_per_group<E, B>() > 1 ? rows_per_group<E, B>() / 2 : 1;
}

// Resident workgroups per CU for (kernel, dynamic LDS) on the current device
// and its CU count, cached after the first query (host side, thread-safe).
// Also raises the kernel's dynamic-LDS limit when lds needs it.
hipError_t cached_occupancy(const void* kernel, size_t lds, int threads, int* per_cu, int* cus);

// Launch of one kernel instantiation with a persistent grid: as many waves as
// fit on the device at once (capped by the row-block count).  Fewer waves
// would even out the row blocks per wave, but cost more in memory-level
// parallelism than the tail they save.
template <class KERNEL>
hipError_t launch_persistent(KERNEL kernel, const GemvParams& p, size_t lds, hipStream_t st) {
    int cus = 0, per_cu = 0;
    hipError_t e = cached_occupancy(reinterpret_cast<const void*>(kernel), lds, kGemvThreads, &per_cu, &cus);
    if (e != hipSuccess) return e;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    constexpr uint64_t waves = kGemvThreads / 64;
    const uint64_t want = ((uint64_t)p.total_rb + waves - 1) / waves;
    const uint64_t cap = (uint64_t)per_cu * (uint64_t)cus;
    const uint32_t blocks = (uint32_t)(want < cap ? want : cap);
    GemvParams q = p;
    q.grid = blocks;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kGemvThreads), lds, st, q);
    return hipGetLastError();
}

// Latency-mode launch: one wave per row block.
template <class KERNEL>
hipError_t launch_oneshot(KERNEL kernel, const GemvParams& p, size_t lds, hipStream_t st) {
    if (lds > 64u * 1024u) {
        int cus = 0, per_cu = 0;
        hipError_t e = cached_occupancy(reinterpret_cast<const void*>(kernel), lds, kGemvThreads, &per_cu, &cus);
        if (e != hipSuccess) return e;
    }
    constexpr uint32_t waves = kGemvThreads / 64;
    GemvParams q = p;
    q.grid = (p.total_rb + waves - 1) / waves;
    hipLaunchKernelGGL(kernel, dim3(q.grid), dim3(kGemvThreads), lds, st, q);
    return hipGetLastError();
}

// Instantiates and launches the GEMV kernel of encoding E for a power-of-two
// register batch B (the host has checked that its activation tile fits LDS);
// oneshot = chunks per lane selects the latency-mode kernel.
// GGUF decode takes f32 activations, the reference's precision contract for
// quantized linears (crates/dyninfer-compiler/src/lib.rs:289-306); bf16
// activations reach GGUF weights only through the Q4_0 MFMA path.
template <class E>
hipError_t launch_gguf_gemv(const GemvParams& p, uint32_t B, uint32_t R, uint32_t oneshot, bool xbf16,
                            hipStream_t st) {
    if (xbf16) return hipErrorInvalidValue;
    const size_t lds = (size_t)xtile_bytes(E::ENC, B, p.K);
    if (oneshot) {
        // chunks per lane (the host's limits): 1..4 for one activation row
        // (Q6_K 1..2), 1..2 for 2 rows, 1 for 4
        if (R != 1) return hipErrorInvalidValue;
#define DMX_ONESHOT(b, c)                                                                             \
    if (B == b && oneshot == c) return launch_oneshot(gguf_gemv_oneshot_kernel<E, c, b, false>, p, lds, st);
        DMX_ONESHOT(1, 1)
        DMX_ONESHOT(1, 2)
        if constexpr (E::ENC != ENC_Q6_K) {
            DMX_ONESHOT(1, 3)
            DMX_ONESHOT(1, 4)
        }
        if constexpr (max_register_batch(E::ENC) >= 2) {
            DMX_ONESHOT(2, 1)
            DMX_ONESHOT(2, 2)
        }
        if constexpr (max_register_batch(E::ENC) >= 4) DMX_ONESHOT(4, 1)
#undef DMX_ONESHOT
        return hipErrorInvalidValue;
    }
    if (B == 1 && R == 1) return launch_persistent(gguf_gemv_kernel<E, 1, 1, false>, p, lds, st);
#define DMX_CASE(b)                                                                                       \
    case b:                                                                                               \
        if constexpr (b <= max_register_batch(E::ENC)) {                                                  \
            if (R == (uint32_t)rows_per_group<E, b>())                                                    \
                return launch_persistent(gguf_gemv_kernel<E, b, rows_per_group<E, b>(), false>, p, lds, st); \
            if constexpr (b > 1)                                                                          \
                if (R == (uint32_t)rows_per_group_narrow<E, b>())                                         \
                    return launch_persistent(gguf_gemv_kernel<E, b, rows_per_group_narrow<E, b>(), false>, p, \
                                             lds, st);                                                    \
        }                                                                                                 \
        return hipErrorInvalidValue;
    switch (B) {
        DMX_CASE(1)
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef DMX_CASE
}

}  // namespace dmx
