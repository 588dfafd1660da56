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
//     current task is computed, and the first task's right after the
//     activation loads (before the staging arithmetic), so HBM latency
//     overlaps staging and arithmetic;
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

// Activations off..off+3 of the source as f32 (f32 or bf16 source).  off is a
// multiple of 4 and rows start 16-byte aligned, so this is one aligned 16-byte
// (f32) or 8-byte (bf16) load.
template <bool XBF16>
__device__ __forceinline__ void load_x4(const void* __restrict__ x, uint32_t off, float (&v)[4]) {
    if constexpr (XBF16) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 q = *gptr<u32x2>(static_cast<const uint16_t*>(x) + off);
        v[0] = __uint_as_float(q[0] << 16);
        v[1] = __uint_as_float(q[0] & 0xFFFF0000u);
        v[2] = __uint_as_float(q[1] << 16);
        v[3] = __uint_as_float(q[1] & 0xFFFF0000u);
    } else {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 q = *gptr<f32x4>(static_cast<const float*>(x) + off);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = q[i];
    }
}

// Reduction over the N (4 or 8) adjacent lanes of one chunk, every lane
// receiving the result: xor-1 and xor-2 quad permutes, then for 8 lanes the
// half-row mirror (each quad meets the other quad of its 8).  Every lane adds
// the same operands (commuted), so all hold the same value.
template <int N, class OP>
__device__ __forceinline__ uint32_t lanes_reduce(uint32_t v, OP op) {
    static_assert(N == 4 || N == 8, "a chunk's code dwords span 4 or 8 lanes");
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    if constexpr (N == 8) v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    return v;
}

// max(|a|, |b|, |c|) as one v_max3_f32 with abs modifiers (the compiler's
// fmaxf would first canonicalise each loaded value).  A NaN operand can only
// change the scale exponent it feeds.
__device__ __forceinline__ float absmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Staging threads per scale group (activation row b, chunk u, group g): SP
// adjacent threads (SP = 1, 2 or 4, dividing NT) share a group, thread q
// taking code dwords t = q·NT/SP .. (q+1)·NT/SP - 1.  Pair h = g + NG·k of
// code dword t belongs to group g (grp(t, h) = h mod NG); a thread loads, for
// each of its code dwords, the group's runs of 4 activations (NXR runs for
// one-group chunks, run g otherwise, at xrun0(r) + TSTRIDE·t), takes the
// group's largest magnitude and sums over its SP lanes (DPP, no LDS), and
// stores its pairs.  With SP = 1 a group needs no cross-lane step at all;
// wider SP spreads the group over more lanes, which keeps each load
// instruction's addresses denser (fewer cache lines per instruction) when
// the workgroup has threads to spare.  Checked at compile time by
// group_runs_ok: the positions of group g are those of group 0 shifted by
// RUNSTRIDE·g = xrun0(g).
template <class E>
constexpr bool group_runs_ok() {
    for (int t = 0; t < E::NT; t++)
        for (int h = 0; h < E::PPT; h++)
            for (int e = 0; e < 2; e++) {
                const int g = h % E::NG;
                if (E::grp(t, h) != g) return false;
                if (E::xoff(t, h, e) - E::RUNSTRIDE * g != E::xoff(t, h - g, e)) return false;
                if (E::NG > 1 && xrun_of<E>(h - g, e) != 0) return false;  // group 0 reads run 0 only
                if (E::dv(t, h) != E::dv(0, h)) return false;               // the x16 flag is per pair slot
            }
    if (E::NG > 1) {
        if (E::NXR != E::NG) return false;
        for (int r = 0; r < E::NXR; r++)
            if (E::xrun0(r) != E::RUNSTRIDE * r) return false;
    }
    return E::PPT % E::NG == 0;
}

// op over the SP adjacent lanes of a group (SP = 1, 2, 4), the result in every lane
template <int SP, class OP>
__device__ __forceinline__ uint32_t sp_reduce(uint32_t v, OP op) {
    if constexpr (SP >= 2) v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    if constexpr (SP >= 4) v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    return v;
}

template <class E, int SP>
struct GStage {
    static constexpr int TT = E::NT / SP;                   // code dwords per thread
    static constexpr int RPG = E::NG == 1 ? E::NXR : 1;     // runs of 4 per code dword in one group
    float v[TT][RPG][4];
    uint32_t item;  // b·nch + u
    uint32_t g;     // scale group within the chunk
    uint32_t q;     // part of the group (code dwords q·TT ..)
    bool live;      // the group exists: the thread stores
};

// Issues the loads of staging thread idx (the values are not used here, so
// loads issued after this are not waited for).
template <class E, int SP, int B, bool XBF16>
__device__ __forceinline__ void gstage_load(const GemvParams& p, uint32_t nch, uint32_t idx, GStage<E, SP>& s) {
    using S = GStage<E, SP>;
    const uint32_t groups = (uint32_t)B * nch * (uint32_t)E::NG;
    s.q = SP == 1 ? 0u : idx % (uint32_t)SP;
    const uint32_t gi0 = SP == 1 ? idx : idx / (uint32_t)SP;
    s.live = gi0 < groups;
    const uint32_t gi = s.live ? gi0 : groups - 1u;  // spare lanes redo the last group, unstored
    s.g = E::NG == 1 ? 0u : gi % (uint32_t)E::NG;
    s.item = E::NG == 1 ? gi : gi / (uint32_t)E::NG;
    const uint32_t b = B == 1 ? 0u : s.item / nch, u = s.item - b * nch;
    // Rows past the batch restage row 0: in bounds, and their sums are never
    // stored.  Activation offsets are 32-bit (the activations are < 4 GiB).
    const uint32_t base = (b < p.batch ? b : 0u) * p.ldx + E::xbase(u) + (uint32_t)E::RUNSTRIDE * s.g +
                          (uint32_t)E::TSTRIDE * (uint32_t)S::TT * s.q;
#pragma unroll
    for (int tt = 0; tt < S::TT; tt++)
#pragma unroll
        for (int r = 0; r < S::RPG; r++)
            load_x4<XBF16>(p.x, base + (uint32_t)(E::xrun0(r) + E::TSTRIDE * tt), s.v[tt][r]);
}

// The rest of staging thread s: the group's power of two s = 2^(e-14) from
// its largest magnitude (frexp exponent e, so |x|/s < 2^14), its pairs in
// decode order (one RNE rounding of x/s, or of x/(16s) for pairs meeting x16
// codes) and, from part q = 0, the constants -C = -Σ coef·v and s·Σx over the
// stored values v (f32 sums over the SP parts).
template <class E, int SP, int B>
__device__ __forceinline__ void gstage_store(uint8_t* lds, uint32_t nch, const GStage<E, SP>& s) {
    using XT = XTile<E>;
    using S = GStage<E, SP>;
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    constexpr int KP = E::PPT / E::NG, NV = S::TT * S::RPG * 4;
    const float* vv = &s.v[0][0][0];
    // largest magnitude: independent triples, then their maximum
    float m3[(NV + 2) / 3];
#pragma unroll
    for (int i = 0; i < NV; i += 3) m3[i / 3] = absmax3(vv[i], vv[i + 1 < NV ? i + 1 : i], vv[i + 2 < NV ? i + 2 : i]);
    constexpr int N3 = (NV + 2) / 3;
    float m = m3[0];
#pragma unroll
    for (int i = 1; i < N3; i += 2) m = absmax3(m, m3[i], m3[i + 1 < N3 ? i + 1 : i]);
    uint32_t mx = sp_reduce<SP>(__float_as_uint(m), [](uint32_t a, uint32_t b) { return a > b ? a : b; });
    int ex = 0;
    (void)frexpf(__uint_as_float(mx), &ex);  // non-negative floats order as integers
    ex = ex < -110 ? -110 : ex;                // keeps s = 2^(e-14) a normal f32
    uint32_t pr[S::TT][KP];
    float C[2] = {0.0f, 0.0f}, Sx[2] = {0.0f, 0.0f};  // two chains each
#pragma unroll
    for (int tt = 0; tt < S::TT; tt++)
#pragma unroll
        for (int k = 0; k < KP; k++) {
            const int h0 = E::NG * k;  // pair h0 + g of code dword q·TT + tt
            const bool dv = E::NG == 1 ? E::dv(0, h0) : E::dv(0, h0 + (int)s.g);
            const int sh = (dv ? 10 : 14) - ex;
            auto val = [&](int e) {
                const int r = xrun_of<E>(h0, e);
                return s.v[tt][r][E::xoff(0, h0, e) - E::xrun0(r)];
            };
            const f32x2 f = {ldexpf(val(0), sh), ldexpf(val(1), sh)};
            pr[tt][k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));  // v_cvt_pk_f16_f32 (RNE)
            const uint32_t c1 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)E::coef(false)) * 0x00010001u;
            const uint32_t c16 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)E::coef(true)) * 0x00010001u;
            const int ch = (tt * KP + k) & 1;
            C[ch] = dot2(pr[tt][k], dv ? c16 : c1, C[ch]);
            if constexpr (XT::NCF == 4) Sx[ch] = dot2(pr[tt][k], dv ? 0x4C004C00u : 0x3C003C00u, Sx[ch]);  // (16, 16) or (1, 1)
        }
    auto fadd = [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); };
    const float Ct = __uint_as_float(sp_reduce<SP>(__float_as_uint(C[0] + C[1]), fadd));
    float St = 0.0f;
    if constexpr (XT::NCF == 4) St = __uint_as_float(sp_reduce<SP>(__float_as_uint(Sx[0] + Sx[1]), fadd));
    if (s.live) {
        uint32_t* xp = reinterpret_cast<uint32_t*>(lds) + (size_t)s.item * XT::XPW + s.q * (uint32_t)(S::TT * E::PPT);
        float* xc = reinterpret_cast<float*>(lds + (size_t)B * nch * XT::XPW * 4u);
        if constexpr (E::NG == 1 && (S::TT * E::PPT) % 4 == 0) {
            // the thread's pairs are TT·PPT consecutive dwords
#pragma unroll
            for (int i = 0; i < S::TT * E::PPT; i += 4)
                *reinterpret_cast<uint4*>(xp + i) =
                    make_uint4(pr[i / KP][i % KP], pr[(i + 1) / KP][(i + 1) % KP], pr[(i + 2) / KP][(i + 2) % KP],
                               pr[(i + 3) / KP][(i + 3) % KP]);
        } else if constexpr (E::NG == 1 && (S::TT * E::PPT) % 2 == 0) {
#pragma unroll
            for (int i = 0; i < S::TT * E::PPT; i += 2)
                *reinterpret_cast<uint2*>(xp + i) = make_uint2(pr[i / KP][i % KP], pr[(i + 1) / KP][(i + 1) % KP]);
        } else {
#pragma unroll
            for (int tt = 0; tt < S::TT; tt++)
#pragma unroll
                for (int k = 0; k < KP; k++) xp[tt * E::PPT + E::NG * k + (int)s.g] = pr[tt][k];
        }
        if (s.q == 0) {
            const float sc = ldexpf(1.0f, ex - 14);
            float* c = xc + ((size_t)s.item * E::NG + s.g) * XT::NCF;
            if constexpr (XT::NCF == 4) {
                *reinterpret_cast<float4*>(c) = make_float4(-Ct, sc, sc * St, 0.0f);
            } else {
                *reinterpret_cast<float2*>(c) = make_float2(-Ct, sc);
            }
        }
    }
}

// Stages activation rows [0, batch) into the tile (rows up to B restage row
// 0): B·nch·NG·SP staging threads in rounds of TH (the workgroup size).  The
// first round's activation loads are issued, then mid() (the caller's first
// weight loads), then the first round is computed: loads return in issue
// order, so the activations arrive ahead of the weights and the staging
// arithmetic runs while the weights are in flight.  Waves with no group in a
// round skip it (a wave-uniform branch).  Later rounds (long rows, large
// batches) load after the weights.  Ends with a barrier.
template <class E, int SP, int B, bool XBF16, int TH, class MID>
__device__ __forceinline__ void stage_x_sp(uint8_t* lds, const GemvParams& p, MID&& mid) {
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const uint32_t total = (uint32_t)B * nch * (uint32_t)E::NG * (uint32_t)SP;
    const uint32_t wave0 = threadIdx.x & ~63u;  // first thread of this wave
    GStage<E, SP> s;
    const bool first = wave0 < total;
    if (first) gstage_load<E, SP, B, XBF16>(p, nch, threadIdx.x, s);
    __builtin_amdgcn_sched_barrier(0);
    mid();
    __builtin_amdgcn_sched_barrier(0);
    if (first) gstage_store<E, SP, B>(lds, nch, s);
    for (uint32_t base = TH; base < total; base += TH) {
        if (base + wave0 < total) {
            gstage_load<E, SP, B, XBF16>(p, nch, base + threadIdx.x, s);
            gstage_store<E, SP, B>(lds, nch, s);
        }
    }
    __syncthreads();
}

// ---- Staging of several f32 activation rows: one thread per code dword.
// Its loads are the densest (consecutive lanes on consecutive 16-byte runs),
// which matters once the rows hold many groups: thread-per-group staging of 4
// rows of 4096 (512 groups, eight 16-byte loads per lane 128 bytes apart, a
// cache line per lane per load) took ~4 us before the first product, and the
// Qwen3-8B GGUF step at 4 rows ran 2.50 ms against 2.31 ms with this staging.
// One staging thread's share: code dword t = idx % NT of (activation row,
// chunk) item = idx / NT; its NXR runs of 4 activations.
template <class E>
struct XStage {
    float v[E::NXR][4];
    uint32_t item;
    bool live;  // item < B·nch: the thread stores
};

// Issues the loads of staging thread idx (no use of the loaded values, so
// loads issued after it are not waited for).
template <class E, int B, bool XBF16>
__device__ __forceinline__ void xstage_load(const GemvParams& p, uint32_t nch, uint32_t idx, XStage<E>& s) {
    const uint32_t items = (uint32_t)B * nch;
    const uint32_t it = idx / (uint32_t)E::NT, t = idx % (uint32_t)E::NT;
    s.live = it < items;
    s.item = s.live ? it : items - 1u;  // spare threads redo the last chunk, unstored
    const uint32_t b = B == 1 ? 0u : s.item / nch, u = s.item - b * nch;
    // Rows past the batch restage row 0: in bounds, and their sums are never
    // stored.  Activation offsets are 32-bit (the activations are < 4 GiB).
    const uint32_t base = (b < p.batch ? b : 0u) * p.ldx + E::xbase(u) + (uint32_t)E::TSTRIDE * t;
#pragma unroll
    for (int r = 0; r < E::NXR; r++) load_x4<XBF16>(p.x, base + (uint32_t)E::xrun0(r), s.v[r]);
}

// The rest of staging thread (t, s.item): picks each scale group's power of
// two s = 2^(e-14) from the group's largest magnitude over the chunk (frexp
// exponent e, so |x|/s < 2^14), writes the dword's PPT f16 pairs in decode
// order (one RNE rounding of x/s, or of x/(16s) for pairs meeting x16 codes)
// and, from lane t = 0, the group constants -C = -Σ coef·v and s·Σx over the
// stored values v (their f32 sums reduced across the chunk's NT lanes).
template <class E, int B>
__device__ __forceinline__ void xstage_store(uint8_t* lds, uint32_t nch, uint32_t t, const XStage<E>& s) {
    using XT = XTile<E>;
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    uint32_t* xp = reinterpret_cast<uint32_t*>(lds);
    float* xc = reinterpret_cast<float*>(lds + (size_t)B * nch * XT::XPW * 4u);
    auto val = [&](int h, int e) -> float {
        const int r = xrun_of<E>(h, e);
        return s.v[r][E::xoff(0, h, e) - E::xrun0(r)];
    };
    // each group's largest magnitude: its 2·PPT/NG activations folded three at
    // a time (the running maximum is non-negative, so its abs is a no-op)
    constexpr int NV = 2 * E::PPT / E::NG;
    static_assert(NV >= 3, "a group holds at least 3 activations per dword");
    uint32_t mx[E::NG];
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        float a[NV];
        int n = 0;
#pragma unroll
        for (int h = 0; h < E::PPT; h++)
            if (E::grp(0, h) == g) {
                a[n++] = val(h, 0);
                a[n++] = val(h, 1);
            }
        float m = absmax3(a[0], a[1], a[2]);
#pragma unroll
        for (int i = 3; i < NV; i += 2) m = absmax3(m, a[i], a[i + 1 < NV ? i + 1 : i]);
        mx[g] = __float_as_uint(m);  // non-negative floats order as integers
    }
    int ex[E::NG];
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        mx[g] = lanes_reduce<E::NT>(mx[g], [](uint32_t a, uint32_t b) { return a > b ? a : b; });
        int e = 0;
        (void)frexpf(__uint_as_float(mx[g]), &e);
        ex[g] = e < -110 ? -110 : e;  // keeps s = 2^(e-14) a normal f32
    }
    uint32_t pr[E::PPT];
    float C[E::NG], S[E::NG];
#pragma unroll
    for (int g = 0; g < E::NG; g++) C[g] = S[g] = 0.0f;
#pragma unroll
    for (int h = 0; h < E::PPT; h++) {
        const int g = E::grp(0, h);
        const bool dv = E::dv(0, h);
        const int sh = (dv ? 10 : 14) - ex[g];
        const f32x2 f = {ldexpf(val(h, 0), sh), ldexpf(val(h, 1), sh)};
        pr[h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));  // v_cvt_pk_f16_f32 (RNE)
        const uint32_t cf = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)E::coef(dv)) * 0x00010001u;
        C[g] = dot2(pr[h], cf, C[g]);
        if constexpr (XT::NCF == 4) S[g] = dot2(pr[h], dv ? 0x4C004C00u : 0x3C003C00u, S[g]);  // (16, 16) or (1, 1)
    }
    auto fadd = [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); };
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        C[g] = __uint_as_float(lanes_reduce<E::NT>(__float_as_uint(C[g]), fadd));
        if constexpr (XT::NCF == 4) S[g] = __uint_as_float(lanes_reduce<E::NT>(__float_as_uint(S[g]), fadd));
    }
    if (s.live) {
        uint32_t* dst = xp + (size_t)s.item * XT::XPW + t * (uint32_t)E::PPT;
        if constexpr (E::PPT % 4 == 0) {
#pragma unroll
            for (int h = 0; h < E::PPT; h += 4)
                *reinterpret_cast<uint4*>(dst + h) = make_uint4(pr[h], pr[h + 1], pr[h + 2], pr[h + 3]);
        } else {
            static_assert(E::PPT == 2, "pairs per code dword: 2, 4 or 8");
            *reinterpret_cast<uint2*>(dst) = make_uint2(pr[0], pr[1]);
        }
        if (t == 0) {
#pragma unroll
            for (int g = 0; g < E::NG; g++) {
                const float sc = ldexpf(1.0f, ex[g] - 14);
                float* c = xc + ((size_t)s.item * E::NG + g) * XT::NCF;
                if constexpr (XT::NCF == 4) {
                    *reinterpret_cast<float4*>(c) = make_float4(-C[g], sc, sc * S[g], 0.0f);
                } else {
                    *reinterpret_cast<float2*>(c) = make_float2(-C[g], sc);
                }
            }
        }
    }
}

// Stages activation rows [0, batch) into the tile (rows up to B restage row 0),
// one thread per code dword: B·nch·NT staging threads, P per workgroup thread
// per round.  The first round's activation loads are issued, then mid() (the
// caller's first weight loads), then the first round is computed: loads
// return in issue order, so the activations arrive ahead of the weights and
// the staging arithmetic runs while the weights are in flight.  Later rounds
// (large batches) load after the weights.  Ends with a barrier.
template <class E, int B, bool XBF16, int P, int TH, class MID>
__device__ __forceinline__ void stage_x_rounds(uint8_t* lds, const GemvParams& p, MID&& mid) {
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const uint32_t total = (uint32_t)B * nch * (uint32_t)E::NT;
    const uint32_t t = threadIdx.x % (uint32_t)E::NT;  // the workgroup size is a multiple of NT
    XStage<E> s[P];
#pragma unroll
    for (int ps = 0; ps < P; ps++) xstage_load<E, B, XBF16>(p, nch, threadIdx.x + (uint32_t)ps * TH, s[ps]);
    __builtin_amdgcn_sched_barrier(0);
    mid();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ps = 0; ps < P; ps++) xstage_store<E, B>(lds, nch, t, s[ps]);
    for (uint32_t base = (uint32_t)P * TH; base < total; base += (uint32_t)P * TH) {
#pragma unroll
        for (int ps = 0; ps < P; ps++)
            xstage_load<E, B, XBF16>(p, nch, base + threadIdx.x + (uint32_t)ps * TH, s[ps]);
#pragma unroll
        for (int ps = 0; ps < P; ps++) xstage_store<E, B>(lds, nch, t, s[ps]);
    }
    __syncthreads();
}

// Rounds of P passes, P the power of two covering the staging threads, at
// most 32 activations (registers) per thread in flight: every variant is
// compiled into the kernel, so the widest one sets its register count.  TH is
// the workgroup size.  (16 activations, so two rounds of loads at 4 rows of
// 4096: per step, Qwen3-8B Q4_K_M at 4 rows 2.48 against 2.41 ms, GGUF 2.17
// against 2.16 ms.)
template <class E, int B, bool XBF16, int TH, class MID>
__device__ __forceinline__ void stage_x_dwords(uint8_t* lds, const GemvParams& p, MID&& mid) {
    constexpr int PMAX = 8 / E::NXR > 0 ? 8 / E::NXR : 1;
    const uint32_t passes = ((uint32_t)B * (p.K / (uint32_t)E::CW) * (uint32_t)E::NT + TH - 1u) / TH;
    if (PMAX == 1 || passes <= 1u) stage_x_rounds<E, B, XBF16, 1, TH>(lds, p, mid);
    else if constexpr (PMAX >= 2) {
        if (PMAX == 2 || passes <= 2u) stage_x_rounds<E, B, XBF16, 2, TH>(lds, p, mid);
        else stage_x_rounds<E, B, XBF16, (PMAX >= 4 ? 4 : 2), TH>(lds, p, mid);
    }
}


// Activation staging mode of a GEMV kernel, a template parameter chosen per
// launch (xmode()): the source dtype and the staging threads per scale
// group.  One staging variant per kernel keeps each kernel's code small: these
// launches are short, and each starts by fetching its code (a kernel holding
// both variants, picked at run time, ran the Qwen3-0.6B GGUF step 410 us
// against 393 us).
enum XMode : int {
    XM_F32 = 0,        // f32 rows, one thread per group
    XM_BF16 = 1,       // bf16 rows, one thread per group
    XM_F32_SPLIT = 2,  // f32 rows, two threads per 32-activation group
};

// Two threads per group for f32 rows with 32-activation groups when the
// staged rows hold 64..128 groups: a thread then issues four 16-byte loads
// instead of eight, and more of the workgroup's waves share the staging.
// Below 64 groups a single wave stages either way, and the cross-lane step
// of a split costs more than the loads it saves.  Measured per step (one
// MI355X, graph replay): the Qwen3-8B GGUF step 1.30 -> 1.27-1.29 ms with the
// split at K = 4096 (128 groups); the Qwen3-0.6B projections (K = 1024, 32
// groups) 393 us unsplit against 405 us split; bf16 rows gain nothing.
// Several f32 activation rows (B > 1) stage one thread per code dword
// (stage_x_dwords); bf16 rows, half the bytes per group, stage one thread per
// group at every batch (the Qwen3-0.6B MLX step at 4 rows: 617 us against
// 633 us).
template <class E>
inline int xmode(bool x_bf16, uint32_t B, uint32_t K) {
    if (x_bf16) return XM_BF16;
    const uint32_t groups = B * (K / (uint32_t)E::CW) * (uint32_t)E::NG;
    return B == 1 && E::RUNLEN == 32 && groups >= 64u && groups <= 128u ? XM_F32_SPLIT : XM_F32;
}
// The mode of a B-row kernel: the split names no other kernel than f32 at B > 1.
constexpr int xmode_rows(int xm, int B) { return B > 1 && xm == XM_F32_SPLIT ? XM_F32 : xm; }

template <class E, int B, int XM, int TH = kGemvThreads, class MID>
__device__ __forceinline__ void stage_x_auto(uint8_t* lds, const GemvParams& p, MID&& mid) {
    if constexpr (B > 1 && XM != XM_BF16) {
        stage_x_dwords<E, B, false, TH>(lds, p, mid);
    } else {
        static_assert(group_runs_ok<E>(), "scale groups disagree with xoff()");
        constexpr int SP = XM == XM_F32_SPLIT && B == 1 ? 2 : 1;
        static_assert(E::NT % SP == 0 && (SP == 1 || E::RUNLEN == 32), "a group's code dwords split evenly");
        stage_x_sp<E, SP, B, XM == XM_BF16, TH>(lds, p, mid);
    }
}

// Staging for the streaming kernel (long launches whose waves all wait at
// the staging barrier): the widest split (4, 2 or 1 threads per group,
// dividing NT) whose threads fit one round of the workgroup, so that each
// thread's share, and the barrier's wait, is shortest.  Measured on the
// Qwen3-8B Q4_K_M gate/up (Q4_K 2 x 12288 x 4096): 13.4-13.5 us per launch at
// four threads per group against 13.9 us at two and 14.4-14.8 us at one.
template <class E, bool XBF16, int TH, class MID>
__device__ __forceinline__ void stage_x_fit(uint8_t* lds, const GemvParams& p, MID&& mid) {
    static_assert(group_runs_ok<E>(), "scale groups disagree with xoff()");
    const uint32_t groups = (p.K / (uint32_t)E::CW) * (uint32_t)E::NG;
    if constexpr (E::NT % 4 == 0 && TH <= 512) {
        if (4u * groups <= (uint32_t)TH) return stage_x_sp<E, 4, 1, XBF16, TH>(lds, p, mid);
    }
    if constexpr (E::NT % 2 == 0) {
        if (2u * groups <= (uint32_t)TH) return stage_x_sp<E, 2, 1, XBF16, TH>(lds, p, mid);
    }
    stage_x_sp<E, 1, 1, XBF16, TH>(lds, p, mid);
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
// task of compute.  stage(mid) stages the activations (with a barrier) in
// every wave and calls mid(), which issues the first task's loads, between
// issuing the activation loads and using them.
// The kernel arguments the GEMV set-up reads, made operands of empty asm
// statements at the kernel's top: the compiler then loads them together, two
// rounds of scalar loads, instead of each where it is first needed behind a
// wait for the one before (five rounds before the first activation load).
// Per launch, Qwen3-8B at one row: down_proj (persistent pipeline) 11.7 ->
// 11.5 us; at four rows q/k/v 10.7 -> 10.5, o 7.9 -> 7.6, down 17.9 -> 17.6.
// The latency-mode kernels, whose set-up is shorter, do not take it (q/k/v at
// one row 5.18 -> 5.27 us, the Qwen3-0.6B step 384 -> 396 us with it).
__device__ __forceinline__ void gemv_args_up_front(const GemvParams& p) {
    asm volatile("" ::"s"(p.w[0]), "s"(p.w[1]), "s"(p.w[2]), "s"(p.w[3]), "s"(p.y[0]), "s"(p.y[1]), "s"(p.y[2]),
                 "s"(p.y[3]), "s"(p.x));
    asm volatile("" ::"s"(p.n[0]), "s"(p.n[1]), "s"(p.n[2]), "s"(p.n[3]), "s"(p.wave_end[0]), "s"(p.wave_end[1]),
                 "s"(p.wave_end[2]), "s"(p.wave_end[3]), "s"(p.K), "s"(p.lanes_log2), "s"(p.nprob), "s"(p.batch),
                 "s"(p.res_steps), "s"(p.total_rb), "s"(p.y_bf16));
}

template <class E, int R, int B, int TH, class LOAD, class STAGE>
__device__ __forceinline__ void gemv_pipeline(const GemvParams& p, const uint8_t* lds, LOAD&& load, STAGE&& stage) {
    gemv_args_up_front(p);
    const uint32_t lane = threadIdx.x & 63u;
    // The launch shape comes from compile-time constants (TH: the workgroup
    // size) and the parameters: reading blockDim/gridDim costs a load from the
    // dispatch packet that the first weight loads would wait behind.
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)(TH / 64) + (threadIdx.x >> 6));
    const uint32_t L = 1u << p.lanes_log2;
    const uint32_t j = lane & (L - 1u), g = lane >> p.lanes_log2;
    const uint32_t rows_per_rb = (64u >> p.lanes_log2) * (uint32_t)R;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const uint32_t cpl = (nch + L - 1u) >> p.lanes_log2;  // chunks per lane per row block
    // This wave's problem (fixed for the launch: the host gives each problem a
    // range of waves in proportion to its row blocks) and its row blocks wi,
    // wi + nw, ... of that problem: the problem's waves read neighbouring row
    // blocks at a time, a compact front through the matrix (DRAM locality).
    uint32_t pi = 0;
#pragma unroll
    for (int i = 0; i + 1 < kMaxProblems; i++) pi += ((uint32_t)i + 1u < p.nprob && wid >= p.wave_end[i]) ? 1u : 0u;
    RowBlock blk0;
    blk0.w = pick(pi, p.w);
    blk0.sc = pick(pi, p.sc);
    blk0.bi = pick(pi, p.bi);
    blk0.y = pick(pi, p.y);
    blk0.n = pick(pi, p.n);
    const uint32_t wbeg = pi == 0 ? 0u : pick(pi - 1u, p.wave_end), wend = pick(pi, p.wave_end);
    const uint32_t prb = (blk0.n + rows_per_rb - 1u) / rows_per_rb;  // the problem's row blocks
    const uint32_t wi = wid - wbeg, nw = wend - wbeg;
    const uint32_t T = wi < prb ? (prb - wi + nw - 1u) / nw * cpl : 0u;  // tasks of this wave

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
    // the task loaded next: row block nrb (a wave without row blocks loads
    // rows clamped into the matrix), chunk round nc
    uint32_t nrb = wi, nc = 0;
    RowBlock nblk = blk0;
    nblk.base = nrb * rows_per_rb;
    // wave-uniform and branch-free; past the end the last task is loaded again
    auto advance = [&](uint32_t t) {
        const bool more = t + 1 < T;
        const bool wrap = more && nc + 1 == cpl;
        nc = wrap ? 0u : (more ? nc + 1 : nc);
        nrb = wrap ? nrb + nw : nrb;
        nblk.base = nrb * rows_per_rb;
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
    stage([&] { load_task(ba, nblk, nc); });
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
// lane issues the loads of all CPL of its chunks right after the activation
// loads, the activations are staged while they are in flight, so the whole
// launch waits on one memory latency; then it multiplies them for the B
// activation rows, the L lanes reduce, and lane 0 stores.  TH is the
// workgroup size.
template <class E, int CPL, int B, int TH, class LOAD, class STAGE>
__device__ __forceinline__ void gemv_oneshot(const GemvParams& p, const uint8_t* lds, LOAD&& load, STAGE&& stage) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)(TH / 64) + (threadIdx.x >> 6));
    const uint32_t L = 1u << p.lanes_log2;
    const uint32_t j = lane & (L - 1u), g = lane >> p.lanes_log2;
    const uint32_t rows_per_rb = 64u >> p.lanes_log2;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const bool active = wid < p.total_rb;
    const RowBlock blk = row_block(p, active ? wid : p.total_rb - 1u, rows_per_rb);
    const uint32_t row = blk.base + g < blk.n ? blk.base + g : blk.n - 1u;
    typename E::Raw buf[CPL];
    stage([&] {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const uint32_t u = j + (uint32_t)c * L;
            buf[c] = load(blk, row, u < nch ? u : nch - 1u);
        }
    });
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
template <class E, int B, int R, int XM, int TH = kGemvThreads>
__global__ __launch_bounds__(TH) void gguf_gemv_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    const uint32_t rowbytes = (p.K / (uint32_t)E::QK) * (uint32_t)E::BB;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) { return E::load(rb.w, row * rowbytes, u); };
    gemv_pipeline<E, R, B, TH>(p, xlds, load, [&](auto&& mid) { stage_x_auto<E, B, XM, TH>(xlds, p, mid); });
}

template <class E, int CPL, int B, int XM, int TH>
__global__ __launch_bounds__(TH) void gguf_gemv_oneshot_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    const uint32_t rowbytes = (p.K / (uint32_t)E::QK) * (uint32_t)E::BB;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) { return E::load(rb.w, row * rowbytes, u); };
    gemv_oneshot<E, CPL, B, TH>(p, xlds, load, [&](auto&& mid) { stage_x_auto<E, B, XM, TH>(xlds, p, mid); });
}

// ---------------------------------------------------------------- MLX affine U4
// Raw bytes of chunk u of a row: 16 bytes of packed words plus the group's
// scale and bias (f32, or f16/bf16 bits).
struct MlxLoad {
    const GemvParams& p;
    uint32_t ngroups;
    bool f32s;
    __device__ __forceinline__ explicit MlxLoad(const GemvParams& q)
        : p(q), ngroups(q.K / q.group), f32s(q.sdtype == DT_F32) {}
    __device__ __forceinline__ EncMlxU4::Raw operator()(const RowBlock& rb, uint32_t row, uint32_t u) const {
        EncMlxU4::Raw r;
        const uint8_t* wb = rb.w;
        load_dwords<4>(reinterpret_cast<const uint32_t*>(wb + (row * (p.K / 2u) + u * 16u)), r.w);
        const uint32_t gi = row * ngroups + div_magic(32u * u, p.gmagic);  // chunk u: k = 32u .. 32u + 31
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

template <int B, int R, int XM, int TH = kGemvThreads>
__global__ __launch_bounds__(TH) void mlx_u4_gemv_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    gemv_pipeline<EncMlxU4, R, B, TH>(p, xlds, MlxLoad(p),
                                      [&](auto&& mid) { stage_x_auto<EncMlxU4, B, XM, TH>(xlds, p, mid); });
}

template <int CPL, int B, int XM, int TH>
__global__ __launch_bounds__(TH) void mlx_u4_gemv_oneshot_kernel(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t xlds[];
    gemv_oneshot<EncMlxU4, CPL, B, TH>(p, xlds, MlxLoad(p),
                                        [&](auto&& mid) { stage_x_auto<EncMlxU4, B, XM, TH>(xlds, p, mid); });
}

// Widest rows per lane group instantiated for a register batch B: more rows
// amortise each activation read from LDS and the per-task overhead, fewer
// keep the accumulators in registers (gemv_tiles adds the narrower tiles).
template <class E, int B>
constexpr int rows_per_group() {
    if constexpr (wide_chunks(E::ENC)) return B <= 2 ? 2 : 1;  // 64-weight chunks
    else return B <= 2 ? 4 : 2;
}

// Resident workgroups per CU for (kernel, dynamic LDS) on the current device
// and its CU count, cached after the first query (host side, thread-safe).
// Also raises the kernel's dynamic-LDS limit when lds needs it.
hipError_t cached_occupancy(const void* kernel, size_t lds, int threads, int* per_cu, int* cus);

// Row blocks of rows_per_rb rows over the problems (rb_begin, total_rb).
inline void layout_row_blocks(GemvParams& p, uint32_t rows_per_rb) {
    uint32_t rbs = 0;
    for (int i = 0; i < kMaxProblems; i++) {
        p.rb_begin[i] = rbs;
        if ((uint32_t)i < p.nprob) rbs += (p.n[i] + rows_per_rb - 1) / rows_per_rb;
    }
    p.total_rb = rbs;
}

// Waves of the persistent grid per problem (p.wave_end), in proportion to
// each problem's row blocks, at least one each: problem i < nprob-1 gets
// 1 + floor((W - nprob)·rb_i / rb_total) waves and the last the rest (at
// least one, since the others take at most W - 1 together).
inline void split_waves(GemvParams& p, uint32_t rows_per_rb, uint32_t threads) {
    const uint64_t W = (uint64_t)p.grid * (threads / 64);
    uint64_t rb[kMaxProblems] = {}, total = 0;
    for (uint32_t i = 0; i < p.nprob; i++) total += rb[i] = (p.n[i] + rows_per_rb - 1) / rows_per_rb;
    uint64_t end = 0;
    for (uint32_t i = 0; i < (uint32_t)kMaxProblems; i++) {
        if (i + 1 < p.nprob) end += 1 + (W - p.nprob) * rb[i] / (total ? total : 1);
        else end = W;
        p.wave_end[i] = (uint32_t)end;
    }
}

typedef void (*GemvKernel)(GemvParams);
constexpr int kGemvMaxTiles = 6;

// One persistent-pipeline instantiation: rows per lane group and its kernel.
struct GemvTile {
    uint32_t R;
    GemvKernel kernel;
    uint32_t threads;  // workgroup size
};

// Persistent launch over the instantiated tiles t[0..n) (widest first).  Each
// tile's grid is as many workgroups as fit on the device at once (its
// occupancy x CUs), capped by its row-block count, and its waves are split
// over the problems (split_waves).  Long streams (the busiest wave has at
// least 8 tasks; cpl = chunks per lane per row block): the widest tile whose
// busiest CU holds within 5% of an even split of all rows over the CUs (its
// busiest wave's rows times its waves), since wider tiles amortise the
// per-task and per-row-block work over more weights.  Otherwise, or when no
// tile splits that evenly, the tile whose busiest wave has the fewest rows
// (rows, not row blocks: a wave's time is its share of the weight stream),
// ties to the widest; for short streams this also keeps more waves, and
// loads, in flight.  Measured: the 8B lm_head (Q6_K 151936x4096) 109 us on
// 1-row tiles (6 waves per SIMD, the fewest rows per wave) against 99 us on
// 2-row tiles (4 per SIMD, 2% over the even split); the 8B down (Q6_K
// 4096x12288, 3 tasks per wave) 13.1 us on 1-row tiles against 13.8 us on
// 2-row tiles (both split evenly, 16 and 8 waves per CU); the 8B gate/up (two
// 12288-row problems) on 4-row tiles left half the waves 2 row blocks and
// half 1 (49% of HBM peak), 1- and 2-row tiles split them evenly (54%).
// Between tiles of equal rows per wave, the one whose busiest CU holds fewer
// rows (a grid below the CU count in 512-thread workgroups leaves CUs idle
// that 256-thread workgroups fill), ties to the first listed.  The even-split
// rule takes the first-listed workgroup size only: at one workgroup per CU
// (the 8B Q6_K down_proj at 4 rows, 96 KiB of activations) 256 threads split
// evenly with half the waves, 23.3 us per launch against 17.9.
inline hipError_t launch_persistent_best(const GemvTile* t, int n, const GemvParams& p0, size_t lds,
                                         uint32_t cpl, hipStream_t st) {
    const uint32_t groups = 64u >> p0.lanes_log2;  // lane groups per wave
    uint64_t total_rows = 0;
    for (uint32_t k = 0; k < p0.nprob; k++) total_rows += p0.n[k];
    int pick = -1, even = -1;
    uint64_t best = ~(uint64_t)0, best_load = ~(uint64_t)0;
    GemvParams q = p0, chosen = p0, chosen_even = p0;
    for (int i = 0; i < n; i++) {
        q = p0;
        const uint32_t rows_per_rb = groups * t[i].R;
        const uint64_t waves = t[i].threads / 64;
        layout_row_blocks(q, rows_per_rb);
        int cus = 0, per_cu = 0;
        hipError_t e = cached_occupancy(reinterpret_cast<const void*>(t[i].kernel), lds, (int)t[i].threads, &per_cu, &cus);
        if (e != hipSuccess) return e;
        if (per_cu < 1 || cus < 1) continue;
        const uint64_t cap = (uint64_t)per_cu * (uint64_t)cus;
        const uint64_t want = ((uint64_t)q.total_rb + waves - 1) / waves;
        q.grid = (uint32_t)(want < cap ? want : cap);
        split_waves(q, rows_per_rb, t[i].threads);
        uint64_t rbs = 0;  // row blocks of the busiest wave
        for (uint32_t k = 0; k < q.nprob; k++) {
            const uint64_t nw = q.wave_end[k] - (k ? q.wave_end[k - 1] : 0u);
            const uint64_t prb = (q.n[k] + rows_per_rb - 1) / rows_per_rb;
            const uint64_t r = (prb + nw - 1) / nw;
            rbs = r > rbs ? r : rbs;
        }
        const uint64_t rows = rbs * rows_per_rb;
        const uint64_t load = rows * waves * (((uint64_t)q.grid + (uint64_t)cus - 1) / (uint64_t)cus);
        if (even < 0 && t[i].threads == t[0].threads && rbs * cpl >= 8 &&
            load * 100 <= total_rows * 105 / (uint64_t)cus) {
            even = i;
            chosen_even = q;
        }
        if (rows < best || (rows == best && load < best_load)) {
            best = rows;
            best_load = load;
            pick = i;
            chosen = q;
        }
    }
    if (even >= 0) {
        pick = even;
        chosen = chosen_even;
    }
    if (pick < 0) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(t[pick].kernel, dim3(chosen.grid), dim3(t[pick].threads), lds, st, chosen);
    return hipGetLastError();
}

// The persistent tiles instantiated for register batch B: the default rows per
// group W, half of it, and for one activation row every power of two down
// to one row.  gemv_tile<R>() names the kernel of R rows, of `threads`
// threads per workgroup.  2-8 activation rows list them twice, in 512- and
// 256-thread workgroups (kGemvMaxTiles entries at most).
template <class E, int B, class MK>
int gemv_tiles(GemvTile* t, MK&& gemv_tile, uint32_t threads = kGemvThreads) {
    constexpr int W = rows_per_group<E, B>();
    int n = 0;
    t[n++] = {(uint32_t)W, gemv_tile(std::integral_constant<int, W>()), threads};
    if constexpr (W >= 2) t[n++] = {(uint32_t)(W / 2), gemv_tile(std::integral_constant<int, W / 2>()), threads};
    if constexpr (W >= 4 && B == 1) t[n++] = {(uint32_t)(W / 4), gemv_tile(std::integral_constant<int, W / 4>()), threads};
    return n;
}

// Latency-mode launch: one wave per row block of one row per lane group, in
// workgroups of 512 threads (k512) or 256 (k256): the size whose busiest CU
// holds fewer waves, ties to 512 (each workgroup stages the activations once).
// Every workgroup lands on a CU of its own while the grid is at most the CU
// count, so 1,024 waves fill all 256 CUs in 256-thread groups and half of
// them in 512-thread groups; measured on the Qwen3-0.6B projections (1,024
// and 3,072 waves) 256 threads took 5-15% less time per launch, and on
// launches that split evenly either way (2,048, 4,096, 6,144 waves) it cost
// up to 12%.  A null k512 (a kernel built for 256 threads only) always
// launches k256.
template <class KERNEL>
hipError_t launch_oneshot(KERNEL k512, KERNEL k256, GemvParams p, size_t lds, hipStream_t st) {
    int cus = 0, per_cu = 0;
    hipError_t e = k512 ? cached_occupancy(reinterpret_cast<const void*>(k512), lds, 512, &per_cu, &cus) : hipSuccess;
    if (e != hipSuccess) return e;
    e = cached_occupancy(reinterpret_cast<const void*>(k256), lds, 256, &per_cu, &cus);
    if (e != hipSuccess) return e;
    if (cus < 1) return hipErrorInvalidConfiguration;
    layout_row_blocks(p, 64u >> p.lanes_log2);
    auto busiest = [&](uint32_t waves) {  // waves on the busiest CU, groups of `waves`
        const uint64_t wgs = ((uint64_t)p.total_rb + waves - 1) / waves;
        return (wgs + (uint64_t)cus - 1) / (uint64_t)cus * waves;
    };
    const bool small = !k512 || busiest(4) < busiest(8);
    const uint32_t waves = small ? 4u : 8u;
    p.grid = (p.total_rb + waves - 1) / waves;
    hipLaunchKernelGGL(small ? k256 : k512, dim3(p.grid), dim3(waves * 64u), lds, st, p);
    return hipGetLastError();
}

// Instantiates and launches the GEMV kernel of encoding E for a power-of-two
// register batch B (the host has checked that its activation tile fits LDS);
// oneshot = chunks per lane selects the latency-mode kernel, 0 the
// persistent pipeline.  The row-block layout is set here, per tile.
// Activations are f32 (the reference's precision contract for quantized
// linears, crates/dyninfer-compiler/src/lib.rs:289-306) or bf16, staged as XM says (XMode).
template <class E, int XM>
hipError_t launch_gguf_gemv_stream(GemvParams p, size_t lds, hipStream_t st);  // gemv_stream.hpp

template <class E, int XM>
hipError_t launch_gguf_gemv_x(const GemvParams& p, uint32_t B, uint32_t oneshot, hipStream_t st) {
    const size_t lds = (size_t)xtile_bytes(E::ENC, B, p.K);
    if (B == 1 && !oneshot) {  // long stream of one activation row: the streaming kernel where it fits
        // (the streaming kernel picks its staging split itself: two modes, not three)
        const hipError_t e = launch_gguf_gemv_stream<E, XM == XM_BF16 ? XM_BF16 : XM_F32>(p, lds, st);
        if (e != hipErrorNotSupported) return e;
    }
    if (oneshot) {
        // chunks per lane (the host's limits): 1..4 for one activation row
        // (64-weight chunks 1..2), 1..2 for 2 rows, 1 for 4
#define DMX_ONESHOT(b, c)                                                                             \
    if (B == b && oneshot == c)                                                                       \
        return launch_oneshot(gguf_gemv_oneshot_kernel<E, c, b, xmode_rows(XM, b), 512>,                         \
                              gguf_gemv_oneshot_kernel<E, c, b, xmode_rows(XM, b), 256>, \
                              p, lds, st);
        DMX_ONESHOT(1, 1)
        DMX_ONESHOT(1, 2)
        if constexpr (!wide_chunks(E::ENC)) {
            DMX_ONESHOT(1, 3)
            DMX_ONESHOT(1, 4)
        }
        if constexpr (max_register_batch(E::ENC) >= 2) {
            DMX_ONESHOT(2, 1)
            DMX_ONESHOT(2, 2)
        }
        if constexpr (max_register_batch(E::ENC) >= 4) DMX_ONESHOT(4, 1)
        if constexpr (max_register_batch(E::ENC) >= 8) {
            DMX_ONESHOT(8, 1)
            // 8 rows of 2 chunks per lane take ~300 registers: 256-thread workgroups only
            if (B == 8 && oneshot == 2)
                return launch_oneshot<GemvKernel>(nullptr, gguf_gemv_oneshot_kernel<E, 2, 8, xmode_rows(XM, 8), 256>,
                                                  p, lds, st);
        }
#undef DMX_ONESHOT
        return hipErrorInvalidValue;
    }
    GemvTile t[kGemvMaxTiles];
    int n = 0;
    // One activation row and K > 8192: 1024-thread workgroups, one per CU,
    // stage the activations half as often per CU, in one round of loads.
    // Staging is VALU work per workgroup (~7.5 instructions per activation
    // for Q6_K) and a launch's waves all stage before their first product: on
    // the 8B down_proj (Q6_K 4096x12288, 3 tasks per wave) it ended ~8,000
    // cycles in (two rounds of 512 threads, the second queued behind the
    // first task's weights), and 1024 threads took 12.1-12.4 us against
    // 13.0-13.5 us.  At K = 4096 1024 threads measured 1-2% slower.
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const bool big = B == 1 && p.K > 8192u;
#define DMX_CASE(b)                                                                                            \
    case b:                                                                                                    \
        if constexpr (b <= max_register_batch(E::ENC)) {                                                       \
            n = gemv_tiles<E, b>(t, [](auto r) -> GemvKernel { return gguf_gemv_kernel<E, b, decltype(r)::value, xmode_rows(XM, b)>; }); \
            n += gemv_tiles<E, b>(t + n, [](auto r) -> GemvKernel { return gguf_gemv_kernel<E, b, decltype(r)::value, xmode_rows(XM, b), 256>; }, 256u); \
        }                                                                                                      \
        break;
    switch (B) {
    case 1:
        n = big ? gemv_tiles<E, 1>(t, [](auto r) -> GemvKernel { return gguf_gemv_kernel<E, 1, decltype(r)::value, XM, 1024>; }, 1024u)
                : gemv_tiles<E, 1>(t, [](auto r) -> GemvKernel { return gguf_gemv_kernel<E, 1, decltype(r)::value, XM>; });
        break;
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
    default: break;
    }
#undef DMX_CASE
    if (n == 0) return hipErrorInvalidValue;
    return launch_persistent_best(t, n, p, lds, (nch + (1u << p.lanes_log2) - 1u) >> p.lanes_log2, st);
}



}  // namespace dmx
