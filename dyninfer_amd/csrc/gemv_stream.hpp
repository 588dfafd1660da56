// Batch-1 streaming GEMV for long weight streams (GGUF Q4_0/Q4_1/Q8_0/Q6_K/Q4_K/Q5_K/IQ4_XS).
//
// Same arithmetic as the persistent pipeline in gemv_kernels.hpp (activations
// staged in LDS as scaled f16 pairs, codes decoded by the exponent trick into
// v_dot2_f32_f16), with the per-task work cut to the decode and the dot
// products:
//   * a wave's G = 64/L lane groups own G consecutive weight rows at a time
//     (a "row step"); lane j of a group holds chunks j, j+L, ..., j+(CPL-1)L
//     of its row, so CPL = chunks/L is a compile-time constant and the row's
//     sum is reduced over the group once, after its CPL chunks;
//   * every load address is a per-lane constant (fixed for the launch: the
//     lane's row within the step and chunk within the round) plus a
//     wave-uniform base (row step, chunk round), so a load costs no vector
//     arithmetic: scalar base register, lane offset register;
//   * the realignment of 2-byte-aligned blocks is a per-lane constant too
//     (every scalar step is a multiple of 4 bytes);
//   * D chunk loads per lane are in flight in a ring of registers: after a
//     chunk's products the lane reloads its buffer with the chunk D tasks
//     ahead, so a lane keeps D - 1 chunks in flight while it computes;
//   * the last row step of a weight is moved back to end at its last row
//     (rows are computed twice there, stored twice with the same value), so
//     no lane ever needs a row clamp; a wave's task list is padded to a
//     whole number of unrolled rounds by repeating its last row step;
//   * a row's sum goes to a wave-private LDS slot, and the wave writes all
//     its rows to y after its stream, a few coalesced stores: a global store
//     inside the stream shares the load counter with the weight loads, and
//     waiting for a load behind it also waits for the store's
//     acknowledgment (measured on the Qwen3-8B gate/up: 12.5 us per launch
//     with a store per row, 11.5 us without).
// Waves are assigned to weights in proportion to their rows (split_waves) and
// walk row steps wi, wi + nw, ... of their weight (neighbouring waves on
// neighbouring rows).
#pragma once
#include <utility>

#include "gemv_kernels.hpp"

namespace dmx {

// Per-lane constants of a lane's chunk stream and the loads of one chunk:
// init() gets the byte shift of the weight base within its dword (bsh) and
// the byte offset of the lane's first chunk from the row step's base.
template <class E>
struct StreamLane {  // GGUF Q4_0 / Q8_0 (2-byte-aligned blocks) and Q4_1 (4-byte-aligned)
    uint32_t off, sh;
    __device__ __forceinline__ void init(uint32_t bsh, uint32_t lane_off) {
        const uint32_t o = bsh + lane_off;
        off = o & ~3u;
        sh = o & 3u;
    }
    __device__ __forceinline__ typename E::Raw load(const uint8_t* sb) const {
        typename E::Raw r;
        load_dwords<E::NDW>(reinterpret_cast<const uint32_t*>(sb + off), r.d);
        if constexpr (E::ENC != ENC_Q4_1) r.sh = sh;
        return r;
    }
};

template <>
struct StreamLane<EncQ6K> {  // lane offset = its super-block's; quarter (n, s) = lane bits 1, 0
    uint32_t off, sh, oa, oh;
    __device__ __forceinline__ void init(uint32_t bsh, uint32_t lane_off, uint32_t q) {
        const uint32_t o = bsh + lane_off;
        off = o & ~3u;
        sh = o & 3u;
        const uint32_t n = (q >> 1) & 1u, s = q & 1u;
        oa = 64u * n + 16u * s;
        oh = 128u + 32u * n + 16u * s;
    }
    __device__ __forceinline__ EncQ6K::Raw load(const uint8_t* sb) const {
        const uint8_t* al = sb + off;
        EncQ6K::Raw r;
        load_dwords<5>(reinterpret_cast<const uint32_t*>(al + oa), r.a);
        load_dwords<5>(reinterpret_cast<const uint32_t*>(al + oa + 32u), r.b);
        load_dwords<5>(reinterpret_cast<const uint32_t*>(al + oh), r.h);
        load_dwords<5>(reinterpret_cast<const uint32_t*>(al + 192u), r.s);  // sc[0..16) and d
        r.sh = sh;
        return r;
    }
};

template <>
struct StreamLane<EncQ4K> {  // lane offset = its super-block's; step i = lane bits 1, 0
    uint32_t off, oq;
    __device__ __forceinline__ void init(uint32_t bsh, uint32_t lane_off, uint32_t q) {
        off = bsh + lane_off;  // the base is 4-byte aligned (bsh = 0)
        oq = off + 16u + 32u * q;
    }
    __device__ __forceinline__ EncQ4K::Raw load(const uint8_t* sb) const {
        EncQ4K::Raw r;
        load_dwords<4>(reinterpret_cast<const uint32_t*>(sb + off), r.h);
        load_dwords<EncQ4K::NT>(reinterpret_cast<const uint32_t*>(sb + oq), r.q);
        return r;
    }
};

template <>
struct StreamLane<EncQ5K> {  // lane offset = its super-block's; step i = lane bits 1, 0
    uint32_t off, oq;
    __device__ __forceinline__ void init(uint32_t bsh, uint32_t lane_off, uint32_t q) {
        off = bsh + lane_off;  // the base is 4-byte aligned (bsh = 0)
        oq = off + 48u + 32u * q;
    }
    __device__ __forceinline__ EncQ5K::Raw load(const uint8_t* sb) const {
        EncQ5K::Raw r;
        load_dwords<4>(reinterpret_cast<const uint32_t*>(sb + off), r.h);
        load_dwords<EncQ5K::NT>(reinterpret_cast<const uint32_t*>(sb + off + 16u), r.hb);
        load_dwords<EncQ5K::NT>(reinterpret_cast<const uint32_t*>(sb + oq), r.q);
        return r;
    }
};

template <>
struct StreamLane<EncIQ4XS> {  // lane offset = its super-block's; sub-block ib = lane bits 2..0
    uint32_t off, oq;
    __device__ __forceinline__ void init(uint32_t bsh, uint32_t lane_off, uint32_t ib) {
        off = bsh + lane_off;  // the base is 4-byte aligned (bsh = 0)
        oq = off + 8u + 16u * ib;
    }
    __device__ __forceinline__ EncIQ4XS::Raw load(const uint8_t* sb) const {
        EncIQ4XS::Raw r;
        load_dwords<2>(reinterpret_cast<const uint32_t*>(sb + off), r.h);
        load_dwords<EncIQ4XS::NT>(reinterpret_cast<const uint32_t*>(sb + oq), r.q);
        return r;
    }
};

// f(integral_constant<int, i>) for i = 0..N-1, unrolled.
template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>()), ...);
}
template <int N, class F>
__device__ __forceinline__ void unroll(F&& f) {
    unroll_seq(f, std::make_integer_sequence<int, N>());
}

// y + the chunk's contribution, B = 1: xq = the chunk's f16 pairs in LDS,
// cq = its per-group constants (-C, s[, s·Σx]).
template <class E>
__device__ __forceinline__ float stream_chunk(const typename E::Chunk& c, const uint32_t* xq, const float* cq, float y) {
    float acc[E::NG], sc[E::NG], sm[E::NG];
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        float negc;
        load_consts<E>(cq, (uint32_t)g, negc, sc[g], sm[g]);
        acc[g] = negc;
    }
#pragma unroll
    for (int t = 0; t < E::NT; t++) {
        uint32_t pr[E::PPT], xv[E::PPT];
        E::pairs(c, t, pr);
        load_xpairs<E>(xq, 0u, t, xv);
#pragma unroll
        for (int h = 0; h < E::PPT; h++) {
            float& a = acc[E::grp(t, h)];
            a = dot2(pr[h], xv[h], a);
        }
    }
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        y = fmaf(E::gscale(c, g) * acc[g], sc[g], y);
        if constexpr (E::AFFINE) y = fmaf(E::goffset(c, g), sm[g], y);
    }
    return y;
}

// Ring depth D (chunk loads per lane in flight or being computed,
// independent of CPL: the loop is unrolled lcm(D, CPL) tasks so that ring
// slots and chunk rounds stay compile-time) and waves per CU.  The memory
// system streams this access pattern fastest with one to two tasks of loads
// in flight per wave at 16-24 waves per CU: more bytes in flight lower the
// read rate (a load-only probe over 56.6 MB block-strided streams: 9.9-10.4
// us per launch with one or two tasks per wave, 11 us with four, 12-14 us
// with eight).  Measured on the Qwen3-8B shapes (kernel time): gate/up Q4_0
// 12.2 us at D = 2 and 16 waves per CU (12.5-13.1 us at 12, 24, 32 waves or
// D = 1, 3); the Q6_K lm_head 88.5 us at D = 3 (96 us at D = 2).
template <class E>
constexpr int stream_depth() {
    return E::ENC == ENC_Q6_K ? 3 : 2;
}
constexpr uint32_t kStreamWaves = 16;
// The streaming instantiations that keep their ring and chunk state in
// registers: with 64-weight chunks the unrolled rounds of Q4_K, Q5_K and Q6_K
// spill at 1024 threads (128 registers per lane) for Q4_K at 3+ chunks per
// lane, Q5_K at 2+ and Q6_K at 2, 4, 6 and 8, and at 512 threads for Q4_K and
// Q5_K at 4+.  Those shapes run the persistent pipeline instead, which is
// faster than the spilling kernels by far (single row, per launch: Q4_K 16384
// x 12288 91.6 -> 24.7 us, x 16384 258 -> 31.8 us, Q5_K 16384 x 12288 130 ->
// 31.0 us, Q6_K 16384 x 16384 58.1 -> 46.4 us).
template <class E, int CPL, int TH>
constexpr bool stream_fits() {
    if constexpr (E::ENC == ENC_Q4_K) return TH == 1024 ? CPL <= 2 : CPL <= 3;
    if constexpr (E::ENC == ENC_Q5_K) return TH == 1024 ? CPL <= 1 : CPL <= 3;
    if constexpr (E::ENC == ENC_Q6_K) return TH == 1024 ? CPL == 1 || CPL == 3 : true;
    return true;
}
constexpr int stream_gcd(int a, int b) { return b ? stream_gcd(b, a % b) : a; }

template <class E, int CPL, int XM, int TH>
__global__ __launch_bounds__(TH) void gguf_gemv_stream_kernel(const GemvParams p) {
    constexpr int D = stream_depth<E>();
    constexpr int U = D / stream_gcd(D, CPL) * CPL;  // tasks per unrolled round: lcm(D, CPL)
    using XT = XTile<E>;
    extern __shared__ __align__(16) uint8_t xlds[];
    gemv_args_up_front(p);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)(TH / 64) + (threadIdx.x >> 6));
    const uint32_t lg = p.lanes_log2, L = 1u << lg, G = 64u >> lg;
    const uint32_t j = lane & (L - 1u), g = lane >> lg;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    const uint32_t rowbytes = (p.K / (uint32_t)E::QK) * (uint32_t)E::BB;
    // chunk round stride in bytes: L chunks of CW weights
    const uint32_t cstride = L * (uint32_t)E::CW / (uint32_t)E::QK * (uint32_t)E::BB;

    // this wave's weight (fixed for the launch) and its row steps wi, wi + nw, ...
    uint32_t pi = 0;
#pragma unroll
    for (int i = 0; i + 1 < kMaxProblems; i++) pi += ((uint32_t)i + 1u < p.nprob && wid >= p.wave_end[i]) ? 1u : 0u;
    const uint8_t* w = pick(pi, p.w);
    void* y = pick(pi, p.y);
    const uint32_t n = pick(pi, p.n);
    const uint32_t wbeg = pi == 0 ? 0u : pick(pi - 1u, p.wave_end), wend = pick(pi, p.wave_end);
    const uint32_t wi = wid - wbeg, nw = wend - wbeg;
    const uint32_t nrs = (n + G - 1u) / G;                            // row steps of the weight
    const uint32_t ks = wi < nrs ? (nrs - wi + nw - 1u) / nw : 0u;   // row steps of this wave
    const uint32_t T = ks * (uint32_t)CPL;  // tasks (row step k, chunk round c) = task k·CPL + c

    const uint32_t bsh = (uint32_t)((uintptr_t)w & 3u);
    const uint8_t* abase = w - bsh;  // 4-byte aligned
    StreamLane<E> sl;
    // lane j's chunk: block j / CPB, part j % CPB (CPB chunks per block; L is a
    // multiple of CPB, so every chunk round keeps the part)
    constexpr uint32_t CPB = (uint32_t)(E::QK / E::CW);
    if constexpr (CPB > 1) sl.init(bsh, g * rowbytes + (j / CPB) * (uint32_t)E::BB, j % CPB);
    else sl.init(bsh, g * rowbytes + j * (uint32_t)E::BB);
    // first row of row step k (the last step ends at the weight's last row)
    auto row0 = [&](uint32_t k) {
        const uint32_t kk = k < ks ? k : (ks ? ks - 1u : 0u);
        const uint32_t r = (wi + kk * nw) * G;
        return r + G <= n ? r : n - G;
    };
    auto sbase = [&](uint32_t t) { return abase + row0(t / (uint32_t)CPL) * rowbytes + (t % (uint32_t)CPL) * cstride; };
    const uint32_t* xq0 = reinterpret_cast<const uint32_t*>(xlds) + j * (uint32_t)XT::XPW;
    const float* cq0 = reinterpret_cast<const float*>(xlds + (size_t)nch * XT::XPW * 4u) + j * (uint32_t)(E::NG * XT::NCF);

    // this wave's row sums: res[k·G + g], after the activation tile
    const uint32_t xtb = (uint32_t)(((uint64_t)nch * XT::chunk_bytes + 15u) & ~(uint64_t)15u);
    float* res = reinterpret_cast<float*>(xlds + xtb) + (threadIdx.x >> 6) * p.res_steps * G;

    typename E::Raw buf[D];
    stage_x_fit<E, XM == XM_BF16, TH>(xlds, p, [&] {
#pragma unroll
        for (int d = 0; d < D; d++) buf[d] = sl.load(sbase((uint32_t)d));
    });
    if (ks == 0) return;
    auto store = [&](uint32_t row, float v) {
        if (p.y_bf16) gptr_mut<uint16_t>(y)[row] = f32_to_bf16_bits(v);
        else gptr_mut<float>(y)[row] = v;
    };
    float acc = 0.0f;
    // task t0 + u: its chunk is in ring slot u % D.  The slot is unpacked
    // into registers, refilled with task t0 + u + D (when `refill` is set;
    // past the end: the last row step again), and only then are the products
    // computed; the scheduling barrier keeps the refill there (the compiler
    // would otherwise hoist the next slot's unpack above it, waiting for
    // every load in flight).
    auto task = [&](uint32_t t0, auto uc, bool refill) {
        constexpr int u = decltype(uc)::value;
        constexpr int d = u % D;
        const uint32_t c = (uint32_t)(u % CPL);
        const typename E::Chunk ch = E::unpack(buf[d], j);
        if (refill) buf[d] = sl.load(sbase(t0 + (uint32_t)u + (uint32_t)D));
        __builtin_amdgcn_sched_barrier(0);
        acc = stream_chunk<E>(ch, xq0 + c * L * (uint32_t)XT::XPW, cq0 + c * L * (uint32_t)(E::NG * XT::NCF), acc);
        if (u % CPL == CPL - 1) {
            acc = group_sum(acc, L);
            const uint32_t k = (t0 + (uint32_t)u) / (uint32_t)CPL;
            if (j == 0) res[k * G + g] = acc;
            acc = 0.0f;
        }
    };
    // whole rounds of U tasks, branch-free (U is a multiple of CPL, so a
    // round starts a row step), then the last round, whole or partial, task
    // by task: it reloads only tasks that exist, so a wave's end does not wait
    // for D loads of its last row step again (per step, Qwen3-8B GGUF 1.295 ->
    // 1.284 ms, Q4_K_M 1.407 -> 1.390 ms)
    uint32_t t0 = 0;
    for (; t0 + (uint32_t)U < T; t0 += (uint32_t)U) unroll<U>([&](auto uc) { task(t0, uc, true); });
    if (t0 < T)
        unroll<U>([&](auto uc) {
            const uint32_t t = t0 + (uint32_t)decltype(uc)::value;
            if (t < T) task(t0, uc, t + (uint32_t)D < T);
        });
    // the wave's rows: lane l stores entries l, l + 64, ... (a row step's G rows are contiguous)
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    for (uint32_t i = lane; i < ks * G; i += 64u) store(row0(i / G) + i % G, res[i]);
}

// Launch: lanes per row L (a power of two, 8..64) and CPL = chunks / L from
// the instantiated set: the widest L with CPL >= 2, else the widest with
// CPL = 1; every weight needs at least G = 64/L rows.  Every scalar step
// (a row, a chunk round) must be a multiple of 4 bytes so that a lane's
// realignment is fixed: rows of an even number of blocks (Q4_0, Q8_0; Q6_K
// an even number of super-blocks) and, for the super-block encodings, L >= 8.  Returns
// hipErrorNotSupported when nothing fits or the instantiation would spill
// (stream_fits): the caller then runs the persistent pipeline.
template <class E, int XM>
hipError_t launch_gguf_gemv_stream(GemvParams p, size_t lds, hipStream_t st) {
    const uint32_t nch = p.K / (uint32_t)E::CW;
    if (((p.K / (uint32_t)E::QK) * (uint32_t)E::BB) % 4u) return hipErrorNotSupported;
    uint32_t nmin = ~0u;
    for (uint32_t i = 0; i < p.nprob; i++) nmin = p.n[i] < nmin ? p.n[i] : nmin;
    auto fits = [&](uint32_t l, uint32_t c) {
        return nch % (1u << l) == 0 && nch / (1u << l) == c && (64u >> l) <= nmin;
    };
    int cpl = 0;
    uint32_t lg = 0;
    for (uint32_t l = 6; l >= 3 && !cpl; l--)
        for (uint32_t c : {2u, 3u, 4u, 6u, 8u})
            if (fits(l, c)) {
                cpl = (int)c;
                lg = l;
            }
    for (uint32_t l = 6; l >= 3 && !cpl; l--)
        if (fits(l, 1u)) {
            cpl = 1;
            lg = l;
        }
    if (!cpl) return hipErrorNotSupported;
    p.lanes_log2 = lg;
    // one 1024-thread workgroup per CU stages long activation rows half as often
    const bool big = p.K > 8192u;
    const uint32_t threads = big ? 1024u : 512u;
    GemvKernel k = nullptr;
#define DMX_STREAM(c)                                                                                        \
    if constexpr (stream_fits<E, c, 1024>())                                                                 \
        if (cpl == c && big) k = gguf_gemv_stream_kernel<E, c, XM, 1024>;                                    \
    if constexpr (stream_fits<E, c, 512>())                                                                  \
        if (cpl == c && !big) k = gguf_gemv_stream_kernel<E, c, XM, 512>;
    DMX_STREAM(1)
    DMX_STREAM(2)
    DMX_STREAM(3)
    DMX_STREAM(4)
    DMX_STREAM(6)
    DMX_STREAM(8)
#undef DMX_STREAM
    if (!k) return hipErrorNotSupported;
    int cus = 0, per_cu = 0;
    hipError_t e = cached_occupancy(reinterpret_cast<const void*>(k), lds, (int)threads, &per_cu, &cus);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || cus < 1) return hipErrorNotSupported;
    const uint32_t G = 64u >> lg;
    layout_row_blocks(p, G);
    const uint64_t waves = threads / 64u;
    const uint32_t xtb = (uint32_t)(((uint64_t)lds + 15u) & ~(uint64_t)15u);
    uint64_t wgs_per_cu = kStreamWaves / waves;
    wgs_per_cu = wgs_per_cu < 1 ? 1 : (wgs_per_cu < (uint64_t)per_cu ? wgs_per_cu : (uint64_t)per_cu);
    const uint64_t cap = wgs_per_cu * (uint64_t)cus, want = ((uint64_t)p.total_rb + waves - 1) / waves;
    p.grid = (uint32_t)(want < cap ? want : cap);
    split_waves(p, G, threads);
    // LDS for the row sums of the busiest wave (within 32 KB per workgroup and
    // without costing occupancy, else the persistent pipeline runs).  Streams
    // of under three row steps per wave also run the persistent pipeline: a
    // wave that loads its only rows at once is the many-bytes-in-flight case
    // (the Qwen3-8B down_proj, one row per wave: 12.6 us here, 11.7 us there).
    uint32_t steps = 0, fewest = ~0u;
    for (uint32_t i = 0; i < p.nprob; i++) {
        const uint32_t nw = p.wave_end[i] - (i ? p.wave_end[i - 1] : 0u), nrs = (p.n[i] + G - 1u) / G;
        const uint32_t s = nw ? (nrs + nw - 1u) / nw : nrs;
        steps = s > steps ? s : steps;
        fewest = s < fewest ? s : fewest;
    }
    if (fewest < 3u) return hipErrorNotSupported;
    const uint64_t res = (uint64_t)steps * G * 4u * waves;
    if (res > 32768u) return hipErrorNotSupported;
    p.res_steps = steps;
    const size_t lds_all = xtb + (size_t)res;
    int per_cu2 = 0;
    e = cached_occupancy(reinterpret_cast<const void*>(k), lds_all, (int)threads, &per_cu2, &cus);  // raises the LDS limit
    if (e != hipSuccess) return e;
    if ((uint64_t)per_cu2 < wgs_per_cu) return hipErrorNotSupported;
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(threads), lds_all, st, p);
    return hipGetLastError();
}

template <class E>
hipError_t launch_gguf_gemv(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st) {
    switch (xmode<E>(xbf16, B, p.K)) {
    case XM_BF16: return launch_gguf_gemv_x<E, XM_BF16>(p, B, oneshot, st);
    case XM_F32_SPLIT:
        if constexpr (E::RUNLEN == 32) return launch_gguf_gemv_x<E, XM_F32_SPLIT>(p, B, oneshot, st);
        return hipErrorInvalidValue;
    default: return launch_gguf_gemv_x<E, XM_F32>(p, B, oneshot, st);
    }
}

}  // namespace dmx
