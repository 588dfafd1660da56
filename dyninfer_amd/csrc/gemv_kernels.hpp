// Decode GEMV kernel templates (activation rows 1..16) for GGUF Q4_0/Q4_1/Q8_0/
// Q6_K and MLX affine U4.
//
// Semantics: y[b, o] = Σ_k x[b, k] · w[o, k] with f32 accumulation, w the
// reference's dequantised weight (gguf_codegen.rs:268-314 `emit_linear`,
// mlx_affine.rs:557-626 `emit_linear_u4`).  IREE's reduction order is itself
// unspecified, so results agree within f32 reassociation, not bitwise.
//
// Mapping (wave64; the packed weights are streamed once from HBM):
//   * the weight rows are cut into row blocks of G·R rows (G = 64/L lane
//     groups per wave, R rows per group); L lanes of a group split the K range:
//     lane j takes chunks j, j+L, ... (cpl = chunks/L of them per row block);
//   * the grid is persistent (occupancy x CUs waves): wave w walks row blocks
//     w, w+W, ... and the lane's sequence of (row block, chunk) tasks runs as
//     one software pipeline — the next task's weight bytes are loaded before
//     the current task is computed, across row-block boundaries, so HBM
//     latency hides behind arithmetic instead of being paid per wave;
//   * GGUF blocks are only 2-byte aligned: each is loaded from the 4-byte-
//     aligned dword containing its start and realigned in registers;
//   * activations are staged once per workgroup in LDS as f32 (padded by 16
//     bytes per chunk so the L lanes of a group hit distinct banks), or read
//     through L1/L2 when B·K does not fit;
//   * per weight: one v_cvt_f32_ubyte and one fma per activation row; each
//     group's scale d and offset m are applied once as d·Σc·x + m·Σx
//     (encodings.hpp), and Σx is shared by the R rows;
//   * at the end of a row block the L lanes combine their R·B partial sums
//     with cross-lane shuffles and lane 0 of the group stores.
// Several weights that share one activation (q/k/v, gate/up) are served by one
// launch: row blocks are numbered across the problems.
#pragma once
#include "encodings.hpp"
#include "kernels.hpp"

namespace dmx {

// a[i] for a wave-uniform i.  The four values are pinned in scalar registers
// first: otherwise the optimiser folds the select chain back into a dynamic
// index of the kernel-argument array, which it can only serve from a private
// (scratch) copy of the array.
template <class T>
__device__ __forceinline__ T pick(uint32_t i, const T (&a)[kMaxProblems]) {
    static_assert(kMaxProblems == 4, "pick() assumes 4 problems");
    T v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
    asm("" : "+s"(v0), "+s"(v1), "+s"(v2), "+s"(v3));
    return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}

// Four consecutive activations of row r at element k, as f32.
template <bool XBF16>
__device__ __forceinline__ float4 load_x4(const void* __restrict__ x, uint32_t ldx, uint32_t r, uint32_t k) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    if constexpr (XBF16) {
        const uint16_t* xp = static_cast<const uint16_t*>(x) + (size_t)r * ldx + k;
        const u32x2 v = *gptr<u32x2>(xp);
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
    } else {
        const float* xp = static_cast<const float*>(x) + (size_t)r * ldx + k;
        const f32x4 v = *gptr<f32x4>(xp);
        return make_float4(v.x, v.y, v.z, v.w);
    }
}

// LDS activation layout: f32 [B][KP] with 4 padding floats after every chunk
// of CW, KP = K + 4·K/CW.
template <int CW>
__device__ __forceinline__ uint32_t lds_index(uint32_t k) { return k + 4u * (k / (uint32_t)CW); }

template <int CW>
__host__ __device__ constexpr size_t lds_bytes(uint32_t B, uint32_t K) {
    return (size_t)B * (K + 4u * (K / (uint32_t)CW)) * 4u;
}

template <int CW>
struct XLds {
    const float* xs;
    uint32_t KP;
    __device__ __forceinline__ float4 load(uint32_t b, uint32_t k) const {
        return *reinterpret_cast<const float4*>(xs + (size_t)b * KP + lds_index<CW>(k));
    }
};

// Activations read through L1/L2, for B·K too large for LDS.
template <bool XBF16>
struct XGlobal {
    const void* x;
    uint32_t ldx, batch;
    __device__ __forceinline__ float4 load(uint32_t b, uint32_t k) const {
        // rows beyond `batch` re-read row 0 (in bounds); their sums are never stored
        return load_x4<XBF16>(x, ldx, b < batch ? b : 0u, k);
    }
};

// Copies x[0..batch) (f32 or bf16, row stride ldx) into LDS as f32 in the
// padded layout, rows >= batch zero-filled.  All threads of the workgroup take
// part; ends with a barrier.
template <int CW, int B, bool XBF16>
__device__ __forceinline__ void stage_x(float* xs, const void* __restrict__ x, uint32_t K, uint32_t ldx,
                                        uint32_t batch) {
    const uint32_t kq = K / 4u, KP = K + 4u * (K / (uint32_t)CW);
    for (uint32_t i = threadIdx.x; i < (uint32_t)B * kq; i += blockDim.x) {
        const uint32_t b = i / kq, k = (i - b * kq) * 4u;
        const float4 v = b < batch ? load_x4<XBF16>(x, ldx, b, k) : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(xs + (size_t)b * KP + lds_index<CW>(k)) = v;
    }
    __syncthreads();
}

// Dot of one chunk position for R rows: acc[i][b] += Σ_groups d·Σc·x + m·Σx.
template <class E, int R, int B, class XS>
__device__ __forceinline__ void chunk_dot(const typename E::Chunk (&c)[R], const XS& xsrc, uint32_t k0,
                                          float (&acc)[R][B]) {
#pragma unroll
    for (int g = 0; g < E::NG; g++) {
        float part[R][B];
        float sx[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            sx[b] = 0.0f;
#pragma unroll
            for (int i = 0; i < R; i++) part[i][b] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < E::QUADS; q++) {
            const uint32_t k = k0 + (uint32_t)E::kofs(g, q);
            float cf[R][4];
#pragma unroll
            for (int i = 0; i < R; i++) {
                const uint32_t v = E::codes(c[i], g, q);
                cf[i][0] = ubyte_f32<0>(v);
                cf[i][1] = ubyte_f32<1>(v);
                cf[i][2] = ubyte_f32<2>(v);
                cf[i][3] = ubyte_f32<3>(v);
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const float4 xv = xsrc.load((uint32_t)b, k);
                sx[b] += (xv.x + xv.y) + (xv.z + xv.w);
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float a = part[i][b];
                    a = fmaf(cf[i][0], xv.x, a);
                    a = fmaf(cf[i][1], xv.y, a);
                    a = fmaf(cf[i][2], xv.z, a);
                    a = fmaf(cf[i][3], xv.w, a);
                    part[i][b] = a;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float d = E::scale(c[i], g), m = E::offset(c[i], g);
#pragma unroll
            for (int b = 0; b < B; b++) acc[i][b] = fmaf(m, sx[b], fmaf(d, part[i][b], acc[i][b]));
        }
    }
}

// Row block -> problem, its row count and first row (all wave-uniform: kept
// in scalar registers so selecting the problem's pointers never indexes the
// kernel-argument arrays dynamically).
struct RowBlock {
    uint32_t pi, n, base;
};

__device__ __forceinline__ RowBlock row_block(const GemvParams& p, uint32_t rb, uint32_t rows_per_rb) {
    uint32_t pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; i++) pi += (i < (int)p.nprob && rb >= p.rb_begin[i]) ? 1u : 0u;
    RowBlock r;
    r.pi = pi;
    r.n = pick(pi, p.n);
    r.base = (rb - pick(pi, p.rb_begin)) * rows_per_rb;
    return r;
}

template <int R, int B>
__device__ __forceinline__ void reduce_store(float (&acc)[R][B], const RowBlock& rb, uint32_t row0, uint32_t j,
                                             uint32_t L, const GemvParams& p) {
    for (uint32_t off = L >> 1; off > 0; off >>= 1) {
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int b = 0; b < B; b++) acc[i][b] += __shfl_xor(acc[i][b], (int)off, 64);
    }
    if (j == 0) {
        void* y = pick(rb.pi, p.y);
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t row = row0 + (uint32_t)i;
            if (row >= rb.n) continue;
#pragma unroll
            for (int b = 0; b < B; b++) {
                if ((uint32_t)b < p.batch) {
                    const size_t idx = (size_t)b * rb.n + row;
                    if (p.y_bf16) static_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(acc[i][b]);
                    else static_cast<float*>(y)[idx] = acc[i][b];
                }
            }
        }
    }
}

// The persistent task pipeline shared by all encodings.  load(rb, row, u)
// returns the raw bytes of chunk u of a row (rows past the end are clamped to
// the last row by the caller: in bounds, their sums are never stored).  Every
// load is unconditional — at the end of the sequence the current task is
// loaded again — so the compiler's wait counters can keep all of a lane's
// loads in flight across one task of compute.
template <class E, int R, int B, class XS, class LOAD>
__device__ __forceinline__ void gemv_pipeline(const GemvParams& p, const XS& xsrc, LOAD&& load) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t W = gridDim.x * (blockDim.x >> 6);
    const uint32_t L = 1u << p.lanes_log2;
    const uint32_t j = lane & (L - 1u), g = lane >> p.lanes_log2;
    const uint32_t rows_per_rb = (64u >> p.lanes_log2) * (uint32_t)R;
    const uint32_t cpl = (p.K / (uint32_t)E::CW) >> p.lanes_log2;  // chunks per lane per row block
    if (wid >= p.total_rb) return;
    const uint32_t T = (p.total_rb - wid + W - 1) / W * cpl;  // tasks of this wave

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
            dst[i] = load(rb, row, j + c * L);
        }
    };

    // Two register buffers in ping-pong (no copies between them, so waiting
    // for one buffer never waits for the loads in flight into the other).
    typename E::Raw ba[R], bb[R];
    uint32_t nrb = wid, nc = 0;  // the task loaded next
    RowBlock nblk = row_block(p, nrb, rows_per_rb);
    auto advance = [&](uint32_t t) {
        if (t + 1 < T) {  // wave-uniform; past the end the last task is loaded again
            if (++nc == cpl) {
                nc = 0;
                nrb += W;
                nblk = row_block(p, nrb, rows_per_rb);
            }
        }
    };
    auto compute = [&](const typename E::Raw (&buf)[R], const RowBlock& blk, uint32_t c) {
        typename E::Chunk ch[R];
#pragma unroll
        for (int i = 0; i < R; i++) ch[i] = E::unpack(buf[i]);
        chunk_dot<E, R, B>(ch, xsrc, (j + c * L) * (uint32_t)E::CW, acc);
        if (c + 1 == cpl) {
            reduce_store<R, B>(acc, blk, blk.base + g * (uint32_t)R, j, L, p);
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int b = 0; b < B; b++) acc[i][b] = 0.0f;
        }
    };
    load_task(ba, nblk, nc);
    uint32_t t = 0;
    for (; t + 2 <= T; t += 2) {
        // task t is in ba: load task t+1 into bb, compute ba
        RowBlock blk = nblk;
        uint32_t c = nc;
        advance(t);
        load_task(bb, nblk, nc);
        compute(ba, blk, c);
        // task t+1 is in bb: load task t+2 into ba, compute bb
        blk = nblk;
        c = nc;
        advance(t + 1);
        load_task(ba, nblk, nc);
        compute(bb, blk, c);
    }
    if (t < T) compute(ba, nblk, nc);  // odd task count: the last task is in ba
}

// ---------------------------------------------------------------- GGUF
// XL: activations staged in LDS (dynamic shared memory, lds_bytes<CW>(B, K)).
template <class E, int B, int R, bool XBF16, bool XL>
__global__ __launch_bounds__(256) void gguf_gemv_kernel(const GemvParams p) {
    extern __shared__ float xs_dyn[];
    if constexpr (XL) stage_x<E::CW, B, XBF16>(xs_dyn, p.x, p.K, p.ldx, p.batch);
    const size_t rowbytes = (size_t)(p.K / (uint32_t)E::CW) * E::BB;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) {
        return E::load_raw(pick(rb.pi, p.w) + (size_t)row * rowbytes, u);
    };
    if constexpr (XL) gemv_pipeline<E, R, B>(p, XLds<E::CW>{xs_dyn, p.K + 4u * (p.K / (uint32_t)E::CW)}, load);
    else gemv_pipeline<E, R, B>(p, XGlobal<XBF16>{p.x, p.ldx, p.batch}, load);
}

// ---------------------------------------------------------------- MLX affine U4
template <int B, int R, bool XBF16, bool XL>
__global__ __launch_bounds__(256) void mlx_u4_gemv_kernel(const GemvParams p) {
    using E = EncMlxU4;
    extern __shared__ float xs_dyn[];
    if constexpr (XL) stage_x<E::CW, B, XBF16>(xs_dyn, p.x, p.K, p.ldx, p.batch);
    const uint32_t ngroups = p.K / p.group;
    const uint32_t chunks_per_group = p.group / 32u;
    const bool f32s = p.sdtype == DT_F32;
    auto load = [&](const RowBlock& rb, uint32_t row, uint32_t u) {
        E::Raw r;
        const uint32_t* wbase = reinterpret_cast<const uint32_t*>(pick(rb.pi, p.w));
        load_dwords<4>(wbase + (size_t)row * (p.K / 8u) + (size_t)u * 4u, r.w);
        const size_t gi = (size_t)row * ngroups + u / chunks_per_group;
        const uint8_t* scb = pick(rb.pi, p.sc);
        const uint8_t* bib = pick(rb.pi, p.bi);
        if (f32s) {
            r.s = gptr<uint32_t>(scb)[gi];
            r.b = gptr<uint32_t>(bib)[gi];
        } else {
            r.s = gptr<uint16_t>(scb)[gi];
            r.b = gptr<uint16_t>(bib)[gi];
        }
        r.kind = p.sdtype;
        return r;
    };
    if constexpr (XL) gemv_pipeline<E, R, B>(p, XLds<E::CW>{xs_dyn, p.K + 4u * (p.K / (uint32_t)E::CW)}, load);
    else gemv_pipeline<E, R, B>(p, XGlobal<XBF16>{p.x, p.ldx, p.batch}, load);
}

// Rows per lane group for a register batch B: more rows amortise each
// activation load and Σx, fewer keep the accumulators in registers.
template <class E, int B>
constexpr int rows_per_group() {
    if constexpr (E::CW == 256) return 1;  // 53-dword super-blocks: keep occupancy >= 3 waves/SIMD
    else return B <= 2 ? 4 : (B <= 8 ? 2 : 1);
}

// Largest activation bytes staged in LDS per workgroup.
constexpr size_t kMaxLdsX = 64u * 1024u;

// Resident workgroups per CU for (kernel, dynamic LDS) on the current device
// and its CU count, cached after the first query (host side, thread-safe).
hipError_t cached_occupancy(const void* kernel, size_t lds, int* per_cu, int* cus);

// Launch of one kernel instantiation with a persistent grid: as many
// workgroups as fit on the device at once (capped by the row-block count).
template <class KERNEL>
hipError_t launch_persistent(KERNEL kernel, const GemvParams& p, size_t lds, hipStream_t st) {
    int cus = 0, per_cu = 0;
    hipError_t e = cached_occupancy(reinterpret_cast<const void*>(kernel), lds, &per_cu, &cus);
    if (e != hipSuccess) return e;
    const uint64_t want = ((uint64_t)p.total_rb + 3) / 4;  // 4 waves per workgroup
    const uint64_t cap = (uint64_t)(per_cu < 1 ? 1 : per_cu) * (uint64_t)cus;
    const uint32_t blocks = (uint32_t)(want < cap ? want : cap);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), lds, st, p);
    return hipGetLastError();
}

// Instantiates and launches the GEMV kernel of encoding E for a power-of-two
// register batch B <= BMAX.  GGUF decode takes f32 activations, the
// reference's precision contract for quantized linears
// (crates/dyninfer-compiler/src/lib.rs:289-306); bf16 activations reach GGUF
// weights only through the Q4_0 MFMA path.
template <class E, int BMAX>
hipError_t launch_gguf_gemv(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st) {
    if (xbf16) return hipErrorInvalidValue;
    const size_t lds = lds_bytes<E::CW>(B, p.K);
    const bool xl = lds <= kMaxLdsX;
#define DMX_CASE(b)                                                                                    \
    case b:                                                                                            \
        if constexpr (b <= BMAX) {                                                                     \
            constexpr int r = rows_per_group<E, b>();                                                  \
            return xl ? launch_persistent(gguf_gemv_kernel<E, b, r, false, true>, p, lds, st)          \
                      : launch_persistent(gguf_gemv_kernel<E, b, r, false, false>, p, 0, st);          \
        } else {                                                                                       \
            return hipErrorInvalidValue;                                                               \
        }
    switch (B) {
        DMX_CASE(1)
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
        DMX_CASE(16)
    default: return hipErrorInvalidValue;
    }
#undef DMX_CASE
}

inline hipError_t launch_mlx_gemv(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st) {
    const size_t lds = lds_bytes<EncMlxU4::CW>(B, p.K);
    const bool xl = lds <= kMaxLdsX;
#define DMX_CASE(b)                                                                                     \
    case b: {                                                                                           \
        constexpr int r = rows_per_group<EncMlxU4, b>();                                                \
        if (xbf16)                                                                                      \
            return xl ? launch_persistent(mlx_u4_gemv_kernel<b, r, true, true>, p, lds, st)             \
                      : launch_persistent(mlx_u4_gemv_kernel<b, r, true, false>, p, 0, st);             \
        return xl ? launch_persistent(mlx_u4_gemv_kernel<b, r, false, true>, p, lds, st)                \
                  : launch_persistent(mlx_u4_gemv_kernel<b, r, false, false>, p, 0, st);                \
    }
    switch (B) {
        DMX_CASE(1)
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
        DMX_CASE(16)
    default: return hipErrorInvalidValue;
    }
#undef DMX_CASE
}

}  // namespace dmx
