// Q4_0 prefill GEMM on gfx950 MFMA: Y[M, N] = X[M, K] · Wᵀ with f32 accumulation.
//
// Reference semantics: the same `emit_linear` contraction as decode
// (gguf_codegen.rs:268-314) with rows = the prefill window/chunk (512 when
// paged, parameter.rs:107-121, dense_decoder.rs:53-56).
//
// Data path (no repack: W is read as GGUF blocks straight from HBM):
//   * a workgroup computes a BM x BN tile of Y with WM x WN MMA waves, each
//     owning a (BM/WM) x (BN/WN) sub-tile of v_mfma_f32_32x32x16_f16 blocks
//     (two MFMA depths per Q4_0 block of 32; the 32x32 shape reads half the
//     LDS bytes per flop of the 16x16 one);
//   * the producer side (global loads, decode, LDS stores) either runs in the
//     MMA waves themselves, or in PW waves of its own so that one wave's decode
//     (VALU) overlaps another wave's MFMAs on each SIMD instead of all waves of
//     the tile doing the same phase at once;
//   * inside every 32-wide block, K is stored in LDS in the nibble decode order
//     (for each 8 consecutive k from k0: k0, k0+2, k0+1, k0+3, k0+4, k0+6,
//     k0+5, k0+7), for X and W alike, so the products pair up exactly as in
//     natural order, an X load of 8 staged f16 fills one such group, and one
//     v_and_or_b32 decodes two weights (bytes j and j+2 of a dword): a low nibble under the f16
//     exponent of 1024 is 1024+q, a high nibble (bits 4..7) under the exponent
//     of 64 is 64+q, both exact; a packed f16 add gives q-8 (exact) and a packed
//     f16 multiply RNE_f16((q-8)·d), a single rounding of the exact weight
//     (relative error <= 2^-11);
//   * X arrives as f16 from the prefill staging kernel (xprep.hip): each row
//     scaled by a power of two so that its largest magnitude is below 2^15,
//     rounded once (RNE), already in the permuted k order; the tile loads it
//     into LDS unchanged and the epilogue multiplies row m by rs[m];
//   * K advances BK per stage; the global loads run PF stages ahead in a
//     register ring; LDS is double buffered (rows padded by 16 bytes), one
//     barrier per stage;
//   * tiles are ordered so that the tiles sharing W columns run on the same
//     XCD (workgroup i goes to XCD i % 8), reading each W block into one L2.
// Accuracy: |y - y_exact| <= 2^-10·Σ|w||x| (one f16 rounding of each weight and
// of each activation) + f32 accumulation error, inside the 2e-3 normalised
// tolerance.
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

// (a & m) | b as one v_and_or_b32 (mask in a scalar register: a VOP3 op takes
// no literal operand on gfx9).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
    return r;
}

// Global loads and decode of one tile's X and W stages, spread over NT threads.
//
// LDS order inside each 32-wide block: group g (g = 0..3) holds k = 8g..8g+7 as
// the pairs (k0, k0+2), (k0+1, k0+3), (k0+4, k0+6), (k0+5, k0+7), k0 = 8g.
//   X unit: one row's 8 staged f16 of one group (one 16-byte load), copied.
//   W unit: half h of one row's block (the whole 18-byte block is loaded, two
//           loads): quant dwords 2h, 2h+1 hold the low nibbles of k = 8h..8h+7
//           (group h) and the high nibbles of k = 16+8h.. (group h+2); byte j of
//           a dword pairs with byte j+2 under one v_and_or_b32.
template <int BM, int BN, int NB, int PF, int NT>
struct Producer {
    static constexpr int PITCH = 32 * NB + 8;
    static constexpr int XU = BM * 4 * NB / NT;  // X units per thread per stage
    static constexpr int WU = BN * 2 * NB / NT;  // W units per thread per stage
    static_assert(XU >= 1 && WU >= 1 && XU * NT == BM * 4 * NB && WU * NT == BN * 2 * NB, "unit split");
    static constexpr int kLoads = XU + 2 * WU;        // global load instructions per stage
    static constexpr int kValu = 32 * WU;              // decode VALU instructions per stage (approximate)

    uint32_t xraw[PF][XU][4];  // the 8 staged f16 of group g
    uint32_t wraw[PF][WU][5];  // the block's dwords from the aligned dword holding its first byte
    const uint16_t* xrow[XU];
    const uint32_t* wrow[WU];
    uint32_t wsh[WU], wback[WU];
    uint32_t ptid, nkb;

    __device__ __forceinline__ void xunit(int i, uint32_t& r, uint32_t& g8) const {
        const uint32_t u = ptid + (uint32_t)i * NT;
        r = u / (4u * NB);
        g8 = u % (4u * NB);
    }
    __device__ __forceinline__ void wunit(int i, uint32_t& r, uint32_t& b, uint32_t& h) const {
        const uint32_t u = ptid + (uint32_t)i * NT;
        r = u / (2u * NB);
        b = (u / 2u) % (uint32_t)NB;
        h = u & 1u;
    }

    // Per-unit addresses, computed once: rows past M/N re-read the last row (in
    // bounds; their outputs are never stored).  A stage advances X by 32·NB
    // elements and W by NB 18-byte blocks (a multiple of 4 bytes, so a block's
    // byte shift within its dword never changes).
    __device__ __forceinline__ void init(const uint8_t* W, const uint16_t* X, uint32_t tid, uint32_t m0, uint32_t n0,
                                         uint32_t M, uint32_t N, uint32_t K) {
        ptid = tid;
        nkb = K / 32u;
        const size_t rowbytes = (size_t)nkb * 18u;
#pragma unroll
        for (int i = 0; i < XU; i++) {
            uint32_t r, g8;
            xunit(i, r, g8);
            const uint32_t m = m0 + r < M ? m0 + r : M - 1u;
            xrow[i] = X + (size_t)m * K + 8u * g8;
        }
#pragma unroll
        for (int i = 0; i < WU; i++) {
            uint32_t r, b, h;
            wunit(i, r, b, h);
            const uint32_t n = n0 + r < N ? n0 + r : N - 1u;
            const uintptr_t a0 = (uintptr_t)W + (size_t)n * rowbytes;  // block 0 of stage 0
            const uintptr_t a = a0 + b * 18u;
            wsh[i] = (uint32_t)(a & 3u);
            wrow[i] = reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3);
            // dwords back from this block's aligned base to the stage's first block's
            wback[i] = (uint32_t)(((a & ~(uintptr_t)3) - (a0 & ~(uintptr_t)3)) / 4u);
        }
    }

    // Blocks of the last stage past K are missing when K % (32·NB) != 0: such
    // a unit re-reads its stage's first block (which exists, in bounds) and
    // lstore zeroes its d (X: the product with a zero weight is zero).
    __device__ __forceinline__ bool blk_ok(uint32_t st, uint32_t b) const { return (uint32_t)NB * st + b < nkb; }

    // Loads are unconditional so the wait counters can keep all PF stages in flight.
    __device__ __forceinline__ void gload(int slot, uint32_t st) {
#pragma unroll
        for (int i = 0; i < XU; i++) {
            uint32_t r, g8;
            xunit(i, r, g8);
            const uint32_t b = g8 / 4u;
            const uint16_t* xp = xrow[i] + (size_t)st * (32 * NB) - (blk_ok(st, b) ? 0u : 32u * b);
            const u32x4_a4 v = *gptr<u32x4_a4>(xp);
            xraw[slot][i][0] = v.x;
            xraw[slot][i][1] = v.y;
            xraw[slot][i][2] = v.z;
            xraw[slot][i][3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < WU; i++) {
            uint32_t r, b, h;
            wunit(i, r, b, h);
            const uint32_t* al = wrow[i] + (size_t)st * (NB * 18 / 4) - (blk_ok(st, b) ? 0u : wback[i]);
            load_dwords<5>(al, wraw[slot][i]);  // every dword overlaps the block's 18 bytes
        }
    }

    // Decode/convert ring slot `slot` (stage st) into the LDS tiles dx, dw.
    __device__ __forceinline__ void lstore(int slot, _Float16* dx, _Float16* dw, uint32_t st) {
#pragma unroll
        for (int i = 0; i < XU; i++) {
            uint32_t r, g8;
            xunit(i, r, g8);
            const uint32_t* q = xraw[slot][i];
            *reinterpret_cast<uint4*>(&dx[r * PITCH + 8u * g8]) = make_uint4(q[0], q[1], q[2], q[3]);
        }
        const h2 off_lo = {(_Float16)-1032.0f, (_Float16)-1032.0f};
        const h2 off_hi = {(_Float16)-72.0f, (_Float16)-72.0f};
        const uint32_t mag_lo = 0x64006400u, mag_hi = 0x54005400u;
#pragma unroll
        for (int i = 0; i < WU; i++) {
            uint32_t r, b, h;
            wunit(i, r, b, h);
            const uint32_t* q = wraw[slot][i];
            const uint32_t sh = wsh[i];
            const uint32_t dbits = blk_ok(st, b) ? (q[0] >> (8u * sh)) : 0u;  // a missing block weighs zero
            const h2 d2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(dbits, dbits, 0x01000100u));
            const uint32_t sel = 0x05040302u + 0x01010101u * sh;  // quant dword t = block bytes 2+4t..5+4t
            // quant dwords 2h and 2h+1 (raw dwords 2h..2h+2)
            const uint32_t qa = __builtin_amdgcn_perm(h ? q[3] : q[1], h ? q[2] : q[0], sel);
            const uint32_t qb = __builtin_amdgcn_perm(h ? q[4] : q[2], h ? q[3] : q[1], sel);
            auto wv = [&](uint32_t c, h2 off) {
                return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, c) + off) * d2);
            };
            const uint32_t a8 = qa >> 8, b8 = qb >> 8;
            // low nibbles: group h (k0 = 8h): (k0, k0+2) (k0+1, k0+3) from qa, (k0+4, k0+6) (k0+5, k0+7) from qb
            *reinterpret_cast<uint4*>(&dw[r * PITCH + b * 32u + 8u * h]) =
                make_uint4(wv(and_or(qa, 0x000F000Fu, mag_lo), off_lo), wv(and_or(a8, 0x000F000Fu, mag_lo), off_lo),
                           wv(and_or(qb, 0x000F000Fu, mag_lo), off_lo), wv(and_or(b8, 0x000F000Fu, mag_lo), off_lo));
            // high nibbles: group h + 2 (k0 = 16 + 8h)
            *reinterpret_cast<uint4*>(&dw[r * PITCH + b * 32u + 8u * h + 16u]) =
                make_uint4(wv(and_or(qa, 0x00F000F0u, mag_hi), off_hi), wv(and_or(a8, 0x00F000F0u, mag_hi), off_hi),
                           wv(and_or(qb, 0x00F000F0u, mag_hi), off_hi), wv(and_or(b8, 0x00F000F0u, mag_hi), off_hi));
        }
    }
};

// One MMA wave's sub-tile: TM x TN blocks of 32x32 (v_mfma_f32_32x32x16_f16),
// fragments read from LDS.  Operand layout: lane l holds row (or column)
// l % 32 and the 8 k at 8·(l / 32) of the instruction's 16.
template <int BM, int BN, int WM, int WN, int NB>
struct Consumer {
    static constexpr int PITCH = 32 * NB + 8;
    static constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    static_assert(TM * 32 * WM == BM && TN * 32 * WN == BN, "tile must split into 32x32 blocks per wave");
    f32x16 acc[TM][TN];
    uint32_t fr, fk, arow, bcol, lane;

    __device__ __forceinline__ void init(uint32_t lane_, uint32_t cw) {
        lane = lane_;
        fr = lane & 31u;
        fk = (lane >> 5) * 8u;
        arow = (cw / WN) * (BM / WM);
        bcol = (cw % WN) * (BN / WN);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    }

    // A stage's fragments, all read before the first MFMA so that LDS latency
    // is paid once per stage rather than once per MFMA depth.
    struct Frags {
        h8 a[2 * NB][TM], b[2 * NB][TN];
    };

    __device__ __forceinline__ void load(const _Float16* ax, const _Float16* bw, Frags& f) const {
#pragma unroll
        for (int kk = 0; kk < 2 * NB; kk++) {
#pragma unroll
            for (int i = 0; i < TM; i++)
                f.a[kk][i] = *reinterpret_cast<const h8*>(&ax[(arow + i * 32u + fr) * PITCH + kk * 16u + fk]);
#pragma unroll
            for (int j = 0; j < TN; j++)
                f.b[kk][j] = *reinterpret_cast<const h8*>(&bw[(bcol + j * 32u + fr) * PITCH + kk * 16u + fk]);
        }
    }

    __device__ __forceinline__ void mma(const Frags& f) {
#pragma unroll
        for (int kk = 0; kk < 2 * NB; kk++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[kk][i], f.b[kk][j], acc[i][j], 0, 0, 0);
    }

    static constexpr int kMfmas = 2 * NB * TM * TN;

    // D layout of 32x32 MFMA: lane holds column lane%32 and, for r = 0..15,
    // row 8·(r/4) + 4·(lane/32) + r%4.  Row m's sums are multiplied by its
    // staging factor rs[m] (rs covers the rows of every tile, past M too).
    __device__ __forceinline__ void store(void* Y, const float* rs, uint32_t m0, uint32_t n0, uint32_t M, uint32_t N,
                                          uint32_t y_bf16) {
        const uint32_t col_l = lane & 31u, row_l = (lane >> 5) * 4u;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            float f[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4 v = *gptr<f32x4>(rs + m0 + arow + i * 32u + 8u * q + row_l);
                f[4 * q] = v[0]; f[4 * q + 1] = v[1]; f[4 * q + 2] = v[2]; f[4 * q + 3] = v[3];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t col = n0 + bcol + j * 32u + col_l;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t row = m0 + arow + i * 32u + 8u * (r >> 2) + row_l + (r & 3);
                    if (row < M && col < N) {
                        const size_t idx = (size_t)row * N + col;
                        const float v = acc[i][j][r] * f[r];
                        if (y_bf16) gptr_mut<uint16_t>(Y)[idx] = f32_to_bf16_bits(v);
                        else gptr_mut<float>(Y)[idx] = v;
                    }
                }
            }
        }
    }
};

}  // namespace

// WM x WN MMA waves plus PW producer waves (PW = 0: the MMA waves also
// produce).  BK: K per LDS stage (a multiple of 32); PF: stages of global
// loads in flight.
template <int BM, int BN, int WM, int WN, int PW, int BK, int PF>
__global__ __launch_bounds__((WM * WN + PW) * 64) void gemm_q4_0_kernel(const uint8_t* __restrict__ W,
                                                                         const uint16_t* __restrict__ X,
                                                                         const float* __restrict__ rs,
                                                                         void* __restrict__ Y, uint32_t M, uint32_t N,
                                                                         uint32_t K, uint32_t y_bf16) {
    constexpr int NB = BK / 32;
    constexpr int PITCH = BK + 8;
    constexpr int NT = (PW > 0 ? PW : WM * WN) * 64;  // producer threads
    using P = Producer<BM, BN, NB, PF, NT>;
    using C = Consumer<BM, BN, WM, WN, NB>;

    extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
    _Float16* sX = smem;                   // [2][BM * PITCH]
    _Float16* sW = smem + 2 * BM * PITCH;  // [2][BN * PITCH]
    auto bufx = [&](uint32_t s) { return sX + (s & 1u) * BM * PITCH; };
    auto bufw = [&](uint32_t s) { return sW + (s & 1u) * BN * PITCH; };

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware tile order: tiles sharing the same N range go to the same XCD.
    const uint32_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN, T = mt * nt;
    uint32_t tau = blockIdx.x;
    if (T % 8u == 0) tau = (blockIdx.x % 8u) * (T / 8u) + blockIdx.x / 8u;
    const uint32_t n0 = (tau / mt) * BN, m0 = (tau % mt) * BM;
    const uint32_t nst = (K + (uint32_t)BK - 1) / (uint32_t)BK;  // stages; the last may hold fewer than NB blocks

    auto last = [&](uint32_t t) { return t < nst ? t : nst - 1u; };

    if constexpr (PW == 0) {
        // Every wave loads, decodes and multiplies.  Prologue: PF stages of
        // loads in flight (stages past the end re-load the last one), stage 0
        // decoded into LDS buffer 0, barrier.  Stage s, branch-free: refill
        // ring slot s % PF with stage s + PF, read all of stage s's fragments
        // (buffer s & 1), then the MFMAs of stage s interleaved with
        // the decode of stage s + 1 into the other buffer (past the end: the
        // last stage again, never read), barrier.  The MFMAs run in the matrix
        // core while the decode's VALU work issues between them.
        P p;
        C c;
        p.init(W, X, tid, m0, n0, M, N, K);
        c.init(lane, wave);
#pragma unroll
        for (int s = 0; s < PF; s++) p.gload(s, last((uint32_t)s));
        p.lstore(0, bufx(0), bufw(0), 0);
        __syncthreads();
        auto iter = [&](int slot, uint32_t s) {
            p.gload(slot, last(s + PF));
            __builtin_amdgcn_sched_barrier(0);  // the loads leave first, before anything waits
            typename C::Frags f;
            c.load(bufx(s), bufw(s), f);
            c.mma(f);
            p.lstore((slot + 1) % PF, bufx(s + 1), bufw(s + 1), last(s + 1));
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * NB * (C::TM + C::TN), 0);  // DS reads
#pragma unroll
            for (int m = 0; m < C::kMfmas; m++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                     // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, P::kValu / C::kMfmas, 0);  // decode VALU
            }
            __syncthreads();
        };
        uint32_t s0 = 0;
        for (; s0 + PF <= nst; s0 += PF) {
#pragma unroll
            for (int slot = 0; slot < PF; slot++) iter(slot, s0 + (uint32_t)slot);
        }
#pragma unroll
        for (int slot = 0; slot < PF; slot++)
            if (s0 + (uint32_t)slot < nst) iter(slot, s0 + (uint32_t)slot);
        c.store(Y, rs, m0, n0, M, N, y_bf16);
    } else {
        // PW producer waves load and decode stage s + 1 while the MMA waves
        // multiply stage s; one barrier per stage (wave-uniform split: every
        // wave passes the same 1 + nst barriers).
        if (wave < (uint32_t)PW) {
            P p;
            p.init(W, X, tid, m0, n0, M, N, K);
#pragma unroll
            for (int s = 0; s < PF; s++) p.gload(s, last((uint32_t)s));
            p.lstore(0, bufx(0), bufw(0), 0);
            __syncthreads();
            auto iter = [&](int slot, uint32_t s) {
                p.gload(slot, last(s + PF));
                p.lstore((slot + 1) % PF, bufx(s + 1), bufw(s + 1), last(s + 1));
                __syncthreads();
            };
            uint32_t s0 = 0;
            for (; s0 + PF <= nst; s0 += PF) {
#pragma unroll
                for (int slot = 0; slot < PF; slot++) iter(slot, s0 + (uint32_t)slot);
            }
#pragma unroll
            for (int slot = 0; slot < PF; slot++)
                if (s0 + (uint32_t)slot < nst) iter(slot, s0 + (uint32_t)slot);
        } else {
            C c;
            c.init(lane, wave - PW);
            __syncthreads();
            for (uint32_t s = 0; s < nst; s++) {
                typename C::Frags f;
                c.load(bufx(s), bufw(s), f);
                c.mma(f);
                __syncthreads();
            }
            c.store(Y, rs, m0, n0, M, N, y_bf16);
        }
    }
}

bool gemm_q4_0_supported(uint32_t N, uint32_t K, uint32_t M) {
    return N > 0 && M > 0 && K > 0 && K % 32u == 0;
}

namespace {

template <int BM, int BN, int WM, int WN, int PW, int BK, int PF>
hipError_t launch_tile(const uint8_t* w, uint32_t N, uint32_t K, const uint16_t* x, const float* rs, uint32_t M,
                       void* y, uint32_t yb, hipStream_t st) {
    auto kernel = gemm_q4_0_kernel<BM, BN, WM, WN, PW, BK, PF>;
    constexpr int kThreads = (WM * WN + PW) * 64;
    constexpr size_t lds = (size_t)2 * (BM + BN) * (BK + 8) * sizeof(_Float16);
    if constexpr (lds > 64u * 1024u) {
        static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return attr;
    }
    const uint32_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL(kernel, dim3(tiles), dim3(kThreads), lds, st, w, x, rs, y, M, N, K, yb);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_q4_0_launch(const uint8_t* w, uint32_t N, uint32_t K, const uint16_t* xp, const float* rs, uint32_t M,
                            void* y, bool y_bf16, hipStream_t stream) {
    if (!gemm_q4_0_supported(N, K, M)) return hipErrorInvalidValue;
    const uint32_t yb = y_bf16 ? 1u : 0u;
    auto tiles = [&](uint32_t bm, uint32_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    // The largest tile (most reuse of each decoded weight and converted
    // activation) that still gives most CUs a workgroup.  The 128x128 tile
    // runs eight producer waves beside its eight MMA waves.  Launches too small
    // for these tiles take the K-split kernel (K a multiple of 256), whose four
    // waves per tile each multiply a quarter of K.  (Chosen from timing sweeps
    // of M in {128, 512, 2048} at the Qwen3-0.6B FFN shapes: at M = 128 and
    // for K = 3072 the K-split kernel takes 40-60% less time, at M = 512 with
    // 192 tiles of 128x64 5% more.)
    constexpr uint32_t kCus = 256;
    if (tiles(128, 128) >= kCus) return launch_tile<128, 128, 2, 4, 8, 64, 2>(w, N, K, xp, rs, M, y, yb, stream);
    if (tiles(128, 64) >= kCus * 3 / 4) return launch_tile<128, 64, 4, 2, 0, 128, 2>(w, N, K, xp, rs, M, y, yb, stream);
    if (gemm_q4_0_ks_supported(N, K, M)) return gemm_q4_0_ks_launch(w, N, K, xp, rs, M, y, y_bf16, stream);
    return launch_tile<64, 64, 2, 2, 0, 128, 2>(w, N, K, xp, rs, M, y, yb, stream);
}

}  // namespace dmx
