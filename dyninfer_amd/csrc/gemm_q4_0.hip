// Q4_0 prefill GEMM on gfx950 MFMA: Y[M, N] = X[M, K] · Wᵀ with f32 accumulation.
//
// Reference semantics: the same `emit_linear` contraction as decode
// (gguf_codegen.rs:268-314) with rows = the prefill window/chunk (512 when
// paged, parameter.rs:107-121, dense_decoder.rs:53-56).
//
// Data path (no repack: W is read as GGUF blocks straight from HBM):
//   * a workgroup (4 waves) computes a BM x BN tile of Y (64x128 or 128x64,
//     picked per shape so the grid covers the 256 CUs); each wave a 2x4 or
//     4x2 set of v_mfma_f32_16x16x32_f16 blocks;
//   * K advances 64 per stage (two Q4_0 blocks = two MFMA depths); the
//     global loads of stage s+3 are issued when stage s is staged, so three
//     stages (192 K) of loads are in flight behind the MFMA work;
//   * W: each thread loads Q4_0 blocks (realigned from 2-byte alignment) and
//     dequantises them to f16 in registers: the nibble becomes 1024+q by
//     OR-ing it under the f16 exponent of 1024 (exact), a packed f16 add gives
//     q-8 (exact) and a packed f16 multiply gives RNE_f16((q-8)·d) — one
//     rounding of the exact weight, relative error <= 2^-11;
//   * X: bf16 is narrowed to f16 with v_cvt_pkrtz (exact for |x| in f16's
//     normal range: bf16 carries 8 significant bits, f16 11);
//   * both operands are staged through double-buffered LDS (rows padded by 16
//     bytes so the 16 rows a fragment read touches fall in distinct banks);
//     one barrier per stage;
//   * tiles are ordered so that the tiles sharing W columns run on the same
//     XCD (workgroup i goes to XCD i % 8), reading each W block into one L2.
// Accuracy: |y - y_exact| <= 2^-11·Σ|w||x| + f32 accumulation error, inside
// the 2e-3 normalised tolerance.
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BK = 64;          // K per LDS stage (two Q4_0 blocks)
constexpr int PITCH = BK + 8;   // f16 elements per LDS row (+16 bytes)
constexpr int PREFETCH = 3;     // stages of global loads in flight

// 8 bf16 (one uint4) -> 8 f16 (4 dwords).
__device__ __forceinline__ uint4 bf16x8_to_f16(const uint4& a) {
    const uint32_t v[4] = {a.x, a.y, a.z, a.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = __uint_as_float(v[i] << 16);
        const float hi = __uint_as_float(v[i] & 0xFFFF0000u);
        // round-toward-zero is exact here: a bf16 value in f16's normal range
        // needs 8 significant bits.
        o[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Dequantise 16 weights of a Q4_0 block held in `e` (realigned block dwords):
// half 0 = low nibbles (k 0..15), half 1 = high nibbles (k 16..31), as 8
// dwords of consecutive f16 pairs.
__device__ __forceinline__ void q4_0_half_to_f16(const uint32_t (&e)[5], uint32_t half, uint32_t (&o)[8]) {
    const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(e[0] & 0xFFFFu));
    const h2 d2 = {dh, dh};
    const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const uint32_t shift = half * 4u;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t q = __builtin_amdgcn_alignbyte(e[t + 1], e[t], 2) >> shift;
        const uint32_t p0 = (__builtin_amdgcn_perm(q, q, 0x0C010C00u) & 0x000F000Fu) | 0x64006400u;
        const uint32_t p1 = (__builtin_amdgcn_perm(q, q, 0x0C030C02u) & 0x000F000Fu) | 0x64006400u;
        o[2 * t] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, p0) + off) * d2);
        o[2 * t + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, p1) + off) * d2);
    }
}

}  // namespace

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_q4_0_kernel(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                        void* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                                        uint32_t y_bf16) {
    static_assert(BM * BN == 8192, "tile must hold 8192 outputs (4 waves x 2048)");
    // 2x2 waves: 64x128 -> waves of 32x64; 128x64 -> waves of 64x32
    constexpr int TM = BM / 2 / 16;           // 16x16 tiles per wave along M
    constexpr int TN = BN / 2 / 16;           // 16x16 tiles per wave along N
    constexpr int XV = BM * BK * 2 / 16 / 256;  // uint4 of X per thread per stage
    constexpr int XT = BK * 2 / 16;              // uint4 per X row (8)
    // W blocks per stage: BN rows x 2 = 2*BN; each thread dequantises 32/WS weights of one block
    constexpr int WS = 256 / (2 * BN);           // threads per block: 1 (BN=128) or 2 (BN=64)
    constexpr int WW = 32 / WS;                  // weights per thread

    __shared__ __attribute__((aligned(16))) _Float16 sX[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 sW[2][BN * PITCH];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;

    // XCD-aware tile order: tiles sharing the same N range go to the same XCD.
    const uint32_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN, T = mt * nt;
    uint32_t tau = blockIdx.x;
    if (T % 8u == 0) tau = (blockIdx.x % 8u) * (T / 8u) + blockIdx.x / 8u;
    const uint32_t n0 = (tau / mt) * BN, m0 = (tau % mt) * BM;
    const uint32_t nkb = K / 32u;                         // Q4_0 blocks per row
    const uint32_t nst = (K + (uint32_t)BK - 1) / (uint32_t)BK;  // stages; the last holds one block when K % 64 == 32

    // X loader: thread covers XV consecutive uint4 of row xr starting at column xc (uint4 units)
    const uint32_t xr = tid * XV / XT, xc = (tid * XV) % XT;
    const bool xvalid = m0 + xr < M;
    const uint16_t* xsrc = X + (size_t)(xvalid ? m0 + xr : 0u) * K + xc * 8u;
    // W loader: thread covers weights [wh*WW, +WW) of block wb (0/1) of row wr
    const uint32_t wr = tid / (2u * WS), wb = (tid / WS) & 1u, wh = tid % WS;
    const bool wvalid = n0 + wr < N;
    const uint8_t* wsrc = W + (size_t)(wvalid ? n0 + wr : 0u) * nkb * 18u + wb * 18u;

    f4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    uint4 xreg[PREFETCH][XV];
    uint32_t wreg[PREFETCH][5], wsh[PREFETCH];
    // A thread's X columns and W block of a stage lie in one 32-wide Q4_0 block
    // (column block 2*st + xc/4, W block 2*st + wb); past K they are zero and
    // never loaded.
    const uint32_t xblk = xc / 4u;

    // Loads are unconditional (a block past K re-reads block 0 of the row, in
    // bounds, and is zeroed in lstore) so that the wait counters can keep all
    // PREFETCH stages in flight.
    auto gload = [&](int slot, uint32_t st) {
        const uint32_t xs = 2u * st + xblk < nkb ? st : 0u;
        const uint4* xp = reinterpret_cast<const uint4*>(xsrc + (size_t)xs * BK);
#pragma unroll
        for (int v = 0; v < XV; v++) {
            const u32x4_a4 t = *gptr<u32x4_a4>(xp + v);
            xreg[slot][v] = make_uint4(t.x, t.y, t.z, t.w);
        }
        const uint32_t wbk = 2u * st + wb < nkb ? 2u * st : 0u;
        const uintptr_t a = (uintptr_t)(wsrc + (size_t)wbk * 18u);
        wsh[slot] = (uint32_t)(a & 3u);
        load_dwords<5>(reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3), wreg[slot]);
    };
    // Out-of-range rows/blocks are zeroed with bit masks rather than selects:
    // a select lets the compiler branch around the conversion, and the branch
    // makes its wait-counter analysis fall back to waiting for every load.
    auto lstore = [&](int slot, int buf, uint32_t st) {
        const uint32_t xm = (xvalid && 2u * st + xblk < nkb) ? 0xFFFFFFFFu : 0u;
        const uint32_t wm_ = (wvalid && 2u * st + wb < nkb) ? 0xFFFFFFFFu : 0u;
        uint4* dx = reinterpret_cast<uint4*>(&sX[buf][xr * PITCH + xc * 8u]);
#pragma unroll
        for (int v = 0; v < XV; v++) {
            const uint4 c = bf16x8_to_f16(xreg[slot][v]);
            dx[v] = make_uint4(c.x & xm, c.y & xm, c.z & xm, c.w & xm);
        }
        uint32_t e[5];
        realign<5>(wreg[slot], wsh[slot], e);
        uint4* dw = reinterpret_cast<uint4*>(&sW[buf][wr * PITCH + wb * 32u + wh * WW]);
#pragma unroll
        for (int h = 0; h < WW / 16; h++) {
            uint32_t o[8];
            q4_0_half_to_f16(e, wh * (WW / 16) + h, o);
            dw[2 * h] = make_uint4(o[0] & wm_, o[1] & wm_, o[2] & wm_, o[3] & wm_);
            dw[2 * h + 1] = make_uint4(o[4] & wm_, o[5] & wm_, o[6] & wm_, o[7] & wm_);
        }
    };

#pragma unroll
    for (int s = 0; s < PREFETCH; s++) gload(s, (uint32_t)s < nst ? (uint32_t)s : 0u);

    const uint32_t fr = lane & 15u, fk = (lane >> 4) * 8u;
    const uint32_t arow = wm * (BM / 2), bcol = wn * (BN / 2);
    auto stage = [&](int slot, uint32_t st) {
        const int buf = (int)(st & 1u);
        lstore(slot, buf, st);
        gload(slot, st + PREFETCH < nst ? st + PREFETCH : st);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK / 32; kk++) {
            h8 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const h8*>(&sX[buf][(arow + i * 16u + fr) * PITCH + kk * 32u + fk]);
#pragma unroll
            for (int j = 0; j < TN; j++)
                b[j] = *reinterpret_cast<const h8*>(&sW[buf][(bcol + j * 16u + fr) * PITCH + kk * 32u + fk]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    uint32_t s0 = 0;
    for (; s0 + PREFETCH <= nst; s0 += PREFETCH) {
#pragma unroll
        for (int slot = 0; slot < PREFETCH; slot++) stage(slot, s0 + (uint32_t)slot);
    }
#pragma unroll
    for (int slot = 0; slot < PREFETCH; slot++)
        if (s0 + (uint32_t)slot < nst) stage(slot, s0 + (uint32_t)slot);

    // D layout of 16x16 MFMA: lane holds rows 4*(lane/16) + r, column lane%16.
    const uint32_t col_l = lane & 15u, row_l = (lane >> 4) * 4u;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const uint32_t col = n0 + bcol + j * 16u + col_l;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t row = m0 + arow + i * 16u + row_l + r;
                if (row < M && col < N) {
                    const size_t idx = (size_t)row * N + col;
                    if (y_bf16) static_cast<uint16_t*>(Y)[idx] = f32_to_bf16_bits(acc[i][j][r]);
                    else static_cast<float*>(Y)[idx] = acc[i][j][r];
                }
            }
        }
}

bool gemm_q4_0_supported(uint32_t N, uint32_t K, uint32_t M) {
    return N > 0 && M > 0 && K > 0 && K % 32u == 0;
}

hipError_t gemm_q4_0_launch(const uint8_t* w, uint32_t N, uint32_t K, const void* x, uint32_t M, void* y,
                            bool y_bf16, hipStream_t stream) {
    if (!gemm_q4_0_supported(N, K, M)) return hipErrorInvalidValue;
    // 64x128 tiles unless that leaves fewer workgroups than 128x64 would need
    // waves for (tall X, narrow W); both hold 8192 outputs.
    const uint32_t t_a = ((M + 63) / 64) * ((N + 127) / 128);
    const uint32_t t_b = ((M + 127) / 128) * ((N + 63) / 64);
    const auto* xp = static_cast<const uint16_t*>(x);
    if (M >= 2 * N || t_b < t_a) {
        hipLaunchKernelGGL((gemm_q4_0_kernel<128, 64>), dim3(t_b), dim3(256), 0, stream, w, xp, y, M, N, K,
                           y_bf16 ? 1u : 0u);
    } else {
        hipLaunchKernelGGL((gemm_q4_0_kernel<64, 128>), dim3(t_a), dim3(256), 0, stream, w, xp, y, M, N, K,
                           y_bf16 ? 1u : 0u);
    }
    return hipGetLastError();
}

}  // namespace dmx
