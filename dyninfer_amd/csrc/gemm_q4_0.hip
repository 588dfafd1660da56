// Q4_0 prefill GEMM on gfx950 MFMA: Y[M, N] = X[M, K] · Wᵀ with f32 accumulation.
//
// Reference semantics: the same `emit_linear` contraction as decode
// (gguf_codegen.rs:268-314) with rows = the prefill window/chunk (512 when
// paged, parameter.rs:107-121, dense_decoder.rs:53-56).
//
// Data path (no repack: W is read as GGUF blocks straight from HBM):
//   * each workgroup (4 waves, 2x2) computes a 128x128 tile of Y; each wave a
//     64x64 sub-tile as 4x4 v_mfma_f32_16x16x32_f16 blocks;
//   * the K loop advances one Q4_0 block (32) per step — exactly one MFMA depth;
//   * W: each thread loads one 18-byte block (realigned from 2-byte alignment)
//     and dequantises 16 of its weights to f16 in registers: the nibble becomes
//     1024+q by OR-ing it under the f16 exponent of 1024 (exact), one packed
//     f16 add gives q-8 (exact) and one packed f16 multiply gives
//     RNE_f16((q-8)·d) — a single rounding of the exact weight, relative error
//     <= 2^-11;
//   * X: bf16 is widened and re-narrowed to f16 (exact for |x| in f16's normal
//     range; bf16 has 8 significant bits, f16 11);
//   * both operands are staged through double-buffered LDS tiles (row pitch
//     padded to 80 bytes so the 16 rows a fragment read touches fall in
//     distinct banks); one barrier per K step.
// Accuracy: |y - y_exact| <= 2^-11 · Σ|w||x| + f32 accumulation error, inside
// the 2e-3 normalised tolerance.
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int PITCH = 40;  // f16 elements per LDS row: 32 + 8 padding (80 bytes)

// 16 bf16 (two uint4) -> 16 f16 packed in 8 dwords.
__device__ __forceinline__ void bf16x16_to_f16(const uint4& a, const uint4& b, uint32_t (&o)[8]) {
    const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float lo = __uint_as_float(v[i] << 16);
        const float hi = __uint_as_float(v[i] & 0xFFFF0000u);
        // round-toward-zero is exact here: a bf16 value in f16's normal range
        // needs 8 significant bits.
        o[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
}

// Dequantise the 16 weights of a Q4_0 block held in `e` (realigned block
// dwords) selected by `half` (0: low nibbles = k 0..15, 1: high = k 16..31)
// into 8 dwords of consecutive f16 pairs.
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
        const h2 w0 = (__builtin_bit_cast(h2, p0) + off) * d2;
        const h2 w1 = (__builtin_bit_cast(h2, p1) + off) * d2;
        o[2 * t] = __builtin_bit_cast(uint32_t, w0);
        o[2 * t + 1] = __builtin_bit_cast(uint32_t, w1);
    }
}
}  // namespace

__global__ __launch_bounds__(256) void gemm_q4_0_kernel(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                        void* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                                        uint32_t y_bf16) {
    __shared__ __attribute__((aligned(16))) _Float16 sX[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 sW[2][BN * PITCH];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t nkb = K / BK;

    // Loader role: tile row lr, half lh of the 32-wide K step.
    const uint32_t lr = tid >> 1, lh = tid & 1u;
    const bool xvalid = m0 + lr < M;
    const bool wvalid = n0 + lr < N;
    const uint16_t* xsrc = X + (size_t)(xvalid ? m0 + lr : 0u) * K + lh * 16u;
    const uint8_t* wsrc = W + (size_t)(wvalid ? n0 + lr : 0u) * nkb * 18u;

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    uint4 xr0, xr1;
    uint32_t wr[5], wsh;
    auto gload = [&](uint32_t kb) {
        const uint4* xp = reinterpret_cast<const uint4*>(xsrc + (size_t)kb * BK);
        xr0 = xp[0];
        xr1 = xp[1];
        const uintptr_t a = (uintptr_t)(wsrc + (size_t)kb * 18u);
        wsh = (uint32_t)(a & 3u);
        load_dwords<5>(reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3), wr);
    };
    auto lstore = [&](int buf) {
        uint32_t xh[8], wh[8];
        bf16x16_to_f16(xr0, xr1, xh);
        uint32_t e[5];
        realign(wr, wsh, e);
        q4_0_half_to_f16(e, lh, wh);
        uint4* dx = reinterpret_cast<uint4*>(&sX[buf][lr * PITCH + lh * 16u]);
        uint4* dw = reinterpret_cast<uint4*>(&sW[buf][lr * PITCH + lh * 16u]);
        const uint4 z = make_uint4(0, 0, 0, 0);
        dx[0] = xvalid ? make_uint4(xh[0], xh[1], xh[2], xh[3]) : z;
        dx[1] = xvalid ? make_uint4(xh[4], xh[5], xh[6], xh[7]) : z;
        dw[0] = wvalid ? make_uint4(wh[0], wh[1], wh[2], wh[3]) : z;
        dw[1] = wvalid ? make_uint4(wh[4], wh[5], wh[6], wh[7]) : z;
    };

    gload(0);
    lstore(0);
    __syncthreads();
    const uint32_t fr = lane & 15u, fk = (lane >> 4) * 8u;
    for (uint32_t kb = 0; kb < nkb; kb++) {
        const int cur = (int)(kb & 1u);
        if (kb + 1 < nkb) gload(kb + 1);
        h8 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = *reinterpret_cast<const h8*>(&sX[cur][(wm * 64u + i * 16u + fr) * PITCH + fk]);
            b[i] = *reinterpret_cast<const h8*>(&sW[cur][(wn * 64u + i * 16u + fr) * PITCH + fk]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        if (kb + 1 < nkb) lstore(cur ^ 1);
        __syncthreads();
    }

    // D layout of 16x16 MFMA: lane holds rows 4*(lane/16) + r, column lane%16.
    const uint32_t col_l = lane & 15u, row_l = (lane >> 4) * 4u;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t col = n0 + wn * 64u + j * 16u + col_l;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t row = m0 + wm * 64u + i * 16u + row_l + r;
                if (row < M && col < N) {
                    const size_t idx = (size_t)row * N + col;
                    if (y_bf16) static_cast<uint16_t*>(Y)[idx] = f32_to_bf16_bits(acc[i][j][r]);
                    else static_cast<float*>(Y)[idx] = acc[i][j][r];
                }
            }
        }
}

bool gemm_q4_0_supported(uint32_t N, uint32_t K, uint32_t M) {
    return N > 0 && M > 0 && K > 0 && K % 32 == 0;
}

hipError_t gemm_q4_0_launch(const uint8_t* w, uint32_t N, uint32_t K, const void* x, uint32_t M, void* y,
                            bool y_bf16, hipStream_t stream) {
    if (!gemm_q4_0_supported(N, K, M)) return hipErrorInvalidValue;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(gemm_q4_0_kernel, grid, dim3(256), 0, stream, w, static_cast<const uint16_t*>(x), y, M, N, K,
                       y_bf16 ? 1u : 0u);
    return hipGetLastError();
}

}  // namespace dmx
