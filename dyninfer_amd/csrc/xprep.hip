// Prefill activation staging for the MFMA GEMMs: X [M, K] (f32 or bf16) to
// f16 once per call, in the k order the GEMMs' weight decode produces.
//
//   xh[m, :] = RNE_f16(x[m, :] · 2^(15 - e_m)),   rs[m] = 2^(e_m - 15),
//
// e_m the binary exponent of the row's largest magnitude (max |x| < 2^e_m),
// so every scaled value is below 2^15 (no f16 overflow) and the row's large
// values keep f16's full 11-bit precision.  The scaling is exact (a power of
// two); the one rounding is RNE to f16, relative 2^-11 for scaled magnitudes
// in f16's normal range.  A value more than 2^29 below its row's largest
// lands among f16's subnormals (absolute error <= 2^-25 scaled, i.e.
// 2^-40·max|x| per activation).  The GEMMs accumulate x_h·w in f32 and
// multiply the tile by rs[m] in the epilogue.
//
// k order inside every group of 8 (the permutation is applied identically to
// the weights' LDS tiles, so products pair up as in natural order):
//   XPERM_PAIR2: 0, 2, 1, 3, 4, 6, 5, 7   one v_and_or_b32 decodes bytes j and
//                j+2 of a dword (GGUF Q4_0/Q4_1/Q8_0 codes, Q6_K ql/qh);
//   XPERM_PAIR4: 0, 4, 1, 5, 2, 6, 3, 7   nibbles i and i+4 of an MLX u32 word.
//
// Mapping: one wave per row (4 rows per 256-thread workgroup); lane l takes
// the 8-element groups l, l+64, ...  Rows with K <= 2048 keep their values in
// registers between the max pass and the conversion pass; longer rows reload
// them (cache hits).  NaN and inf: the row's scale is taken as 2^15 and the
// non-finite values propagate to the row's outputs.
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

namespace {

typedef _Float16 xh2 __attribute__((ext_vector_type(2)));
typedef float xf2 __attribute__((ext_vector_type(2)));
typedef float xf4 __attribute__((ext_vector_type(4)));

constexpr int kXprepWaves = 4;

template <bool XBF16>
__device__ __forceinline__ void load8(const void* x, size_t off, float (&v)[8]) {
    if constexpr (XBF16) {
        const u32x4_a4 q = *gptr<u32x4_a4>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(q[i] << 16);
            v[2 * i + 1] = __uint_as_float(q[i] & 0xFFFF0000u);
        }
    } else {
        const xf4 a = *gptr<xf4>(static_cast<const float*>(x) + off);
        const xf4 b = *gptr<xf4>(static_cast<const float*>(x) + off + 4);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    }
}

__device__ __forceinline__ uint32_t absbits_max8(const float (&v)[8], uint32_t m) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t b = __float_as_uint(v[i]) & 0x7FFFFFFFu;  // |x| bits order as unsigned integers
        m = b > m ? b : m;
    }
    return m;
}

__device__ __forceinline__ uint32_t pk(float a, float b, int sh) {
    const xf2 f = {ldexpf(a, sh), ldexpf(b, sh)};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, xh2));  // RNE
}

template <uint32_t PERM>
__device__ __forceinline__ void store8(uint16_t* xh, size_t off, const float (&v)[8], int sh) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 o;
    if constexpr (PERM == XPERM_PAIR2) {
        o = u32x4{pk(v[0], v[2], sh), pk(v[1], v[3], sh), pk(v[4], v[6], sh), pk(v[5], v[7], sh)};
    } else {
        o = u32x4{pk(v[0], v[4], sh), pk(v[1], v[5], sh), pk(v[2], v[6], sh), pk(v[3], v[7], sh)};
    }
    *gptr_mut<u32x4>(xh + off) = o;
}

// Maximum over the wave (unsigned), every lane receiving it.
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t u = (uint32_t)__shfl_xor((int)v, o, 64);
        v = u > v ? u : v;
    }
    return v;
}

// NR > 0: up to NR groups per lane held in registers (K <= 512·NR); NR = 0: reload.
template <bool XBF16, uint32_t PERM, int NR>
__global__ __launch_bounds__(kXprepWaves * 64) void xprep_kernel(const void* __restrict__ x, uint32_t M, uint32_t K,
                                                                  uint16_t* __restrict__ xh, float* __restrict__ rs) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t m = blockIdx.x * (uint32_t)kXprepWaves + (threadIdx.x >> 6);
    if (m >= M) return;
    const uint32_t groups = K / 8u;
    const size_t row = (size_t)m * K;
    uint32_t mx = 0;
    float v[NR > 0 ? NR : 1][8];
    if constexpr (NR > 0) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const uint32_t g = lane + 64u * (uint32_t)i;
            if (g < groups) {
                load8<XBF16>(x, row + 8u * g, v[i]);
                mx = absbits_max8(v[i], mx);
            }
        }
    } else {
        for (uint32_t g = lane; g < groups; g += 64u) {
            float t[8];
            load8<XBF16>(x, row + 8u * g, t);
            mx = absbits_max8(t, mx);
        }
    }
    mx = wave_umax(mx);
    // binary exponent e of the largest magnitude (|x| < 2^e): biased exponent
    // - 126 for normal values; zero and subnormal rows clamp to -110 (so
    // 2^(15 - e) stays a normal f32); inf / NaN rows take e = 0
    int e = mx >= 0x7F800000u ? 0 : (int)(mx >> 23) - 126;
    e = e < -110 ? -110 : e;
    const int sh = 15 - e;
    if constexpr (NR > 0) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const uint32_t g = lane + 64u * (uint32_t)i;
            if (g < groups) store8<PERM>(xh, row + 8u * g, v[i], sh);
        }
    } else {
        for (uint32_t g = lane; g < groups; g += 64u) {
            float t[8];
            load8<XBF16>(x, row + 8u * g, t);
            store8<PERM>(xh, row + 8u * g, t, sh);
        }
    }
    if (lane == 0) gptr_mut<float>(rs)[m] = ldexpf(1.0f, e - 15);
}

template <bool XBF16, uint32_t PERM>
hipError_t launch_xprep(const void* x, uint32_t M, uint32_t K, uint16_t* xh, float* rs, hipStream_t st) {
    const dim3 grid((M + kXprepWaves - 1) / kXprepWaves), block(kXprepWaves * 64);
    const uint32_t groups = K / 8u;
    if (groups <= 64u) hipLaunchKernelGGL((xprep_kernel<XBF16, PERM, 1>), grid, block, 0, st, x, M, K, xh, rs);
    else if (groups <= 128u) hipLaunchKernelGGL((xprep_kernel<XBF16, PERM, 2>), grid, block, 0, st, x, M, K, xh, rs);
    else if (groups <= 256u) hipLaunchKernelGGL((xprep_kernel<XBF16, PERM, 4>), grid, block, 0, st, x, M, K, xh, rs);
    else hipLaunchKernelGGL((xprep_kernel<XBF16, PERM, 0>), grid, block, 0, st, x, M, K, xh, rs);
    return hipGetLastError();
}

}  // namespace

hipError_t xprep_launch(const void* x, bool x_bf16, uint32_t M, uint32_t K, uint32_t perm, uint16_t* xh, float* rs,
                        hipStream_t st) {
    if (M == 0 || K == 0 || K % 8u || (perm != XPERM_PAIR2 && perm != XPERM_PAIR4)) return hipErrorInvalidValue;
    if (perm == XPERM_PAIR2)
        return x_bf16 ? launch_xprep<true, XPERM_PAIR2>(x, M, K, xh, rs, st)
                      : launch_xprep<false, XPERM_PAIR2>(x, M, K, xh, rs, st);
    return x_bf16 ? launch_xprep<true, XPERM_PAIR4>(x, M, K, xh, rs, st)
                  : launch_xprep<false, XPERM_PAIR4>(x, M, K, xh, rs, st);
}

}  // namespace dmx
