// Prefill activation staging for the MFMA GEMM: X [M, K] (f32 or bf16) to f16
// once per call, laid out as the GEMM's MFMA operands.
//
//   xh value of (m, k) = RNE_f16(x[m, k] · 2^(15 - e_m)),   rs[m] = 2^(e_m - 15),
//
// e_m the binary exponent of the row's largest magnitude (max |x| < 2^e_m),
// so every scaled value is below 2^15 (no f16 overflow) and the row's large
// values keep f16's full 11-bit precision.  The scaling is exact (a power of
// two); the one rounding is RNE to f16, relative 2^-11 for scaled magnitudes
// in f16's normal range.  A value more than 2^29 below its row's largest
// lands among f16's subnormals (absolute error <= 2^-25 scaled, i.e.
// 2^-40·max|x| per activation).  The GEMM accumulates x_h·w in f32 and
// multiplies each output row by rs[m].
//
// Layout: fragments of a v_mfma_f32_32x32x16_f16 operand, 1 KiB each:
//   fragment (mb, ks) = rows 32·mb .. 32·mb+31, k step ks (16 k), at element
//   offset ((mb·K/16 + ks)·64 + lane)·8; lane l holds row 32·mb + l % 32 and
//   8 k for lane half h = l / 32.
// The GEMM advances K in chunks of 64 (k steps 4c .. 4c+3), lane half h
// decoding the chunk's weight block h, so half h of step 4c+t holds 8 k of
// k = 64c + 32h .. 64c + 32h + 31, in the order the block's decode produces:
//   XFRAG_NIB  (Q4_0, Q4_1: code byte j holds k = j and k = j + 16):
//              4t, 4t+2, 4t+1, 4t+3, 16+4t, 18+4t, 17+4t, 19+4t
//   XFRAG_BYTE (Q8_0, Q6_K: one code byte per k):
//              8t, 8t+2, 8t+1, 8t+3, 8t+4, 8t+6, 8t+5, 8t+7
//              (pairs (j, j+2) of a dword decode together)
//   XFRAG_WORD (MLX U4: packed word t of the block holds k = 8t .. 8t+7, LSB
//              first): 8t, 8t+4, 8t+1, 8t+5, 8t+2, 8t+6, 8t+3, 8t+7
//              (nibbles j and j+4 of a word decode together).  Rows M .. roundup(M, 32) - 1
// are written as zeros, so the GEMM reads whole fragments.
//
// Mapping: one wave per row; lane l takes the 8-element output slots l, l+64,
// ... (slot 8c + 2t + h: chunk c, step t, half h).  K <= 4096 and M >= 1024:
// eight rows per 512-thread workgroup, whose slots meet in LDS and leave as
// whole 128-byte lines of the fragments.  Otherwise four rows per 256-thread
// workgroup, each lane storing its own 16-byte slots; rows with K <= 12288
// keep their values in registers between the max pass and the conversion
// pass, longer rows reload them (cache hits), four slots in flight per lane.
// NaN and inf: the row's scale is taken as 2^15 and the non-finite values
// propagate to the row's outputs.
#include "device_common.hpp"
#include "kernels.hpp"

namespace dmx {

namespace {

typedef _Float16 xh2 __attribute__((ext_vector_type(2)));
typedef float xf2 __attribute__((ext_vector_type(2)));
typedef float xf4 __attribute__((ext_vector_type(4)));

constexpr int kXprepWaves = 4;

// The 8 activations of output slot `slot` of a row: two runs of 4 k, at
// k0 and k0 + RUN2 (NIB: 16, BYTE and WORD: 4, i.e. one run of 8).
template <uint32_t LAYOUT>
__device__ __forceinline__ uint32_t slot_k0(uint32_t slot) {
    const uint32_t c = slot >> 3, t = (slot >> 1) & 3u, h = slot & 1u;
    return 64u * c + 32u * h + (LAYOUT == XFRAG_NIB ? 4u * t : 8u * t);
}
template <bool XBF16, uint32_t LAYOUT>
__device__ __forceinline__ void load8(const void* x, size_t row, uint32_t slot, float (&v)[8]) {
    constexpr uint32_t RUN2 = LAYOUT == XFRAG_NIB ? 16u : 4u;
    const size_t k0 = row + slot_k0<LAYOUT>(slot);
    if constexpr (XBF16) {
        typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
        const u32x2_a4 p = *gptr<u32x2_a4>(static_cast<const uint16_t*>(x) + k0);
        const u32x2_a4 q = *gptr<u32x2_a4>(static_cast<const uint16_t*>(x) + k0 + RUN2);
        const uint32_t w[4] = {p.x, p.y, q.x, q.y};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    } else {
        const xf4 a = *gptr<xf4>(static_cast<const float*>(x) + k0);
        const xf4 b = *gptr<xf4>(static_cast<const float*>(x) + k0 + RUN2);
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

// Element offset in xh of row m's output slot (chunk c, step t, half h).
__device__ __forceinline__ size_t frag_offset(uint32_t m, uint32_t slot, uint32_t ksteps) {
    const uint32_t c = slot >> 3, t = (slot >> 1) & 3u, h = slot & 1u;
    return (((size_t)(m >> 5) * ksteps + 4u * c + t) * 64u + (m & 31u) + 32u * h) * 8u;
}

// NIB and BYTE pair (v0, v2), (v1, v3), (v4, v6), (v5, v7); WORD pairs (v0, v4),
// (v1, v5), (v2, v6), (v3, v7).  Non-temporal stores: the staged operand is
// read by the next kernel, not by this one, and streaming it out during the
// kernel rather than leaving dirty L2 lines for the end-of-kernel write-back
// measured 7.3 -> 6.1 us at M = 2048, K = 1024.
typedef uint32_t xu4 __attribute__((ext_vector_type(4)));
template <uint32_t LAYOUT>
__device__ __forceinline__ xu4 pack8(const float (&v)[8], int sh) {
    return LAYOUT == XFRAG_WORD ? xu4{pk(v[0], v[4], sh), pk(v[1], v[5], sh), pk(v[2], v[6], sh), pk(v[3], v[7], sh)}
                                : xu4{pk(v[0], v[2], sh), pk(v[1], v[3], sh), pk(v[4], v[6], sh), pk(v[5], v[7], sh)};
}
template <uint32_t LAYOUT>
__device__ __forceinline__ void store8(uint16_t* xh, size_t off, const float (&v)[8], int sh) {
    __builtin_nontemporal_store(pack8<LAYOUT>(v, sh), gptr_mut<xu4>(xh + off));
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

// NR > 0: up to NR slots per lane held in registers (K <= 512·NR); NR = 0: reload.
template <bool XBF16, uint32_t LAYOUT, int NR>
__global__ __launch_bounds__(kXprepWaves * 64) void xprep_kernel(const void* __restrict__ x, uint32_t M, uint32_t Mp,
                                                                  uint32_t K, uint16_t* __restrict__ xh,
                                                                  float* __restrict__ rs) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t m = blockIdx.x * (uint32_t)kXprepWaves + (threadIdx.x >> 6);
    if (m >= Mp) return;
    const uint32_t slots = K / 8u, ksteps = K / 16u;
    if (m >= M) {  // padding row: zeros
        const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t g = lane; g < slots; g += 64u) store8<LAYOUT>(xh, frag_offset(m, g, ksteps), z, 0);
        if (lane == 0) gptr_mut<float>(rs)[m] = 0.0f;
        return;
    }
    const size_t row = (size_t)m * K;
    uint32_t mx = 0;
    float v[NR > 0 ? NR : 1][8];
    if constexpr (NR > 0) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const uint32_t g = lane + 64u * (uint32_t)i;
            if (g < slots) {
                load8<XBF16, LAYOUT>(x, row, g, v[i]);
                mx = absbits_max8(v[i], mx);
            }
        }
    } else {
        // four slots in flight per lane (cache hits on the second pass)
        for (uint32_t g0 = lane; g0 < slots; g0 += 256u) {
            float t[4][8];
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (g0 + 64u * i < slots) load8<XBF16, LAYOUT>(x, row, g0 + 64u * i, t[i]);
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (g0 + 64u * i < slots) mx = absbits_max8(t[i], mx);
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
            if (g < slots) store8<LAYOUT>(xh, frag_offset(m, g, ksteps), v[i], sh);
        }
    } else {
        for (uint32_t g0 = lane; g0 < slots; g0 += 256u) {
            float t[4][8];
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (g0 + 64u * i < slots) load8<XBF16, LAYOUT>(x, row, g0 + 64u * i, t[i]);
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (g0 + 64u * i < slots) store8<LAYOUT>(xh, frag_offset(m, g0 + 64u * i, ksteps), t[i], sh);
        }
    }
    if (lane == 0) gptr_mut<float>(rs)[m] = ldexpf(1.0f, e - 15);
}

// Rows of K <= kXprepLinesMaxK: eight rows per 512-thread workgroup (one wave
// each), the rows' 16-byte slots gathered in LDS so that the eight rows' slots
// of one (k step, half), consecutive in the fragment, leave as one 128-byte
// line: a store instruction writes 8 whole lines instead of 64 pieces of 64
// lines.
constexpr uint32_t kXprepLinesRows = 8, kXprepLinesMaxK = 4096, kXprepLinesMinRows = 1024;
template <bool XBF16, uint32_t LAYOUT, int NR>
__global__ __launch_bounds__(kXprepLinesRows * 64) void xprep_lines_kernel(const void* __restrict__ x, uint32_t M,
                                                                          uint32_t K, uint16_t* __restrict__ xh,
                                                                          float* __restrict__ rs) {
    static_assert(NR > 0 && NR * 512 <= (int)kXprepLinesMaxK, "the row's slots are held in registers");
    extern __shared__ xu4 tile[];  // [slot][row of the eight]: K · 16 bytes
    const uint32_t lane = threadIdx.x & 63u, r = threadIdx.x >> 6;
    const uint32_t m0 = blockIdx.x * kXprepLinesRows, m = m0 + r;  // Mp is a multiple of 8: m < Mp
    const uint32_t slots = K / 8u, ksteps = K / 16u;
    const bool real = m < M;  // rows M .. Mp - 1 are zeros
    const size_t row = real ? (size_t)m * K : 0u;
    uint32_t mx = 0;
    float v[NR][8];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const uint32_t g = lane + 64u * (uint32_t)i;
        if (g < slots) {
            load8<XBF16, LAYOUT>(x, row, g, v[i]);
#pragma unroll
            for (int q = 0; q < 8; q++) v[i][q] = real ? v[i][q] : 0.0f;
            mx = absbits_max8(v[i], mx);
        }
    }
    mx = wave_umax(mx);
    int e = mx >= 0x7F800000u ? 0 : (int)(mx >> 23) - 126;
    e = e < -110 ? -110 : e;
    const int sh = 15 - e;
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const uint32_t g = lane + 64u * (uint32_t)i;
        if (g < slots) tile[g * kXprepLinesRows + r] = pack8<LAYOUT>(v[i], sh);
    }
    if (lane == 0) gptr_mut<float>(rs)[m] = real ? ldexpf(1.0f, e - 15) : 0.0f;
    __syncthreads();
    // piece p = (slot g, row r') of the eight rows: line g at frag_offset(m0, g)
    for (uint32_t p = threadIdx.x; p < slots * kXprepLinesRows; p += kXprepLinesRows * 64u) {
        const uint32_t g = p / kXprepLinesRows, rr = p % kXprepLinesRows;
        __builtin_nontemporal_store(tile[p], gptr_mut<xu4>(xh + frag_offset(m0 + rr, g, ksteps)));
    }
}

template <bool XBF16, uint32_t LAYOUT>
hipError_t launch_xprep(const void* x, uint32_t M, uint32_t K, uint16_t* xh, float* rs, hipStream_t st) {
    const uint32_t Mp = (M + 31u) & ~31u;
    const dim3 grid((Mp + kXprepWaves - 1) / kXprepWaves), block(kXprepWaves * 64);
    const uint32_t slots = K / 8u;
    // (on fewer rows the 8-row workgroups are too few: M = 512, K = 1024 took
    // 14.5 us per prefill call against 14.1 with 4-row workgroups; at M =
    // 2048 the whole lines gave 28.0 -> 26.8 us at K = 1024, 38.7 -> 30.5 us
    // at K = 3072)
    if (K <= kXprepLinesMaxK && Mp >= kXprepLinesMinRows) {
        const dim3 lgrid(Mp / kXprepLinesRows), lblock(kXprepLinesRows * 64);
        const size_t lds = (size_t)K * 16u;  // 64 KiB at most
        if (slots <= 64u)
            hipLaunchKernelGGL((xprep_lines_kernel<XBF16, LAYOUT, 1>), lgrid, lblock, lds, st, x, M, K, xh, rs);
        else if (slots <= 128u)
            hipLaunchKernelGGL((xprep_lines_kernel<XBF16, LAYOUT, 2>), lgrid, lblock, lds, st, x, M, K, xh, rs);
        else if (slots <= 256u)
            hipLaunchKernelGGL((xprep_lines_kernel<XBF16, LAYOUT, 4>), lgrid, lblock, lds, st, x, M, K, xh, rs);
        else hipLaunchKernelGGL((xprep_lines_kernel<XBF16, LAYOUT, 8>), lgrid, lblock, lds, st, x, M, K, xh, rs);
        return hipGetLastError();
    }
    if (slots <= 64u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 1>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else if (slots <= 128u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 2>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else if (slots <= 256u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 4>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else if (slots <= 512u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 8>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else if (slots <= 1024u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 16>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else if (slots <= 1536u) hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 24>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    else hipLaunchKernelGGL((xprep_kernel<XBF16, LAYOUT, 0>), grid, block, 0, st, x, M, Mp, K, xh, rs);
    return hipGetLastError();
}

template <uint32_t LAYOUT>
hipError_t launch_xprep(const void* x, bool x_bf16, uint32_t M, uint32_t K, uint16_t* xh, float* rs, hipStream_t st) {
    return x_bf16 ? launch_xprep<true, LAYOUT>(x, M, K, xh, rs, st) : launch_xprep<false, LAYOUT>(x, M, K, xh, rs, st);
}

}  // namespace

hipError_t xprep_launch(const void* x, bool x_bf16, uint32_t M, uint32_t K, uint32_t layout, uint16_t* xh, float* rs,
                        hipStream_t st) {
    if (M == 0 || K == 0 || K % 64u) return hipErrorInvalidValue;
    switch (layout) {
        case XFRAG_NIB: return launch_xprep<XFRAG_NIB>(x, x_bf16, M, K, xh, rs, st);
        case XFRAG_BYTE: return launch_xprep<XFRAG_BYTE>(x, x_bf16, M, K, xh, rs, st);
        case XFRAG_WORD: return launch_xprep<XFRAG_WORD>(x, x_bf16, M, K, xh, rs, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dmx
