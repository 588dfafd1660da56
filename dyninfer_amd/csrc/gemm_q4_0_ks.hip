// Prefill GEMM, GGUF Q4_0, K split over the waves of a workgroup:
// Y[M, N] = X[M, K] · Wᵀ with W Q4_0 blocks (N rows of K/32 blocks), f32
// accumulation (gguf_codegen.rs:268-314 `emit_linear`, the Q4_0 dequantisation
// of :412-472).  X arrives staged by xprep.hip: f16 rows scaled by a power of
// two (factor rs[m] applied in the epilogue), k permuted as 0,2,1,3,4,6,5,7
// inside every group of 8.
//
// A workgroup owns one BM×BN tile of Y and splits K into four quarters, one
// per wave, so each wave is an independent pipeline with no barrier until the
// final reduction:
//   * per chunk of 64 k (two Q4_0 blocks) a wave copies its X rows and its W
//     row windows from global memory straight into a wave-private LDS buffer
//     (global_load_lds_dwordx4: 16 bytes per lane, consecutive lanes on
//     consecutive pieces of a row, so a load instruction touches a few cache
//     lines), three buffers deep, with no registers held for loads in flight.
//     X rows keep 128 bytes with their 16-byte pieces XOR-swizzled by row (a
//     16-row fragment read hits 16 distinct bank groups); a W row window is the
//     chunk's 36 bytes from its 4-byte-aligned start as three 16-byte pieces
//     from window bytes 0, 16, 20 + 2·sh (each touching only dwords that hold
//     bytes of the chunk, so no load leaves a page the chunk touches);
//   * each lane reads its v_mfma_f32_16x16x32_f16 operands from LDS: an X
//     fragment (8 staged f16 of one row, in the order one v_and_or_b32
//     decodes nibbles in: 0,2,1,3,4,6,5,7) used as it is, a W
//     fragment 8 weights of one row from 8 qs bytes (low nibbles under the f16
//     exponent of 1024, high nibbles under that of 64, a packed add giving q-8
//     exactly, a packed multiply by d: RNE_f16((q-8)·d), a weight's one
//     rounding);
//   * one block's operands are decoded while the previous block's MFMAs run
//     (scheduling-group barriers interleave them);
//   * the four K-partials meet in LDS: each wave owns every fourth 16×16 tile,
//     the others hand it theirs, the owner adds, scales row m by rs[m] and
//     stores.
// Error: 2^-10·Σ|w||x| (one f16 rounding of each weight and of each staged
// activation) plus f32 accumulation.
#include <type_traits>

#include "encodings.hpp"

namespace dmx {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef half2_t h2;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t __attribute__((may_alias)) u32a;  // LDS dwords written as u32x4

constexpr int kKsWaves = 4;      // K quarters, one per wave
constexpr uint32_t kKsKC = 64;   // k per chunk: two Q4_0 blocks
constexpr uint32_t kKsBufs = 3;  // LDS chunk buffers per wave
constexpr uint32_t kWPitch = 48; // LDS bytes per W row window: three 16-byte pieces

// (a & m) | b, every operand a vector register (m and b differ between lanes)
__device__ __forceinline__ uint32_t and_or_v(uint32_t a, uint32_t m, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(b));
    return r;
}

template <int BM, int BN>
struct Ks {
    static constexpr int TM = BM / 16, TN = BN / 16;  // 16×16 tiles
    static constexpr int NXL = BM / 8;                // X pieces per lane per chunk (8 per row)
    static constexpr int NWS = 3 * BN;                // W pieces per chunk
    static constexpr int NWL = (NWS + 63) / 64;       // W pieces per lane per chunk
    static constexpr uint32_t XB = BM * 128u, WB = NWL * 1024u;  // one chunk buffer: X rows, W pieces
    static constexpr uint32_t WAVE = kKsBufs * (XB + WB);
    static constexpr uint32_t RED = (uint32_t)kKsWaves * TM * TN * 1024u;  // f32 partials [wave][tile][lane][4]
    static constexpr uint32_t LDS = (kKsWaves * WAVE > RED ? kKsWaves * WAVE : RED) + 16u;
    static_assert(BM % 16 == 0 && BN % 16 == 0, "16x16 tiles");
    static_assert(LDS <= 160u * 1024u, "LDS of one workgroup");
};

// 16 bytes per lane from global memory into LDS at dst + 16·lane (dst
// wave-uniform): global_load_lds_dwordx4, counted by vmcnt.
__device__ __forceinline__ void dma16(const void* src, uint8_t* dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// s_waitcnt vmcnt(n) (other counters unconstrained)
template <uint32_t n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8));
}

}  // namespace

template <int BM, int BN, int BSH>
__global__ __launch_bounds__(kKsWaves * 64) void gemm_q4_0_ks_kernel(const uint8_t* __restrict__ w,
                                                                       const uint16_t* __restrict__ x,
                                                                       const float* __restrict__ rs, void* y,
                                                                       uint32_t M, uint32_t N, uint32_t K,
                                                                       uint32_t y_bf16) {
    using T = Ks<BM, BN>;
    constexpr int TM = T::TM, TN = T::TN, NXL = T::NXL, NWL = T::NWL;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t* area = lds + wv * T::WAVE;  // this wave's chunk buffers: [buf][X rows | W pieces]

    // tile: consecutive workgroups take consecutive column tiles, so the
    // workgroups of one XCD (i mod 8) share column tiles, i.e. W rows
    const uint32_t tiles_n = (N + BN - 1u) / BN;
    const uint32_t tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kw = wv * (K / kKsWaves), nch = K / kKsWaves / kKsKC;  // this wave's K range, chunks
    const uint32_t rowbytes = (K / 32u) * 18u;  // a multiple of 144 (K is a multiple of 256)
    const uint8_t* abase = w - BSH;             // 4-byte aligned; chunk windows start at abase + row·rowbytes + 18·kb

    // ---- per-lane constants
    // X DMA: instruction i, lane l -> LDS piece 64i + l = (row 8i + l/8, slot
    // l%8), which holds the row's k-piece g = slot ^ ((row/2) % 8)
    uint32_t xg[NXL];
#pragma unroll
    for (int i = 0; i < NXL; i++) {
        const uint32_t r = 8u * (uint32_t)i + (lane >> 3), g = (lane & 7u) ^ ((r >> 1) & 7u);
        xg[i] = 2u * ((m0 + r < M ? m0 + r : M - 1u) * K + 8u * g);
    }
    // W DMA: instruction i, lane l -> LDS piece s = 64i + l = (row s/3, piece
    // s%3; past the last: a copy of the last); pieces 0, 1, 2 start at window
    // bytes 0, 16, 20 + 2·BSH
    uint32_t wg[NWL];
#pragma unroll
    for (int i = 0; i < NWL; i++) {
        const uint32_t s = 64u * (uint32_t)i + lane < (uint32_t)T::NWS ? 64u * (uint32_t)i + lane : (uint32_t)T::NWS - 1u;
        const uint32_t r = s / 3u, pc = s % 3u;
        wg[i] = (n0 + r < N ? n0 + r : N - 1u) * rowbytes + (pc == 0u ? 0u : (pc == 1u ? 16u : 20u + 2u * BSH));
    }
    // X fragment of step s (k 32s..32s+31 of the chunk), lane (row rr, k-piece
    // 4s + kq): LDS row rr at piece (4s + kq) ^ ((rr/2) % 8)
    const uint32_t rr = lane & 15u, kq = lane >> 4, swz = (rr >> 1) & 7u;
    const uint32_t xo0 = rr * 128u + 16u * (kq ^ swz), xo1 = rr * 128u + 16u * ((4u + kq) ^ swz);
    // W decode: block s of a chunk starts at window byte BSH + 18s (d), its qs
    // at BSH + 18s + 2; a lane takes qs bytes 8h..8h+7 (h = lane/16 % 2) as
    // three window dwords from (BSH + 18s + 2 + 8h) / 4; window dword k sits at
    // LDS dword k (k < 8) or k + 3 - BSH/2 (piece 2)
    const uint32_t h = (lane >> 4) & 1u;
    const uint32_t wrow = T::XB + rr * kWPitch;  // from the buffer start
    uint32_t wo[2][3];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const uint32_t k = (BSH + 18u * (uint32_t)s + 2u) / 4u + 2u * h + (uint32_t)j;
            wo[s][j] = wrow + 4u * (k < 8u ? k : k + 3u - BSH / 2u);
        }
    // lanes 0..31 decode low nibbles (k 0..15 of a block), 32..63 high nibbles
    const bool hiq = lane >= 32u;
    const uint32_t vmask = hiq ? 0x00F000F0u : 0x000F000Fu, vmagic = hiq ? 0x54005400u : 0x64006400u;
    const _Float16 voff = hiq ? (_Float16)-72.0f : (_Float16)-1032.0f;
    const h2 off2 = {voff, voff};

    auto buf = [&](uint32_t c) { return area + (c % kKsBufs) * (T::XB + T::WB); };
    auto dma = [&](uint32_t c) {
        const uint32_t k0 = kw + c * kKsKC;
        const uint8_t* xb = reinterpret_cast<const uint8_t*>(x + k0);  // uniform bases, per-lane 32-bit offsets
        const uint8_t* wb = abase + (k0 / 32u) * 18u;
        uint8_t* d = buf(c);
#pragma unroll
        for (int i = 0; i < NXL; i++) dma16(xb + xg[i], d + 1024u * (uint32_t)i);
#pragma unroll
        for (int i = 0; i < NWL; i++) dma16(wb + wg[i], d + T::XB + 1024u * (uint32_t)i);
    };
    // One 32-k step (one block of each W row) in two stages: fetch() reads
    // the LDS words (X pieces, the W qs dwords and d), decode() decodes W into
    // the MFMA operands (the X pieces are operands as they are).
    struct Raw {
        u32x4 x[TM];
        uint32_t q[TN][3], d[TN];
    };
    struct Frags {
        u32x4 a[TM], b[TN];
    };
    auto fetch = [&](auto step, const uint8_t* bp, Raw& r) {
        constexpr uint32_t s = decltype(step)::value;
        constexpr uint32_t dob = BSH + 18u * s;  // d of block s
#pragma unroll
        for (int mg = 0; mg < TM; mg++)
            r.x[mg] = *reinterpret_cast<const u32x4*>(bp + (s ? xo1 : xo0) + 2048u * (uint32_t)mg);
#pragma unroll
        for (int g = 0; g < TN; g++) {
            const uint8_t* rp = bp + 16u * kWPitch * (uint32_t)g;
            r.d[g] = *reinterpret_cast<const u32a*>(rp + wrow + 4u * (dob / 4u));
#pragma unroll
            for (int j = 0; j < 3; j++) r.q[g][j] = *reinterpret_cast<const u32a*>(rp + wo[s][j]);
        }
    };
    auto decode = [&](auto step, const Raw& r, Frags& f) {
        constexpr uint32_t s = decltype(step)::value;
        constexpr uint32_t dob = BSH + 18u * s;
        constexpr uint32_t sel = 0x03020100u + 0x01010101u * ((dob + 2u) & 3u);  // realigns the qs dwords
#pragma unroll
        for (int mg = 0; mg < TM; mg++) f.a[mg] = r.x[mg];  // k0,k2 k1,k3 k4,k6 k5,k7
#pragma unroll
        for (int g = 0; g < TN; g++) {
            const h2 d2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(r.d[g], r.d[g], (dob & 3u) ? 0x07060706u : 0x05040504u));
            const uint32_t D0 = __builtin_amdgcn_perm(r.q[g][1], r.q[g][0], sel);
            const uint32_t D1 = __builtin_amdgcn_perm(r.q[g][2], r.q[g][1], sel);
            auto wq = [&](uint32_t c) {
                return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, and_or_v(c, vmask, vmagic)) + off2) * d2);
            };
            f.b[g] = u32x4{wq(D0), wq(D0 >> 8), wq(D1), wq(D1 >> 8)};  // k 0,2 1,3 4,6 5,7
        }
    };
    f32x4 acc[TM][TN];
#pragma unroll
    for (int mg = 0; mg < TM; mg++)
#pragma unroll
        for (int g = 0; g < TN; g++) acc[mg][g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [&](const Frags& f) {
#pragma unroll
        for (int mg = 0; mg < TM; mg++)
#pragma unroll
            for (int g = 0; g < TN; g++)
                acc[mg][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, f.a[mg]),
                                                                    __builtin_bit_cast(h8, f.b[g]), acc[mg][g], 0, 0, 0);
    };
    constexpr int kMfmas = TM * TN;
    constexpr int kValu = 17 * TN;            // one step's decode
    constexpr int kReads = TM + 4 * TN;       // one step's LDS reads
    auto interleave = [&]() {
#pragma unroll
        for (int m = 0; m < kMfmas; m++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, (kReads + kMfmas - 1) / kMfmas, 0);   // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x002, (kValu + kMfmas - 1) / kMfmas, 0);    // VALU
        }
    };
    constexpr uint32_t kPer = (uint32_t)(NXL + NWL);  // DMA instructions per chunk
    using S0 = std::integral_constant<uint32_t, 0>;
    using S1 = std::integral_constant<uint32_t, 1>;
    // Software pipeline over steps (two per chunk): in step t the MFMAs of t,
    // the decode of t+1 and the LDS reads of t+2 run together.  Chunk c sits
    // in buffer c % 3; its copy is requested at the start of chunk c-2 (into
    // chunk c-3's buffer, whose last reads were decoded in chunk c-2's
    // predecessor) and awaited at the start of chunk c-1.
    Raw ra, rb;
    Frags fa, fb;
    dma(0u);
    if (nch > 1u) {
        dma(1u);
        wait_vmcnt<kPer>();  // chunk 0 arrived, chunk 1 may be in flight
    } else {
        wait_vmcnt<0>();
    }
    fetch(S0{}, buf(0u), ra);
    fetch(S1{}, buf(0u), rb);
    decode(S0{}, ra, fa);
    // state at the start of chunk c: fa = operands of step 2c, rb = words of
    // step 2c+1, chunk c+1's copy requested
    for (uint32_t c = 0; c + 1u < nch; c++) {
        if (c + 2u < nch) {
            dma(c + 2u);
            wait_vmcnt<kPer>();  // chunk c+1 arrived
        } else {
            wait_vmcnt<0>();
        }
        const uint8_t* bn = buf(c + 1u);
        fetch(S0{}, bn, ra);
        decode(S1{}, rb, fb);
        mma(fa);
        interleave();
        fetch(S1{}, bn, rb);
        decode(S0{}, ra, fa);
        mma(fb);
        interleave();
    }
    decode(S1{}, rb, fb);
    mma(fa);
    interleave();
    mma(fb);

    // ---- the four K-partials: tile t = mg·TN + g belongs to wave t % 4
    __syncthreads();  // every wave is done with its chunk area
    f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int mg = 0; mg < TM; mg++)
#pragma unroll
        for (int g = 0; g < TN; g++) {
            const uint32_t t = (uint32_t)(mg * TN + g);
            if (t % kKsWaves != wv) red[(wv * (uint32_t)(TM * TN) + t) * 64u + lane] = acc[mg][g];
        }
    __syncthreads();
#pragma unroll
    for (int mg = 0; mg < TM; mg++)
#pragma unroll
        for (int g = 0; g < TN; g++) {
            const uint32_t t = (uint32_t)(mg * TN + g);
            if (t % kKsWaves != wv) continue;
            f32x4 v = acc[mg][g];
#pragma unroll
            for (uint32_t o = 0; o < (uint32_t)kKsWaves; o++)
                if (o != wv) v += red[(o * (uint32_t)(TM * TN) + t) * 64u + lane];
            // lane l holds rows 4(l/16)..+3 of column l % 16
            const uint32_t n = n0 + 16u * (uint32_t)g + (lane & 15u);
            const uint32_t mb = m0 + 16u * (uint32_t)mg + 4u * (lane >> 4);
            const f32x4 f = *gptr<f32x4>(rs + mb);  // rs covers whole row groups past M
            const float fr[4] = {f[0], f[1], f[2], f[3]};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t m = mb + (uint32_t)e;
                if (m < M && n < N) {
                    const size_t idx = (size_t)m * N + n;
                    const float o = v[e] * fr[e];
                    if (y_bf16) gptr_mut<uint16_t>(y)[idx] = f32_to_bf16_bits(o);
                    else gptr_mut<float>(y)[idx] = o;
                }
            }
        }
}

namespace {

template <int BM, int BN>
hipError_t launch_ks(const uint8_t* w, uint32_t N, uint32_t K, const uint16_t* x, const float* rs, uint32_t M, void* y,
                     uint32_t yb, hipStream_t st) {
    auto kernel = ((uintptr_t)w & 3u) ? gemm_q4_0_ks_kernel<BM, BN, 2> : gemm_q4_0_ks_kernel<BM, BN, 0>;
    constexpr size_t lds = Ks<BM, BN>::LDS;
    if constexpr (lds > 64u * 1024u) {
        static hipError_t attr0 = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_q4_0_ks_kernel<BM, BN, 0>),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        static hipError_t attr2 = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_q4_0_ks_kernel<BM, BN, 2>),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr0 != hipSuccess) return attr0;
        if (attr2 != hipSuccess) return attr2;
    }
    const uint32_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL(kernel, dim3(tiles), dim3(kKsWaves * 64), lds, st, w, x, rs, y, M, N, K, yb);
    return hipGetLastError();
}

}  // namespace

bool gemm_q4_0_ks_supported(uint32_t N, uint32_t K, uint32_t M) {
    // activation offsets are 32-bit element indices
    return N > 0 && M > 0 && K > 0 && K % (kKsWaves * kKsKC) == 0 && (uint64_t)M * K < (1ull << 31);
}

hipError_t gemm_q4_0_ks_launch(const uint8_t* w, uint32_t N, uint32_t K, const uint16_t* xp, const float* rs,
                               uint32_t M, void* y, bool y_bf16, hipStream_t stream) {
    if (!gemm_q4_0_ks_supported(N, K, M)) return hipErrorInvalidValue;
    const uint32_t yb = y_bf16 ? 1u : 0u;
    auto tiles = [&](uint32_t bm, uint32_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    constexpr uint32_t kCus = 256;
    if (tiles(64, 96) >= kCus) return launch_ks<64, 96>(w, N, K, xp, rs, M, y, yb, stream);
    if (tiles(64, 64) >= kCus) return launch_ks<64, 64>(w, N, K, xp, rs, M, y, yb, stream);
    if (tiles(32, 64) >= kCus) return launch_ks<32, 64>(w, N, K, xp, rs, M, y, yb, stream);
    return launch_ks<32, 32>(w, N, K, xp, rs, M, y, yb, stream);
}

}  // namespace dmx
