// Decode GEMV dispatch: lays out the wave grid over up to four weights that
// share one activation, picks the lanes-per-row split, and calls the
// per-encoding instantiations (gemv_<enc>.hip; kernels in gemv_kernels.hpp).
#include <mutex>
#include <vector>

#include "kernels.hpp"

namespace dmx {

hipError_t gemv_launch_q4_0(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q4_1(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q8_0(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q6_k(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q4_k(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q5_k(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_iq4_xs(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);
hipError_t gemv_launch_mlx_u4(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st);

hipError_t cached_occupancy(const void* kernel, size_t lds, int threads, int* per_cu, int* cus) {
    struct Entry {
        const void* kernel;
        size_t lds;
        int dev, per_cu, cus;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (const Entry& c : cache)
            if (c.kernel == kernel && c.lds == lds && c.dev == dev) {
                *per_cu = c.per_cu;
                *cus = c.cus;
                return hipSuccess;
            }
    }
    int n = 0, blocks = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess && lds > 64u * 1024u)
        e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, lds);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    cache.push_back({kernel, lds, dev, blocks, n});
    *per_cu = blocks;
    *cus = n;
    return hipSuccess;
}

// LDS one workgroup may use on the current device (cached per device).
static hipError_t lds_limit(uint32_t* out) {
    static std::mutex mu;
    static std::vector<std::pair<int, uint32_t>> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& c : cache)
        if (c.first == dev) {
            *out = c.second;
            return hipSuccess;
        }
    int v = 0;
    e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return e;
    const uint32_t lim = (uint32_t)v < kLdsBytes ? (uint32_t)v : kLdsBytes;
    cache.push_back({dev, lim});
    *out = lim;
    return hipSuccess;
}

bool gemv_k_supported(uint32_t enc, uint32_t K) { return xtile_bytes(enc, 1, K) <= kLdsBytes; }

namespace {

struct EncInfo {
    uint32_t chunk_weights;  // weights one lane handles per step
    bool wide;               // 64-weight chunks (Q6_K, Q4_K, Q5_K): fewer chunks per lane in latency mode
};

bool enc_info(uint32_t enc, EncInfo& e) {
    switch (enc) {
    case ENC_Q4_0:
    case ENC_Q4_1:
    case ENC_Q8_0:
    case ENC_IQ4_XS:
    case ENC_MLX_U4: e = {32, false}; return true;
    case ENC_Q6_K: e = {64, true}; return true;
    case ENC_Q4_K:
    case ENC_Q5_K: e = {64, true}; return true;
    default: return false;
    }
}

hipError_t launch(uint32_t enc, const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st) {
    switch (enc) {
    case ENC_Q4_0: return gemv_launch_q4_0(p, B, oneshot, xbf16, st);
    case ENC_Q4_1: return gemv_launch_q4_1(p, B, oneshot, xbf16, st);
    case ENC_Q8_0: return gemv_launch_q8_0(p, B, oneshot, xbf16, st);
    case ENC_Q6_K: return gemv_launch_q6_k(p, B, oneshot, xbf16, st);
    case ENC_Q4_K: return gemv_launch_q4_k(p, B, oneshot, xbf16, st);
    case ENC_Q5_K: return gemv_launch_q5_k(p, B, oneshot, xbf16, st);
    case ENC_IQ4_XS: return gemv_launch_iq4_xs(p, B, oneshot, xbf16, st);
    case ENC_MLX_U4: return gemv_launch_mlx_u4(p, B, oneshot, xbf16, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

uint64_t gemv_workspace_bytes(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t batch, uint32_t K,
                              bool y_bf16, uint32_t group) {
    if (nprob < 1 || nprob > kMaxProblems) return 0;
    return gemv_mfma_workspace_bytes(enc, probs, nprob, batch, K, y_bf16, group);
}

hipError_t gemv_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x, bool x_bf16,
                       uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, void* work, uint64_t work_bytes,
                       hipStream_t stream) {
    EncInfo info;
    if (!enc_info(enc, info) || nprob < 1 || nprob > kMaxProblems || batch < 1 || batch > (uint32_t)kMaxGemvBatch)
        return hipErrorInvalidValue;
    // 5..16 activation rows: every weight decoded once for all rows, on MFMA
    if (gemv_mfma_applies(enc, probs, nprob, batch, K, y_bf16, group))
        return gemv_mfma_launch(enc, probs, nprob, K, x, x_bf16, batch, y_bf16, group, sdtype, work, work_bytes,
                                stream);
    // bf16 outputs and K in several segments: on MFMA when the workspace holds f32 accumulators
    if (y_bf16 && work) {
        const uint64_t need = gemv_mfma_bf16_acc_bytes(enc, probs, nprob, batch, K, group);
        if (need && work_bytes >= need)
            return gemv_mfma_launch_bf16_acc(enc, probs, nprob, K, x, x_bf16, batch, group, sdtype, work, work_bytes,
                                             stream);
    }
    // Register batch: the next power of two, halved while its activation tile
    // does not fit one workgroup's LDS; larger batches run as several passes.
    uint32_t lim = 0;
    hipError_t le = lds_limit(&lim);
    if (le != hipSuccess) return le;
    uint32_t B = 1;
    while (B < batch && B < max_register_batch(enc)) B *= 2;
    while (B > 1 && xtile_bytes(enc, B, K) > lim) B /= 2;
    if (xtile_bytes(enc, B, K) > lim) return hipErrorInvalidValue;
    if (batch > B) {
        const size_t xes = x_bf16 ? 2 : 4, yes = y_bf16 ? 2 : 4;
        for (uint32_t r0 = 0; r0 < batch; r0 += B) {
            const uint32_t nb = batch - r0 < B ? batch - r0 : B;
            GemvProblem sub[kMaxProblems];
            for (int i = 0; i < nprob; i++) {
                sub[i] = probs[i];
                sub[i].y = static_cast<uint8_t*>(probs[i].y) + (size_t)r0 * probs[i].n * yes;
            }
            const void* xr = static_cast<const uint8_t*>(x) + (size_t)r0 * K * xes;
            hipError_t e = gemv_launch(enc, sub, nprob, K, xr, x_bf16, nb, y_bf16, group, sdtype, nullptr, 0, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const uint32_t nch = K / info.chunk_weights;
    // Lanes per row group: the largest power of two <= min(64, chunks), so the
    // lanes of a wave read one contiguous run of rows (each load instruction
    // covers consecutive blocks; splitting a wave over distant rows costs DRAM
    // locality) and a row block's chunks need few rounds.  When L does not
    // divide the chunk count, the lanes past the last chunk add zero.
    uint32_t L = 1;
    while (L < 64 && 2 * L <= nch) L *= 2;
    uint32_t lanes_log2 = 0;
    while ((1u << lanes_log2) < L) lanes_log2++;
    // Latency mode (one wave per row block of one row per lane group, all of
    // a lane's chunks loaded at once) when the matrices give at most 16384
    // such row blocks and a lane few chunks: 4 for one activation row (64-
    // weight chunks: 2; at 3 the 8B down_proj ran slower than the pipeline,
    // Q4_K 4096 x 12288 12.6 against 9.1 us), 2 for 2 and 8 rows (at 8 rows
    // the Qwen3-0.6B MLX step 853 -> 744 us per launch set, q/k/v 6.9 -> 5.5
    // us, down 8.1 -> 7.7; 2 chunks take ~300 registers there, so that kernel
    // runs in 256-thread workgroups only), 1 for 4 (64-weight
    // chunks: at most 2048 row blocks; 12288 x 4096 Q4_K 28.6 us against 17.7
    // us in the pipeline, 1024 x 4096 6.3 against 6.7 us).  64-weight chunks
    // at 2 rows: at most 4096 row blocks at 1 chunk per lane and 2048 at 2
    // (per launch, Q4_K/Q5_K/Q6_K 13824 x 5120: 30.4/32.1/32.0 us in latency
    // mode against 18.9/22.1/21.7 in the pipeline, 12288 x 4096 13.7 against
    // 11.5 us (Q4_K), 4096 x 5120 10.8 against 9.5; 1024 x 5120 6.6 against
    // 6.8, 4096 x 4096 6.8 either way).  More chunks or rows cost more in
    // registers, and waves per SIMD, than the latency saves (timed on the
    // config-1/4 steps).  Otherwise the persistent pipeline, whose rows per
    // lane group the encoding's launcher picks from the occupancy of each
    // instantiated tile.
    uint64_t rbs1 = 0;
    for (int i = 0; i < nprob; i++) rbs1 += (probs[i].n + (64u >> lanes_log2) - 1) / (64u >> lanes_log2);
    const uint32_t cpl = (nch + L - 1) >> lanes_log2;
    const uint32_t max_cpl = B == 1 ? (info.wide ? 2u : 4u) : B == 2 ? 2u : B == 4 ? 1u : B == 8 ? 2u : 0u;
    const uint64_t max_rbs = !info.wide || B == 1 ? 16384u : B == 4 ? 2048u : cpl == 1 ? 4096u : 2048u;
    const uint32_t oneshot = cpl >= 1 && cpl <= max_cpl && rbs1 <= max_rbs ? cpl : 0u;

    GemvParams p = {};
    for (int i = 0; i < kMaxProblems; i++) {
        const GemvProblem& q = probs[i < nprob ? i : nprob - 1];
        p.w[i] = q.w;
        p.sc[i] = q.sc;
        p.bi[i] = q.bi;
        p.y[i] = q.y;
        p.n[i] = i < nprob ? q.n : 0;
    }
    p.nprob = (uint32_t)nprob;
    p.x = x;
    p.K = K;
    p.ldx = K;
    p.ldy = 0;
    p.batch = batch;
    p.lanes_log2 = lanes_log2;
    p.y_bf16 = y_bf16 ? 1u : 0u;
    p.group = group;
    p.gmagic = group_magic(group);
    p.sdtype = sdtype;
    return launch(enc, p, B, oneshot, x_bf16, stream);  // lays out the row blocks per tile
}

}  // namespace dmx
