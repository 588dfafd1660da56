// Decode GEMV dispatch: lays out the wave grid over up to four weights that
// share one activation, picks the lanes-per-row split, and calls the
// per-encoding instantiations (gemv_<enc>.hip; kernels in gemv_kernels.hpp).
#include <mutex>
#include <vector>

#include "kernels.hpp"

namespace dmx {

hipError_t gemv_launch_q4_0(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q4_1(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q8_0(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st);
hipError_t gemv_launch_q6_k(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st);
hipError_t gemv_launch_mlx_u4(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st);

hipError_t cached_occupancy(const void* kernel, size_t lds, int* per_cu, int* cus) {
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
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, lds);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    cache.push_back({kernel, lds, dev, blocks, n});
    *per_cu = blocks;
    *cus = n;
    return hipSuccess;
}

namespace {

struct EncInfo {
    uint32_t chunk_weights;  // weights one lane handles per step
    uint32_t max_b;          // largest register batch instantiated
    bool super_block;        // Q6_K: 256-weight chunks hold fewer rows per lane
};

bool enc_info(uint32_t enc, EncInfo& e) {
    switch (enc) {
    case ENC_Q4_0: e = {32, 16, false}; return true;
    case ENC_Q4_1: e = {32, 16, false}; return true;
    case ENC_Q8_0: e = {32, 16, false}; return true;
    case ENC_Q6_K: e = {256, 8, true}; return true;
    case ENC_MLX_U4: e = {32, 16, false}; return true;
    default: return false;
    }
}

// Rows per lane group; must match rows_per_group<E, B>() in gemv_kernels.hpp.
uint32_t rows_per_group(const EncInfo& e, uint32_t B) {
    if (e.super_block) return 1;
    return B <= 2 ? 4 : (B <= 8 ? 2 : 1);
}

hipError_t launch(uint32_t enc, const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st) {
    switch (enc) {
    case ENC_Q4_0: return gemv_launch_q4_0(p, B, xbf16, st);
    case ENC_Q4_1: return gemv_launch_q4_1(p, B, xbf16, st);
    case ENC_Q8_0: return gemv_launch_q8_0(p, B, xbf16, st);
    case ENC_Q6_K: return gemv_launch_q6_k(p, B, xbf16, st);
    case ENC_MLX_U4: return gemv_launch_mlx_u4(p, B, xbf16, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t gemv_launch(uint32_t enc, const GemvProblem* probs, int nprob, uint32_t K, const void* x, bool x_bf16,
                       uint32_t batch, bool y_bf16, uint32_t group, uint32_t sdtype, hipStream_t stream) {
    EncInfo info;
    if (!enc_info(enc, info) || nprob < 1 || nprob > kMaxProblems || batch < 1 || batch > (uint32_t)kMaxGemvBatch)
        return hipErrorInvalidValue;
    // Batches larger than the widest instantiation run as consecutive passes.
    if (batch > info.max_b) {
        const size_t xes = x_bf16 ? 2 : 4, yes = y_bf16 ? 2 : 4;
        for (uint32_t r0 = 0; r0 < batch; r0 += info.max_b) {
            const uint32_t nb = batch - r0 < info.max_b ? batch - r0 : info.max_b;
            GemvProblem sub[kMaxProblems];
            for (int i = 0; i < nprob; i++) {
                sub[i] = probs[i];
                sub[i].y = static_cast<uint8_t*>(probs[i].y) + (size_t)r0 * probs[i].n * yes;
            }
            const void* xr = static_cast<const uint8_t*>(x) + (size_t)r0 * K * xes;
            hipError_t e = gemv_launch(enc, sub, nprob, K, xr, x_bf16, nb, y_bf16, group, sdtype, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    uint32_t B = 1;
    while (B < batch) B *= 2;
    const uint32_t R = rows_per_group(info, B);
    const uint32_t nch = K / info.chunk_weights;
    uint64_t nsum = 0;
    for (int i = 0; i < nprob; i++) nsum += probs[i].n;
    // Lanes per row group: a power of two dividing the chunk count (every lane
    // gets the same number of chunks per row block), the smallest that still
    // yields >= 4096 row blocks (4 waves per SIMD), at most 64.  Fewer lanes
    // per row mean longer per-lane chunk runs and fewer cross-lane reductions;
    // more lanes mean more waves for matrices with few rows.
    uint32_t lmax = 1;
    while (lmax < 64 && nch % (2 * lmax) == 0) lmax *= 2;
    uint32_t L = 1;
    auto rbs_for = [&](uint32_t l) { return nsum * l / (64ull * R); };
    while (L < lmax && rbs_for(L) < 4096) L *= 2;
    uint32_t lanes_log2 = 0;
    while ((1u << lanes_log2) < L) lanes_log2++;
    const uint32_t rows_per_rb = (64u >> lanes_log2) * R;

    GemvParams p = {};
    uint32_t rbs = 0;
    for (int i = 0; i < kMaxProblems; i++) {
        const GemvProblem& q = probs[i < nprob ? i : nprob - 1];
        p.w[i] = q.w;
        p.sc[i] = q.sc;
        p.bi[i] = q.bi;
        p.y[i] = q.y;
        p.n[i] = i < nprob ? q.n : 0;
        p.rb_begin[i] = rbs;
        if (i < nprob) rbs += (q.n + rows_per_rb - 1) / rows_per_rb;
    }
    p.total_rb = rbs;
    p.nprob = (uint32_t)nprob;
    p.x = x;
    p.K = K;
    p.ldx = K;
    p.ldy = 0;
    p.batch = batch;
    p.lanes_log2 = lanes_log2;
    p.y_bf16 = y_bf16 ? 1u : 0u;
    p.group = group;
    p.sdtype = sdtype;
    return launch(enc, p, B, x_bf16, stream);
}

}  // namespace dmx
