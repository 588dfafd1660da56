// Decode GEMV instantiations for MLX affine U4 (kernel templates in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace dmx {
namespace {
template <int XM>
hipError_t launch_mlx(const GemvParams& p, uint32_t B, uint32_t oneshot, hipStream_t st) {
    using E = EncMlxU4;
    const size_t lds = (size_t)xtile_bytes(E::ENC, B, p.K);
    if (oneshot) {
#define DMX_ONESHOT(b, c)                                                                                  \
    if (B == b && oneshot == c)                                                                            \
        return launch_oneshot(mlx_u4_gemv_oneshot_kernel<c, b, xmode_rows(XM, b), 512>,                      \
                              mlx_u4_gemv_oneshot_kernel<c, b, xmode_rows(XM, b), 256>, \
                              p, lds, st);
        DMX_ONESHOT(1, 1)
        DMX_ONESHOT(1, 2)
        DMX_ONESHOT(1, 3)
        DMX_ONESHOT(1, 4)
        DMX_ONESHOT(2, 1)
        DMX_ONESHOT(2, 2)
        DMX_ONESHOT(4, 1)
        DMX_ONESHOT(8, 1)
        // 8 rows of 2 chunks per lane take ~300 registers: 256-thread workgroups only
        if (B == 8 && oneshot == 2)
            return launch_oneshot<GemvKernel>(nullptr, mlx_u4_gemv_oneshot_kernel<2, 8, xmode_rows(XM, 8), 256>, p,
                                              lds, st);
#undef DMX_ONESHOT
        return hipErrorInvalidValue;
    }
    GemvTile t[kGemvMaxTiles];
    int n = 0;
#define DMX_CASE(b)                                                                                        \
    case b:                                                                                                \
        n = gemv_tiles<E, b>(t, [](auto r) -> GemvKernel { return mlx_u4_gemv_kernel<b, decltype(r)::value, xmode_rows(XM, b)>; }); \
        if constexpr (b > 1)                                                                               \
            n += gemv_tiles<E, b>(t + n, [](auto r) -> GemvKernel { return mlx_u4_gemv_kernel<b, decltype(r)::value, xmode_rows(XM, b), 256>; }, 256u); \
        break;
    switch (B) {
        DMX_CASE(1)
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
    default: break;
    }
#undef DMX_CASE
    if (n == 0) return hipErrorInvalidValue;
    const uint32_t nch = p.K / (uint32_t)E::CW;
    return launch_persistent_best(t, n, p, lds, (nch + (1u << p.lanes_log2) - 1u) >> p.lanes_log2, st);
}
}  // namespace

hipError_t gemv_launch_mlx_u4(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st) {
    switch (xmode<EncMlxU4>(xbf16, B, p.K)) {
    case XM_BF16: return launch_mlx<XM_BF16>(p, B, oneshot, st);
    case XM_F32_SPLIT: return launch_mlx<XM_F32_SPLIT>(p, B, oneshot, st);
    default: return launch_mlx<XM_F32>(p, B, oneshot, st);
    }
}
}  // namespace dmx
