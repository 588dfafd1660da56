// Decode GEMV instantiations for MLX affine U4 (kernel templates in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace dmx {
hipError_t gemv_launch_mlx_u4(const GemvParams& p, uint32_t B, uint32_t R, uint32_t oneshot, bool xbf16, hipStream_t st) {
    using E = EncMlxU4;
    const size_t lds = (size_t)xtile_bytes(E::ENC, B, p.K);
    if (oneshot) {
        if (R != 1) return hipErrorInvalidValue;
#define DMX_ONESHOT(b, c)                                                                                 \
    if (B == b && oneshot == c)                                                                           \
        return xbf16 ? launch_oneshot(mlx_u4_gemv_oneshot_kernel<c, b, true>, p, lds, st)                \
                     : launch_oneshot(mlx_u4_gemv_oneshot_kernel<c, b, false>, p, lds, st);
        DMX_ONESHOT(1, 1)
        DMX_ONESHOT(1, 2)
        DMX_ONESHOT(1, 3)
        DMX_ONESHOT(1, 4)
        DMX_ONESHOT(2, 1)
        DMX_ONESHOT(2, 2)
        DMX_ONESHOT(4, 1)
#undef DMX_ONESHOT
        return hipErrorInvalidValue;
    }
    if (B == 1 && R == 1)
        return xbf16 ? launch_persistent(mlx_u4_gemv_kernel<1, 1, true>, p, lds, st)
                     : launch_persistent(mlx_u4_gemv_kernel<1, 1, false>, p, lds, st);
#define DMX_CASE(b)                                                                                        \
    case b:                                                                                                \
        if (R == (uint32_t)rows_per_group<E, b>())                                                         \
            return xbf16 ? launch_persistent(mlx_u4_gemv_kernel<b, rows_per_group<E, b>(), true>, p, lds, st)  \
                         : launch_persistent(mlx_u4_gemv_kernel<b, rows_per_group<E, b>(), false>, p, lds, st); \
        if constexpr (b > 1)                                                                               \
            if (R == (uint32_t)rows_per_group_narrow<E, b>())                                              \
            return xbf16 ? launch_persistent(mlx_u4_gemv_kernel<b, rows_per_group_narrow<E, b>(), true>, p, lds, \
                                             st)                                                           \
                         : launch_persistent(mlx_u4_gemv_kernel<b, rows_per_group_narrow<E, b>(), false>, p, lds, \
                                             st);                                                          \
        return hipErrorInvalidValue;
    switch (B) {
        DMX_CASE(1)
        DMX_CASE(2)
        DMX_CASE(4)
        DMX_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef DMX_CASE
}
}  // namespace dmx
