// Decode GEMV instantiations for MLX affine U4 (kernel templates in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace dmx {
hipError_t gemv_launch_mlx_u4(const GemvParams& p, uint32_t B, bool xbf16, hipStream_t st) {
    return launch_mlx_gemv(p, B, xbf16, st);
}
}  // namespace dmx
