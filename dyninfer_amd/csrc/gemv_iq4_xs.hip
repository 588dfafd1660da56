// Decode GEMV instantiations for GGUF IQ4_XS (kernel templates in gemv_kernels.hpp).
#include "gemv_stream.hpp"

namespace dmx {
hipError_t gemv_launch_iq4_xs(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st) {
    return launch_gguf_gemv<EncIQ4XS>(p, B, oneshot, xbf16, st);
}
}  // namespace dmx
