// Decode GEMV instantiations for GGUF Q5_K (kernel templates in gemv_kernels.hpp).
#include "gemv_stream.hpp"

namespace dmx {
hipError_t gemv_launch_q5_k(const GemvParams& p, uint32_t B, uint32_t oneshot, bool xbf16, hipStream_t st) {
    return launch_gguf_gemv<EncQ5K>(p, B, oneshot, xbf16, st);
}
}  // namespace dmx
