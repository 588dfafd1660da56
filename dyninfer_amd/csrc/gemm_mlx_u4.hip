// Prefill GEMM kernels of one encoding (compiled on their own, in parallel with the others).
#include "gemm_impl.hpp"

template hipError_t dmx::gemm::launch_plan<dmx::ENC_MLX_U4>(const GemmArgs&, const GemmPlan&, hipStream_t);
