// Routed GEMM instantiations for op type float (see cvmm_gemm_impl.h).
#include "cvmm_gemm_impl.h"

namespace cvmm {
hipError_t launch_routed_gemm_f32(const GemmParams& p, hipStream_t stream) {
  return launch_routed_gemm_op<float>(p, stream);
}
}  // namespace cvmm
