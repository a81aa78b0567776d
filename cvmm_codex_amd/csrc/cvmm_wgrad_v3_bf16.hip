// Weight-gradient fast-path instantiations for op type bf16_t (see cvmm_wgrad_v3.h).
#include "cvmm_wgrad_v3.h"

namespace cvmm {
hipError_t launch_wgrad_v3_bf16(const WgradParams& p, hipStream_t stream) {
  return launch_wgrad_v3_op<bf16_t>(p, stream);
}
}  // namespace cvmm
