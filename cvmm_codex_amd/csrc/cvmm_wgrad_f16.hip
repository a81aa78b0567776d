// Weight-gradient instantiations for op type f16_t (see cvmm_wgrad_impl.h).
#include "cvmm_wgrad_impl.h"

namespace cvmm {
hipError_t launch_wgrad_f16(const WgradParams& p, hipStream_t stream) {
  return launch_wgrad_op<f16_t>(p, stream);
}
}  // namespace cvmm
