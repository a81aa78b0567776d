// Weight-gradient instantiations for op type float (see cvmm_wgrad_impl.h).
#include "cvmm_wgrad_impl.h"

namespace cvmm {
hipError_t launch_wgrad_f32(const WgradParams& p, hipStream_t stream) {
  return launch_wgrad_op<float>(p, stream);
}
}  // namespace cvmm
