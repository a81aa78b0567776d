// Reduce GEMM instantiations for op type bf16_t (see cvmm_reduce.h).
#include "cvmm_reduce.h"

namespace cvmm {
hipError_t launch_routed_reduce_bf16(const ReduceParams& p, hipStream_t stream) {
  return launch_routed_reduce_op<bf16_t>(p, stream);
}
}  // namespace cvmm
