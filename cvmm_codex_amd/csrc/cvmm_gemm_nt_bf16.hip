// Routed GEMM fast-path instantiations for op type bf16_t (cvmm_gemm_ring.h, cvmm_gemm_panel.h, cvmm_gemm_nt.h).
#include "cvmm_gemm_ring.h"

namespace cvmm {
hipError_t launch_routed_gemm_nt_bf16(const GemmParams& p, hipStream_t stream) {
  return launch_routed_gemm_fast_op<bf16_t>(p, stream);
}

// Whether the fast-path dispatch runs the ring kernel for these parameters
// (the only kernel with the activation epilogue); same rules for f16.
bool routed_gemm_ring_applies(const GemmParams& p, int32_t op) { return ring_eligible(p, op); }

bool routed_gemm_panel_applies(const GemmParams& p, int32_t op) { return panel_eligible(p, op); }
}  // namespace cvmm
