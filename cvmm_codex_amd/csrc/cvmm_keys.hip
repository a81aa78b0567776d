// Per-step cast of the expert weights to the MFMA operand type, in the two
// k-contiguous layouts the routed GEMM reads:
//   kt [E][d_out][d_in]  (forward: B rows are output columns, k = d_in)
//   kn [E][d_in][d_out]  (grad-input: B rows are input columns, k = d_out)
// or, for a dense top-k GEMM, with the experts interleaved between the rows
// ([d_out][E][d_in], [d_in][E][d_out]).
// One read of keys (any float storage, any strides), 64x64 tiles transposed
// through LDS so both writes are coalesced.  RNE, the same rounding as the
// in-register cast of the reference kernels (cvmm.py:198-204).
#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_keys.h"

namespace cvmm {

template <typename OutT>
__global__ __launch_bounds__(256) void cast_keys_kernel(const void* __restrict__ keys, int32_t keys_dtype,
                                                        int64_t se, int64_t si, int64_t sj, int64_t d_in,
                                                        int64_t d_out, OutT* __restrict__ kt,
                                                        OutT* __restrict__ kn, int64_t t_se, int64_t t_sr,
                                                        int64_t n_se, int64_t n_sr) {
  __shared__ float tile[64][65];
  const int64_t e = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * 64;   // d_in
  const int64_t j0 = (int64_t)blockIdx.x * 64;   // d_out
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  const int64_t base = e * se;
  for (int r = ty; r < 64; r += 4) {
    const int64_t i = i0 + r, j = j0 + tx;
    float v = 0.f;
    if (i < d_in && j < d_out) v = load_as_f32(keys, keys_dtype, base + i * si + j * sj);
    tile[r][tx] = v;
    if (kn != nullptr && i < d_in && j < d_out) kn[e * n_se + i * n_sr + j] = from_f32<OutT>(v);
  }
  if (kt == nullptr) return;
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t j = j0 + r, i = i0 + tx;
    if (i < d_in && j < d_out) kt[e * t_se + j * t_sr + i] = from_f32<OutT>(tile[tx][r]);
  }
}

// Vectorised fast path (see cast_block): one workgroup per block.
template <typename OutT>
__global__ __launch_bounds__(256) void cast_keys_vec_kernel(const CastArgs<OutT> a) {
  __shared__ float tile[kCastTileFloats];
  cast_block(a, (int64_t)blockIdx.x, tile);
}

hipError_t launch_cast_keys(const void* keys, int32_t keys_dtype, int64_t se, int64_t si, int64_t sj,
                            int32_t n_experts, int64_t d_in, int64_t d_out, int32_t out_dtype, void* kt,
                            void* kn, int32_t layout, hipStream_t stream) {
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0) return hipSuccess;
  if (n_experts > 65535 || (d_in + 63) / 64 > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)((d_out + 63) / 64), (unsigned)((d_in + 63) / 64), (unsigned)n_experts);
  if (cast_vec_ok(keys, keys_dtype, se, si, sj, d_in, d_out, out_dtype, kt, kn)) {
    const int64_t blocks = cast_blocks(n_experts, d_in, d_out);
    if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
    const dim3 vgrid((unsigned)blocks);
    if (out_dtype == kBF16)
      hipLaunchKernelGGL(cast_keys_vec_kernel<bf16_t>, vgrid, dim3(256), 0, stream,
                         make_cast_args<bf16_t>(keys, se, si, n_experts, d_in, d_out, kt, kn, layout));
    else
      hipLaunchKernelGGL(cast_keys_vec_kernel<f16_t>, vgrid, dim3(256), 0, stream,
                         make_cast_args<f16_t>(keys, se, si, n_experts, d_in, d_out, kt, kn, layout));
    return hipGetLastError();
  }
  const CastArgs<bf16_t> o = make_cast_args<bf16_t>(keys, se, si, n_experts, d_in, d_out, kt, kn, layout);
  if (out_dtype == kBF16) {
    hipLaunchKernelGGL(cast_keys_kernel<bf16_t>, grid, dim3(256), 0, stream, keys, keys_dtype, se, si, sj, d_in,
                       d_out, (bf16_t*)kt, (bf16_t*)kn, o.t_se, o.t_sr, o.n_se, o.n_sr);
  } else if (out_dtype == kF16) {
    hipLaunchKernelGGL(cast_keys_kernel<f16_t>, grid, dim3(256), 0, stream, keys, keys_dtype, se, si, sj, d_in,
                       d_out, (f16_t*)kt, (f16_t*)kn, o.t_se, o.t_sr, o.n_se, o.n_sr);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace cvmm
