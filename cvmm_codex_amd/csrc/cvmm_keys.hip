// Per-step cast of the expert weights to the MFMA operand type, in the two
// k-contiguous layouts the routed GEMM reads:
//   kt [E][d_out][d_in]  (forward: B rows are output columns, k = d_in)
//   kn [E][d_in][d_out]  (grad-input: B rows are input columns, k = d_out)
// One read of keys (any float storage, any strides), 64x64 tiles transposed
// through LDS so both writes are coalesced.  RNE, the same rounding as the
// in-register cast of the reference kernels (cvmm.py:198-204).
#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

template <typename OutT>
__global__ __launch_bounds__(256) void cast_keys_kernel(const void* __restrict__ keys, int32_t keys_dtype,
                                                        int64_t se, int64_t si, int64_t sj, int64_t d_in,
                                                        int64_t d_out, OutT* __restrict__ kt,
                                                        OutT* __restrict__ kn) {
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
    if (kn != nullptr && i < d_in && j < d_out) kn[(e * d_in + i) * d_out + j] = from_f32<OutT>(v);
  }
  if (kt == nullptr) return;
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t j = j0 + r, i = i0 + tx;
    if (i < d_in && j < d_out) kt[(e * d_out + j) * d_in + i] = from_f32<OutT>(tile[tx][r]);
  }
}

// Vectorised fast path: fp32 keys with unit column stride, 16-byte aligned
// rows, d_in and d_out multiples of 64.  A 64x64 tile is read as float4 rows
// (16 threads per 256-byte row), written to kn as 8-byte pieces of the same
// rows and, through a padded fp32 LDS tile, to kt as 16-byte pieces of its
// rows (8 consecutive d_in values per thread).
template <typename OutT>
__global__ __launch_bounds__(256) void cast_keys_vec_kernel(const float* __restrict__ keys, int64_t se, int64_t si,
                                                            int64_t d_in, int64_t d_out, OutT* __restrict__ kt,
                                                            OutT* __restrict__ kn) {
  __shared__ float tile[64][65];
  const int64_t e = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * 64;   // d_in
  const int64_t j0 = (int64_t)blockIdx.x * 64;   // d_out
  const int t = threadIdx.x;
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    const float4 v = *reinterpret_cast<const float4*>(keys + e * se + (i0 + r) * si + j0 + c4);
    tile[r][c4] = v.x;
    tile[r][c4 + 1] = v.y;
    tile[r][c4 + 2] = v.z;
    tile[r][c4 + 3] = v.w;
    if (kn != nullptr) {
      union { uint2 u; OutT h[4]; } pk;
      pk.h[0] = from_f32<OutT>(v.x);
      pk.h[1] = from_f32<OutT>(v.y);
      pk.h[2] = from_f32<OutT>(v.z);
      pk.h[3] = from_f32<OutT>(v.w);
      *reinterpret_cast<uint2*>(kn + (e * d_in + i0 + r) * d_out + j0 + c4) = pk.u;
    }
  }
  if (kt == nullptr) return;
  __syncthreads();
  const int i8 = (t & 7) * 8;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = (t >> 3) + 32 * q;
    union { uint4 u; OutT h[8]; } pk;
#pragma unroll
    for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(tile[i8 + k][j]);
    *reinterpret_cast<uint4*>(kt + (e * d_out + j0 + j) * d_in + i0 + i8) = pk.u;
  }
}

hipError_t launch_cast_keys(const void* keys, int32_t keys_dtype, int64_t se, int64_t si, int64_t sj,
                            int32_t n_experts, int64_t d_in, int64_t d_out, int32_t out_dtype, void* kt,
                            void* kn, hipStream_t stream) {
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0) return hipSuccess;
  if (n_experts > 65535 || (d_in + 63) / 64 > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)((d_out + 63) / 64), (unsigned)((d_in + 63) / 64), (unsigned)n_experts);
  const bool vec = keys_dtype == kF32 && sj == 1 && d_in % 64 == 0 && d_out % 64 == 0 && si % 4 == 0 &&
                   se % 4 == 0 && (reinterpret_cast<uintptr_t>(keys) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(kt) & 15) == 0 && (reinterpret_cast<uintptr_t>(kn) & 15) == 0;
  if (vec && (out_dtype == kBF16 || out_dtype == kF16)) {
    if (out_dtype == kBF16)
      hipLaunchKernelGGL(cast_keys_vec_kernel<bf16_t>, grid, dim3(256), 0, stream, (const float*)keys, se, si, d_in,
                         d_out, (bf16_t*)kt, (bf16_t*)kn);
    else
      hipLaunchKernelGGL(cast_keys_vec_kernel<f16_t>, grid, dim3(256), 0, stream, (const float*)keys, se, si, d_in,
                         d_out, (f16_t*)kt, (f16_t*)kn);
    return hipGetLastError();
  }
  if (out_dtype == kBF16) {
    hipLaunchKernelGGL(cast_keys_kernel<bf16_t>, grid, dim3(256), 0, stream, keys, keys_dtype, se, si, sj, d_in,
                       d_out, (bf16_t*)kt, (bf16_t*)kn);
  } else if (out_dtype == kF16) {
    hipLaunchKernelGGL(cast_keys_kernel<f16_t>, grid, dim3(256), 0, stream, keys, keys_dtype, se, si, sj, d_in,
                       d_out, (f16_t*)kt, (f16_t*)kn);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace cvmm
