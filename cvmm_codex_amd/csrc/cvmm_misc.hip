// Small bandwidth kernels around the routed GEMMs: zero fill (used instead of
// hipMemsetAsync so a captured graph holds only kernel nodes), the top-k row
// combine of a route-ordered buffer, fp32 -> storage casts and the ordered
// sum of per-tile routing-weight gradient partials.
#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

// head: bytes before the first 16-byte boundary; body: 16-byte stores; tail.
__global__ void fill_zero_kernel(uint8_t* __restrict__ head, int64_t n_head, uint4* __restrict__ body, int64_t n16,
                                 uint8_t* __restrict__ tail, int64_t n_tail) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) body[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < n_head) head[threadIdx.x] = 0;
  if (blockIdx.x == 0 && threadIdx.x < n_tail) tail[threadIdx.x] = 0;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  uint8_t* b = static_cast<uint8_t*>(p);
  int64_t n_head = (int64_t)((16 - (reinterpret_cast<uintptr_t>(b) & 15)) & 15);
  if ((size_t)n_head > bytes) n_head = (int64_t)bytes;
  const int64_t rest = (int64_t)bytes - n_head;
  const int64_t n16 = rest / 16;
  const int64_t n_tail = rest % 16;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, b, n_head,
                     reinterpret_cast<uint4*>(b + n_head), n16, b + n_head + n16 * 16, n_tail);
  return hipGetLastError();
}

// out[t][n] = rnd(rnd(sum_j w_j * buf[t*k + j][n], mid), out)   (j in route order)
__global__ void combine_rows_kernel(const void* __restrict__ buf, int32_t buf_dtype, int64_t buf_ld,
                                    const void* __restrict__ w, int32_t w_dtype, int32_t w_round, int64_t k,
                                    int64_t n, int32_t mid_dtype, void* __restrict__ out, int32_t out_dtype,
                                    int64_t out_ld) {
  const int64_t t = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * blockDim.x + threadIdx.x;
  if (col >= n) return;
  float s = 0.f;
  for (int64_t j = 0; j < k; ++j) {
    const int64_t r = t * k + j;
    float v = load_as_f32(buf, buf_dtype, r * buf_ld + col);
    if (w != nullptr) v *= round_to(load_as_f32(w, w_dtype, r), w_round);
    s += v;
  }
  if (mid_dtype >= 0) s = round_to(s, mid_dtype);
  store_from_f32(out, out_dtype, t * out_ld + col, s);
}

hipError_t launch_combine_rows(const void* buf, int32_t buf_dtype, int64_t buf_ld, const void* w, int32_t w_dtype,
                               int32_t w_round, int64_t n_tokens, int64_t k, int64_t n, int32_t mid_dtype,
                               void* out, int32_t out_dtype, int64_t out_ld, hipStream_t stream) {
  if (n_tokens <= 0 || n <= 0) return hipSuccess;
  if (n_tokens > 0x7fffffffll) return hipErrorInvalidValue;
  if ((n + 255) / 256 > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)n_tokens, (unsigned)((n + 255) / 256));
  hipLaunchKernelGGL(combine_rows_kernel, grid, dim3(256), 0, stream, buf, buf_dtype, buf_ld, w, w_dtype, w_round,
                     k, n, mid_dtype, out, out_dtype, out_ld);
  return hipGetLastError();
}

__global__ void cast_rows_kernel(const float* __restrict__ acc, int64_t acc_ld, int64_t n, int32_t mid_dtype,
                                 void* __restrict__ out, int32_t out_dtype, int64_t out_ld) {
  const int64_t t = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * blockDim.x + threadIdx.x;
  if (col >= n) return;
  float v = acc[t * acc_ld + col];
  if (mid_dtype >= 0) v = round_to(v, mid_dtype);
  store_from_f32(out, out_dtype, t * out_ld + col, v);
}

hipError_t launch_cast_rows(const float* acc, int64_t acc_ld, int64_t rows, int64_t n, int32_t mid_dtype,
                            void* out, int32_t out_dtype, int64_t out_ld, hipStream_t stream) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  if (rows > 0x7fffffffll) return hipErrorInvalidValue;
  if ((n + 255) / 256 > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)rows, (unsigned)((n + 255) / 256));
  hipLaunchKernelGGL(cast_rows_kernel, grid, dim3(256), 0, stream, acc, acc_ld, n, mid_dtype, out, out_dtype, out_ld);
  return hipGetLastError();
}

__global__ void sum_partials_kernel(const float* __restrict__ part, int64_t rows, int32_t ntiles,
                                    void* __restrict__ out, int32_t out_dtype) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = 0.f;
  for (int32_t t = 0; t < ntiles; ++t) s += part[r * ntiles + t];
  store_from_f32(out, out_dtype, r, s);
}

hipError_t launch_sum_partials(const float* part, int64_t rows, int32_t ntiles, void* out, int32_t out_dtype,
                               hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int64_t blocks = (rows + 255) / 256;
  hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, part, rows, ntiles, out,
                     out_dtype);
  return hipGetLastError();
}

}  // namespace cvmm
