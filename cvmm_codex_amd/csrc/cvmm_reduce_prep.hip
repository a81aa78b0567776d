// Inputs of the reduce GEMM (cvmm_reduce.h), from the selector metadata:
//   a_sorted[q] = A row of sorted route q (op dtype), so that the routes of
//                 one expert and one token group are contiguous rows;
//   info[q]     = (output row = route / top_k, rounded routing weight);
//   lo[g][e]    = first sorted position of expert e whose output row is in
//                 token group g (g = G gives the end of the expert);
//   stages[g]   = the group's (expert, first position, count) stages of at
//                 most maxr routes, in expert order.
// The group bounds rely on the route index increasing within each expert
// (the stable sort's order), which the caller asserts.
#include <cmath>

#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

// One thread per 16-byte chunk of a gathered row; chunk 0 also writes the
// route's info.  Threads past R write the padding info entries.
__global__ __launch_bounds__(256) void reduce_gather_kernel(
    const void* __restrict__ a, int32_t a_dtype, int64_t a_ld, int64_t a_rows, const int64_t* __restrict__ a_idx,
    int64_t a_div, int32_t chunks, int32_t op_dtype, const int64_t* __restrict__ rp, int64_t top_k,
    const void* __restrict__ w, int32_t w_dtype, int32_t w_round, int64_t n_routes, int64_t n_tokens,
    uint4* __restrict__ a_sorted, RouteInfo* __restrict__ info) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t q = t / chunks;
  const int c = (int)(t - q * chunks);
  if (q >= n_routes) {
    const int64_t pq = q - n_routes;
    if (c == 0 && pq < kReducePad) info[n_routes + pq] = RouteInfo{-1, 0.f};
    return;
  }
  int64_t row = a_idx[q];
  row = row >= 0 ? row / a_div : -1;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row >= 0 && row < a_rows) {
    if (a_dtype == op_dtype) {
      v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a) + row * a_ld + c * 8);
    } else {  // fp32 storage: round to the op type
      const float* src = reinterpret_cast<const float*>(a) + row * a_ld + c * 8;
      Chunk16 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (op_dtype == kBF16) o.b[j] = (bf16_t)src[j];
        else o.h[j] = (f16_t)src[j];
      }
      v = o.u;
    }
  }
  a_sorted[q * chunks + c] = v;
  if (c == 0) {
    const int64_t r = rp[q];
    int32_t orow = -1;
    float wv = 0.f;
    if (r >= 0 && r < n_routes && r / top_k < n_tokens) {
      orow = (int32_t)(r / top_k);
      wv = w != nullptr ? round_to(load_as_f32(w, w_dtype, r), w_round) : 1.f;
    }
    info[q] = RouteInfo{orow, wv};
  }
}

// lo[g][e] = first q in expert e's segment with info[q].orow >= g * TG.
__global__ __launch_bounds__(256) void reduce_bounds_kernel(const RouteInfo* __restrict__ info,
                                                            const int64_t* __restrict__ offsets, int32_t n_experts,
                                                            int64_t n_routes, int32_t n_groups, int32_t group,
                                                            int32_t* __restrict__ lo) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)(n_groups + 1) * n_experts;
  if (t >= total) return;
  const int32_t g = (int32_t)(t / n_experts), e = (int32_t)(t % n_experts);
  int64_t start = e > 0 ? offsets[e - 1] : 0, end = offsets[e];
  start = start < 0 ? 0 : (start > n_routes ? n_routes : start);
  end = end < start ? start : (end > n_routes ? n_routes : end);
  const int64_t key = (int64_t)g * group;
  int64_t l = start, h = end;
  while (l < h) {
    const int64_t m = (l + h) >> 1;
    if ((int64_t)info[m].orow < key) l = m + 1;
    else h = m;
  }
  lo[t] = (int32_t)l;
}

// One workgroup per token group: the stage counts of its experts, an
// exclusive scan over the experts (in order), then the stage records.
__global__ __launch_bounds__(256) void reduce_stages_kernel(const int32_t* __restrict__ lo, int32_t n_experts,
                                                            int32_t maxr, ReduceStage* __restrict__ stages,
                                                            int32_t* __restrict__ n_stages) {
  __shared__ int32_t s_off[257];
  const int64_t g = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t E = n_experts;
  const int32_t per = (E + 255) / 256;  // experts tid*per .. +per-1 (in order)
  const int32_t e0 = tid * per, e1 = e0 + per < E ? e0 + per : E;
  int32_t mine = 0;
  for (int32_t e = e0; e < e1; ++e) {
    const int32_t n = lo[(g + 1) * E + e] - lo[g * E + e];
    mine += (n + maxr - 1) / maxr;
  }
  // inclusive scan of the counts (Hillis-Steele), shifted by one
  s_off[tid + 1] = mine;
  if (tid == 0) s_off[0] = 0;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {
    const int32_t add = tid >= d ? s_off[tid + 1 - d] : 0;
    __syncthreads();
    s_off[tid + 1] += add;
    __syncthreads();
  }
  int32_t k = s_off[tid];
  ReduceStage* out = stages + g * kReduceMaxStages;
  for (int32_t e = e0; e < e1; ++e) {
    const int32_t hi = lo[(g + 1) * E + e];
    for (int32_t r = lo[g * E + e]; r < hi; r += maxr, ++k)
      if (k < kReduceMaxStages) out[k] = ReduceStage{r, e * 256 + (hi - r < maxr ? hi - r : maxr)};
  }
  if (tid == 0) n_stages[g] = s_off[256] < kReduceMaxStages ? s_off[256] : kReduceMaxStages;
}

int32_t reduce_stage_routes(int64_t K, int64_t n_routes, int64_t n_groups, int32_t n_experts) {
  const double m = (double)n_routes / ((double)(n_groups > 0 ? n_groups : 1) * (n_experts > 0 ? n_experts : 1));
  const bool small = m + 3.0 * std::sqrt(m) <= 32.0;
  if (small) return 32;
  return K <= 64 ? 96 : 64;
}

hipError_t launch_reduce_prepare(const void* a, int32_t a_dtype, int64_t a_ld, int64_t a_rows, const int64_t* a_idx,
                                 int64_t a_div, int64_t K, int32_t op_dtype, const int64_t* rp, int64_t top_k,
                                 const void* w, int32_t w_dtype, int32_t w_round, const int64_t* offsets,
                                 int32_t n_experts, int64_t n_routes, int64_t n_tokens, int32_t group, int32_t maxr,
                                 void* a_sorted, RouteInfo* info, int32_t* lo, ReduceStage* stages,
                                 int32_t* n_stages, hipStream_t stream) {
  const int32_t chunks = (int32_t)(K / 8);
  const int64_t threads = (n_routes + kReducePad) * chunks;
  hipLaunchKernelGGL(reduce_gather_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a, a_dtype,
                     a_ld, a_rows, a_idx, a_div, chunks, op_dtype, rp, top_k, w, w_dtype, w_round, n_routes, n_tokens,
                     reinterpret_cast<uint4*>(a_sorted), info);
  const int32_t groups = (int32_t)((n_tokens + group - 1) / group);
  const int64_t total = (int64_t)(groups + 1) * n_experts;
  hipLaunchKernelGGL(reduce_bounds_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, info, offsets,
                     n_experts, n_routes, groups, group, lo);
  hipLaunchKernelGGL(reduce_stages_kernel, dim3((unsigned)groups), dim3(256), 0, stream, lo, n_experts, maxr, stages,
                     n_stages);
  return hipGetLastError();
}

hipError_t launch_routed_reduce(const ReduceParams& p, int32_t op_dtype, hipStream_t stream) {
  if (op_dtype == kBF16) return launch_routed_reduce_bf16(p, stream);
  if (op_dtype == kF16) return launch_routed_reduce_f16(p, stream);
  return hipErrorInvalidValue;
}

bool reduce_shape_ok(int32_t op_dtype, int64_t K, int64_t N, int32_t n_experts, int64_t n_routes, int64_t n_tokens,
                     int64_t top_k, int32_t out_dtype) {
  if (!((op_dtype == kBF16 || op_dtype == kF16) && (K == 64 || K == 128) && N > 0 && N % kReduceCols == 0 &&
        n_experts > 0 && n_tokens > 0 && top_k > 0 && n_routes + kReducePad < 0x7fffffffll &&
        (out_dtype == op_dtype || out_dtype == kF32) && (int64_t)n_experts * 256 < 0x7fffffffll))
    return false;
  const int64_t group = reduce_group_tokens(K);
  const int64_t groups = (n_tokens + group - 1) / group;
  const int64_t maxr = reduce_stage_routes(K, n_routes, groups, n_experts);
  return groups * (N / kReduceCols) <= 0x7fffffffll && (groups + 1) * n_experts <= 0x7fffffffll &&
         n_experts + (group * top_k + maxr - 1) / maxr <= kReduceMaxStages;
}

bool reduce_align_ok(const void* b, int64_t b_sk, int64_t b_se, int64_t b_sn, const void* out, int32_t out_dtype,
                     int64_t out_ld) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  return b_sk == 1 && a16(b) && (b_se * 2) % 16 == 0 && (b_sn * 2) % 16 == 0 && a16(out) &&
         (out_ld * (int64_t)dtype_size(out_dtype)) % 16 == 0;
}

}  // namespace cvmm
