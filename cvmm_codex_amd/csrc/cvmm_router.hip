// Router: the step before the path in the reference's MoE callers
// (benchmark_ffn_moe.py:91-97, benchmark_framework_moe.py:129-135):
//   probs = softmax(logits.float()); weights, sel = probs.topk(k)
//   weights = weights / weights.sum(-1).clamp_min(1e-20)     (optional)
//   sel_up = cvmm_prepare_sel2(sel)                            (cvmm.py:1786-1803)
// in two launches: a segment of 4..64 lanes per token computes the softmax in
// registers, picks the top k (descending probability, ties to the lower
// expert id, NaN ranked lowest) with segment reductions and renormalises;
// each workgroup owns the tokens of one sort chunk and leaves that chunk's
// expert histogram, so the second launch is the stable scatter of
// cvmm_sort_routes.  The backward recomputes the softmax and returns the
// logits' gradient.
#include <cmath>

#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

constexpr int kRouteThreads = 256;
constexpr int kRouteHistThreads = 512;  // two waves per SIMD: the selection rounds are latency-bound

// Segments of LPT lanes (4..64) each route one token: lane i of a segment
// holds experts i + LPT * v, v < MAXV.  Reductions over a segment use DPP
// (quad permutes, half-row and row mirrors) and, past 16 lanes, shuffles; every
// lane of the segment ends with the same result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int LPT>
__device__ __forceinline__ float seg_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  if constexpr (LPT >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  if constexpr (LPT >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
  if constexpr (LPT >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if constexpr (LPT >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}
template <int LPT>
__device__ __forceinline__ float seg_sum(float v) {  // same two partials per step: same total in every lane
  v = v + dpp_f<kDppXor1>(v);
  v = v + dpp_f<kDppXor2>(v);
  if constexpr (LPT >= 8) v = v + dpp_f<kDppHalfMirror>(v);
  if constexpr (LPT >= 16) v = v + dpp_f<kDppMirror>(v);
  if constexpr (LPT >= 32) v = v + __shfl_xor(v, 16, 64);
  if constexpr (LPT >= 64) v = v + __shfl_xor(v, 32, 64);
  return v;
}
template <int LPT>
__device__ __forceinline__ int32_t seg_min_i(int32_t v) {
  v = min(v, dpp_i<kDppXor1>(v));
  v = min(v, dpp_i<kDppXor2>(v));
  if constexpr (LPT >= 8) v = min(v, dpp_i<kDppHalfMirror>(v));
  if constexpr (LPT >= 16) v = min(v, dpp_i<kDppMirror>(v));
  if constexpr (LPT >= 32) v = min(v, __shfl_xor(v, 16, 64));
  if constexpr (LPT >= 64) v = min(v, __shfl_xor(v, 32, 64));
  return v;
}

// Softmax of one token's logits in its segment.
template <typename LT, int LPT, int MAXV>
__device__ __forceinline__ void route_softmax(const LT* __restrict__ row, int32_t E, int li, bool active,
                                              float (&p)[MAXV], float* m_out, float* s_out) {
  float m = -INFINITY;
#pragma unroll
  for (int v = 0; v < MAXV; ++v) {
    const int e = li + LPT * v;
    p[v] = active && e < E ? (float)row[e] : -INFINITY;
    m = fmaxf(m, p[v]);
  }
  m = seg_max<LPT>(m);
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < MAXV; ++v) {
    const int e = li + LPT * v;
    p[v] = active && e < E ? expf(p[v] - m) : 0.f;
    s += p[v];
  }
  s = seg_sum<LPT>(s);
#pragma unroll
  for (int v = 0; v < MAXV; ++v) p[v] = p[v] / s;
  *m_out = m;
  *s_out = s;
}

template <typename LT, int LPT, int MAXV>
__global__ __launch_bounds__(kRouteHistThreads) void route_topk_hist_kernel(
    const LT* __restrict__ logits, int64_t ld, int64_t n_tokens, int32_t E, int32_t k, int32_t renorm, int64_t tpc,
    float* __restrict__ weights, int64_t* __restrict__ sel, int32_t* __restrict__ counts) {
  constexpr int SEGS = kRouteHistThreads / LPT;  // tokens per workgroup pass
  constexpr int SLOTS = 64 / LPT;            // results j held by lane j % LPT, slot j / LPT
  extern __shared__ int32_t hist[];          // E + 1 (bucket E: invalid ids, none here)
  const int64_t b = blockIdx.x;
  for (int e = threadIdx.x; e <= E; e += kRouteHistThreads) hist[e] = 0;
  __syncthreads();
  const int li = threadIdx.x % LPT, seg = threadIdx.x / LPT;
  const int64_t t_lo = b * tpc, t_hi = t_lo + tpc < n_tokens ? t_lo + tpc : n_tokens;
  // every lane runs every pass (segment reductions need the whole wave)
  for (int64_t t0 = t_lo; t0 < t_hi; t0 += SEGS) {
    const int64_t t = t0 + seg;
    const bool active = t < t_hi;
    float p[MAXV], m, s;
    route_softmax<LT, LPT, MAXV>(logits + (active ? t : t_lo) * ld, E, li, active, p, &m, &s);
    uint32_t taken = 0;
    float res_w[SLOTS];
    int32_t res_e[SLOTS];
#pragma unroll
    for (int q = 0; q < SLOTS; ++q) {
      res_w[q] = 0.f;
      res_e[q] = 0;
    }
    for (int j = 0; j < k; ++j) {
      // best untaken expert: probability descending (NaN as -inf), ties to
      // the lower id -- the lane's own, then the segment's
      float bv = -INFINITY, pv = 0.f;
      int32_t bi = E;
#pragma unroll
      for (int v = 0; v < MAXV; ++v) {
        const int e = li + LPT * v;
        const float key = isnan(p[v]) ? -INFINITY : p[v];
        if (e < E && !((taken >> v) & 1u) && (key > bv || (key == bv && e < bi))) {
          bv = key;
          bi = e;
          pv = p[v];
        }
      }
      const float mv = seg_max<LPT>(bv);
      const int32_t win = seg_min_i<LPT>(bv == mv ? bi : E);
      const bool mine = win == bi;  // the lane holding the winner
      if (mine) taken |= 1u << (win / LPT);
      const float pw = seg_sum<LPT>(mine ? pv : 0.f);  // the winner's probability (NaN kept)
#pragma unroll
      for (int q = 0; q < SLOTS; ++q)
        if (j == q * LPT + li) {
          res_w[q] = pw;
          res_e[q] = win;
        }
    }
    if (renorm) {
      float part = 0.f;
#pragma unroll
      for (int q = 0; q < SLOTS; ++q)
        if (q * LPT + li < k) part += res_w[q];
      float den = seg_sum<LPT>(part);
      den = den < 1e-20f ? 1e-20f : den;  // clamp_min (NaN passes through)
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) res_w[q] = res_w[q] / den;
    }
    if (active) {
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) {
        const int j = q * LPT + li;
        if (j < k) {
          sel[t * k + j] = res_e[q];
          weights[t * k + j] = res_w[q];
          atomicAdd(&hist[res_e[q]], 1);
        }
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kRouteHistThreads) counts[b * (int64_t)(E + 1) + e] = hist[e];
}

// d logits: with g = d loss / d probs (non-zero at the chosen experts),
// d l_e = p_e (g_e - sum_i g_i p_i); renormalised weights w_j = p_j / S give
// g_j = (dw_j - sum_i dw_i w_i) / S (S clamped: a constant).
template <typename LT, int LPT, int MAXV>
__global__ __launch_bounds__(kRouteThreads) void route_topk_bwd_kernel(
    const LT* __restrict__ logits, int64_t ld, int64_t n_tokens, int32_t E, int32_t k, int32_t renorm,
    const int64_t* __restrict__ sel, const float* __restrict__ gw, LT* __restrict__ glog, int64_t gld) {
  constexpr int SEGS = kRouteThreads / LPT;
  constexpr int SLOTS = 64 / LPT;
  __shared__ float g_lds[SEGS * LPT * MAXV];  // per segment: g of every expert
  const int li = threadIdx.x % LPT, seg = threadIdx.x / LPT;
  const int64_t t = (int64_t)blockIdx.x * SEGS + seg;
  const bool active = t < n_tokens;
  const LT* row = logits + (active ? t : 0) * ld;
  float p[MAXV], m, s;
  route_softmax<LT, LPT, MAXV>(row, E, li, active, p, &m, &s);
  float* gseg = g_lds + seg * LPT * MAXV;
#pragma unroll
  for (int v = 0; v < MAXV; ++v) gseg[li + LPT * v] = 0.f;
  int32_t sj[SLOTS];
  float pj[SLOTS], dwj[SLOTS];
  float ps = 0.f;
#pragma unroll
  for (int q = 0; q < SLOTS; ++q) {
    const int j = q * LPT + li;
    sj[q] = -1;
    pj[q] = dwj[q] = 0.f;
    if (active && j < k) {
      const int64_t id = sel[t * k + j];
      if (id >= 0 && id < E) {
        sj[q] = (int32_t)id;
        pj[q] = expf((float)row[id] - m) / s;  // the forward's value
        dwj[q] = gw[t * k + j];
      }
    }
    ps += pj[q];
  }
  float gj[SLOTS];
#pragma unroll
  for (int q = 0; q < SLOTS; ++q) gj[q] = dwj[q];
  if (renorm) {
    const float S = seg_sum<LPT>(ps);
    if (S < 1e-20f) {
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) gj[q] = dwj[q] / 1e-20f;
    } else {
      float d = 0.f;
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) d += dwj[q] * (pj[q] / S);
      const float dot = seg_sum<LPT>(d);
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) gj[q] = (dwj[q] - dot) / S;
    }
  }
  float cp = 0.f;
#pragma unroll
  for (int q = 0; q < SLOTS; ++q) cp += gj[q] * pj[q];
  const float c = seg_sum<LPT>(cp);
  __syncthreads();  // zeroed g visible
#pragma unroll
  for (int q = 0; q < SLOTS; ++q)
    if (sj[q] >= 0) gseg[sj[q]] = gj[q];
  __syncthreads();
  if (!active) return;
  LT* out = glog + t * gld;
#pragma unroll
  for (int v = 0; v < MAXV; ++v) {
    const int e = li + LPT * v;
    if (e < E) out[e] = (LT)(p[v] * (gseg[e] - c));
  }
}

// Whole tokens per chunk, at least 512 routes and enough routes that the
// count matrix stays within 64K entries: half the plain sort's minimum chunk,
// so the router has more workgroups while the count matrix every scatter
// workgroup reads stays small.
int64_t route_chunk_tokens(int64_t n_tokens, int32_t n_experts, int64_t top_k) {
  const int64_t R = n_tokens * top_k;
  int64_t routes = (R * (int64_t)(n_experts + 1) + 65535) / 65536;
  if (routes < 512) routes = 512;
  return (routes + top_k - 1) / top_k;
}

size_t route_workspace_bytes(int64_t n_tokens, int32_t n_experts, int64_t top_k) {
  const int64_t tpc = route_chunk_tokens(n_tokens, n_experts, top_k);
  const int64_t n_chunks = n_tokens > 0 ? (n_tokens + tpc - 1) / tpc : 1;
  // counts, bucket totals for the column scan, 256 bytes ending in n_invalid
  return sort_counts_bytes(n_chunks, n_experts) + align_up((size_t)(n_experts + 1) * sizeof(int32_t), 256) + 256;
}

template <typename LT, int LPT, int MAXV>
static void launch_hist(const void* logits, int64_t ld, int64_t T, int32_t E, int32_t k, int32_t renorm, int64_t tpc,
                        int64_t n_chunks, float* w, int64_t* sel, int32_t* counts, hipStream_t s) {
  hipLaunchKernelGGL((route_topk_hist_kernel<LT, LPT, MAXV>), dim3((unsigned)n_chunks), dim3(kRouteHistThreads),
                     (size_t)(E + 1) * sizeof(int32_t), s, (const LT*)logits, ld, T, E, k, renorm, tpc, w, sel,
                     counts);
}

// Segment width: 8 experts per lane up to 512 experts, then 16.
template <typename LT>
static void launch_hist_v(const void* logits, int64_t ld, int64_t T, int32_t E, int32_t k, int32_t renorm,
                          int64_t tpc, int64_t n_chunks, float* w, int64_t* sel, int32_t* counts, hipStream_t s) {
  if (E <= 32) launch_hist<LT, 4, 8>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
  else if (E <= 64) launch_hist<LT, 8, 8>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
  else if (E <= 128) launch_hist<LT, 16, 8>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
  else if (E <= 256) launch_hist<LT, 32, 8>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
  else if (E <= 512) launch_hist<LT, 64, 8>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
  else launch_hist<LT, 64, 16>(logits, ld, T, E, k, renorm, tpc, n_chunks, w, sel, counts, s);
}

hipError_t launch_route_topk(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                             int32_t n_experts, int64_t top_k, int32_t renormalize, float* weights, int64_t* sel,
                             int32_t* sorted_sel, int64_t* perm, int64_t* token_index, int64_t* offsets,
                             int32_t* route_pos, void* workspace, hipStream_t stream) {
  if (n_tokens <= 0) return hipSuccess;
  const int64_t tpc = route_chunk_tokens(n_tokens, n_experts, top_k);
  const int64_t n_chunks = (n_tokens + tpc - 1) / tpc;
  if (n_chunks > 0x7fffffffll) return hipErrorInvalidValue;
  int32_t* counts = (int32_t*)workspace;
  int32_t* n_invalid = (int32_t*)((char*)workspace + route_workspace_bytes(n_tokens, n_experts, top_k) - 256);
  const int32_t k = (int32_t)top_k;
  if (logits_dtype == kF32)
    launch_hist_v<float>(logits, logits_ld, n_tokens, n_experts, k, renormalize, tpc, n_chunks, weights, sel, counts,
                         stream);
  else if (logits_dtype == kBF16)
    launch_hist_v<bf16_t>(logits, logits_ld, n_tokens, n_experts, k, renormalize, tpc, n_chunks, weights, sel, counts,
                          stream);
  else
    launch_hist_v<f16_t>(logits, logits_ld, n_tokens, n_experts, k, renormalize, tpc, n_chunks, weights, sel, counts,
                         stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_sort_scatter(sel, n_tokens * top_k, n_experts, tpc * top_k, top_k, counts, sorted_sel, perm,
                             token_index, offsets, route_pos, n_invalid, stream);
}

template <typename LT, int LPT, int MAXV>
static void launch_bwd(const void* logits, int64_t ld, int64_t T, int32_t E, int32_t k, int32_t renorm,
                       const int64_t* sel, const float* gw, void* glog, int64_t gld, hipStream_t s) {
  constexpr int SEGS = kRouteThreads / LPT;
  const int64_t grid = (T + SEGS - 1) / SEGS;
  hipLaunchKernelGGL((route_topk_bwd_kernel<LT, LPT, MAXV>), dim3((unsigned)grid), dim3(kRouteThreads), 0, s,
                     (const LT*)logits, ld, T, E, k, renorm, sel, gw, (LT*)glog, gld);
}

template <typename LT>
static void launch_bwd_v(const void* logits, int64_t ld, int64_t T, int32_t E, int32_t k, int32_t renorm,
                         const int64_t* sel, const float* gw, void* glog, int64_t gld, hipStream_t s) {
  if (E <= 32) launch_bwd<LT, 4, 8>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
  else if (E <= 64) launch_bwd<LT, 8, 8>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
  else if (E <= 128) launch_bwd<LT, 16, 8>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
  else if (E <= 256) launch_bwd<LT, 32, 8>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
  else if (E <= 512) launch_bwd<LT, 64, 8>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
  else launch_bwd<LT, 64, 16>(logits, ld, T, E, k, renorm, sel, gw, glog, gld, s);
}

hipError_t launch_route_topk_backward(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                                      int32_t n_experts, int64_t top_k, int32_t renormalize, const int64_t* sel,
                                      const float* grad_weights, void* grad_logits, int64_t grad_ld,
                                      hipStream_t stream) {
  if (n_tokens <= 0) return hipSuccess;
  if (n_tokens / 4 > 0x7fffffffll) return hipErrorInvalidValue;
  const int32_t k = (int32_t)top_k;
  if (logits_dtype == kF32)
    launch_bwd_v<float>(logits, logits_ld, n_tokens, n_experts, k, renormalize, sel, grad_weights, grad_logits,
                        grad_ld, stream);
  else if (logits_dtype == kBF16)
    launch_bwd_v<bf16_t>(logits, logits_ld, n_tokens, n_experts, k, renormalize, sel, grad_weights, grad_logits,
                         grad_ld, stream);
  else
    launch_bwd_v<f16_t>(logits, logits_ld, n_tokens, n_experts, k, renormalize, sel, grad_weights, grad_logits,
                        grad_ld, stream);
  return hipGetLastError();
}

}  // namespace cvmm
