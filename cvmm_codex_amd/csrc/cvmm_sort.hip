// Selector preparation: stable counting sort of routes by expert.
//
// Replaces the ATen sort of cvmm_prepare_sel / cvmm_prepare_sel2
// (cvmm.py:24-27, cvmm.py:1796-1803) and the offsets binary search
// (cvmm_expert_offsets_kernel, cvmm.py:315-335).
//
// Three launches over chunks of kSortChunk routes:
//   1. histogram   counts[bucket][chunk]      (LDS atomics, bucket E = invalid id)
//   2. scan        exclusive prefix over the bucket-major counts, and the
//                  inclusive per-expert offsets the GEMM schedulers read
//   3. scatter     each chunk walks its routes in index order; a route's rank
//                  among equal keys of its wave comes from ballots over the key
//                  bits, waves of a workgroup take turns, so the order is
//                  stable (equal experts keep route order).
#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

constexpr int kSortThreads = 256;

template <typename IdxT>
__device__ __forceinline__ int32_t bucket_of(IdxT raw, int32_t n_experts) {
  const int32_t key = (int32_t)raw;  // int64 ids wrap like the int32 conversion of cvmm.py:1797
  return (key < 0 || key >= n_experts) ? n_experts : key;
}

template <typename IdxT>
__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(
    const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
    int64_t n_chunks, int32_t* __restrict__ counts) {
  extern __shared__ int32_t hist[];  // n_experts + 1
  const int64_t b = blockIdx.x;
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) hist[e] = 0;
  __syncthreads();
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  for (int64_t i = lo + threadIdx.x; i < hi; i += kSortThreads) {
    atomicAdd(&hist[bucket_of(sel[i], n_experts)], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) counts[(int64_t)e * n_chunks + b] = hist[e];
}

// Single workgroup: exclusive scan of `total` = (E+1)*n_chunks counts in place.
// offsets[e] = #routes whose bucket <= e (the reference's inclusive cumsum).
constexpr int kScanThreads = 1024;
__global__ __launch_bounds__(kScanThreads) void sort_scan_kernel(
    int32_t* __restrict__ counts, int64_t n_chunks, int32_t n_experts, int64_t* __restrict__ offsets,
    int32_t* __restrict__ n_invalid, int64_t n_routes) {
  __shared__ int64_t part[kScanThreads];
  const int64_t total = (int64_t)(n_experts + 1) * n_chunks;
  const int64_t per = (total + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min((int64_t)threadIdx.x * per, total);
  const int64_t hi = min(lo + per, total);
  int64_t s = 0;
  for (int64_t j = lo; j < hi; ++j) s += counts[j];
  part[threadIdx.x] = s;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 1024 partial sums.
  for (int d = 1; d < kScanThreads; d <<= 1) {
    int64_t v = threadIdx.x >= d ? part[threadIdx.x - d] : 0;
    __syncthreads();
    part[threadIdx.x] += v;
    __syncthreads();
  }
  int64_t run = part[threadIdx.x] - s;  // exclusive prefix of this segment
  for (int64_t j = lo; j < hi; ++j) {
    const int32_t c = counts[j];
    // bucket boundary: j == (e+1)*n_chunks marks the end of expert e
    if (j % n_chunks == 0 && j > 0) {
      const int64_t e = j / n_chunks - 1;
      if (e < n_experts) offsets[e] = run;
      // the invalid bucket E starts after expert E-1: everything past it is invalid
      if (e == n_experts - 1 && n_invalid != nullptr) *n_invalid = (int32_t)(n_routes - run);
    }
    counts[j] = (int32_t)run;
    run += c;
  }
}

// Stable scatter of one chunk: within every 256-route round, lanes with equal
// buckets are ranked by a ballot per bucket bit and the waves take their
// positions in order, so equal ids keep their input order.  `pos` holds this
// chunk's next output position per bucket.
template <typename IdxT>
__device__ void scatter_chunk(const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
                              int32_t n_bits, int64_t top_k, int32_t* pos, int32_t* __restrict__ sorted_sel,
                              int64_t* __restrict__ perm, int64_t* __restrict__ token_index,
                              int32_t* __restrict__ route_pos) {
  const int64_t b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  for (int64_t base = lo; base < hi; base += kSortThreads) {
    const int64_t i = base + threadIdx.x;
    const bool valid = i < hi;
    const IdxT key = valid ? sel[i] : (IdxT)0;
    const int32_t bucket = valid ? bucket_of(key, n_experts) : 0;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < n_bits; ++bit) {
      const bool set = (bucket >> bit) & 1;
      const uint64_t bb = __ballot(set);
      peers &= set ? bb : ~bb;
    }
    const int rank = __popcll(peers & lt_mask);
    const int cnt = __popcll(peers);
    for (int w = 0; w < kSortThreads / 64; ++w) {
      if (wave == w && valid) {
        const int32_t p0 = pos[bucket];
        const int64_t p = (int64_t)p0 + rank;
        if (rank == 0) pos[bucket] = p0 + cnt;
        sorted_sel[p] = (int32_t)key;
        perm[p] = i;
        if (token_index != nullptr) token_index[p] = i / top_k;
        if (route_pos != nullptr) route_pos[i] = (int32_t)p;
      }
      __syncthreads();
    }
  }
}

template <typename IdxT>
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
    int64_t n_chunks, const int32_t* __restrict__ bases, int32_t n_bits, int64_t top_k,
    int32_t* __restrict__ sorted_sel, int64_t* __restrict__ perm, int64_t* __restrict__ token_index,
    int32_t* __restrict__ route_pos) {
  extern __shared__ int32_t pos[];  // n_experts + 1 running output positions
  const int64_t b = blockIdx.x;
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) pos[e] = bases[(int64_t)e * n_chunks + b];
  __syncthreads();
  scatter_chunk(sel, n_routes, n_experts, chunk, n_bits, top_k, pos, sorted_sel, perm, token_index, route_pos);
}

// Upper-bound binary search per expert over an already sorted int32 array
// (the reference's cvmm_expert_offsets_kernel, cvmm.py:315-335).
__global__ void expert_offsets_kernel(const int32_t* __restrict__ sorted_sel, int64_t n_routes,
                                      int32_t n_experts, int64_t* __restrict__ offsets) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_experts) return;
  int64_t lo = 0, hi = n_routes;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)sorted_sel[mid] <= e) lo = mid + 1;
    else hi = mid;
  }
  offsets[e] = lo;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int64_t sort_chunk_size(int64_t n_routes) {
  // ~256 workgroups at large R, at least 4 rounds of 256 routes per chunk.
  int64_t c = (n_routes + 255) / 256;
  c = (c + kSortThreads - 1) / kSortThreads * kSortThreads;
  if (c < 1024) c = 1024;
  if (c > 16384) c = 16384;
  return c;
}

size_t sort_workspace_bytes(int64_t n_routes, int32_t n_experts) {
  const int64_t chunk = sort_chunk_size(n_routes);
  const int64_t n_chunks = n_routes > 0 ? (n_routes + chunk - 1) / chunk : 1;
  size_t counts = (size_t)(n_experts + 1) * n_chunks * sizeof(int32_t);
  return align_up(counts, 256) + 256;  // + n_invalid counter
}

hipError_t launch_sort_routes(const void* sel, bool sel_is_int64, int64_t n_routes, int32_t n_experts,
                              int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                              int64_t* offsets, int32_t* route_pos, int32_t* n_invalid_out, void* ws,
                              hipStream_t stream) {
  const int64_t chunk = sort_chunk_size(n_routes);
  const int64_t n_chunks = (n_routes + chunk - 1) / chunk;
  int32_t* counts = (int32_t*)ws;
  int32_t* n_invalid = n_invalid_out ? n_invalid_out
                                     : (int32_t*)((char*)ws + align_up((size_t)(n_experts + 1) * n_chunks * 4, 256));
  const size_t lds = (size_t)(n_experts + 1) * sizeof(int32_t);
  int n_bits = 0;
  while ((1ll << n_bits) <= (int64_t)n_experts) ++n_bits;  // buckets 0..E
  if (sel_is_int64) {
    hipLaunchKernelGGL(sort_hist_kernel<int64_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                       (const int64_t*)sel, n_routes, n_experts, chunk, n_chunks, counts);
  } else {
    hipLaunchKernelGGL(sort_hist_kernel<int32_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                       (const int32_t*)sel, n_routes, n_experts, chunk, n_chunks, counts);
  }
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, counts, n_chunks, n_experts,
                     offsets, n_invalid, n_routes);
  if (sel_is_int64) {
    hipLaunchKernelGGL(sort_scatter_kernel<int64_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                       (const int64_t*)sel, n_routes, n_experts, chunk, n_chunks, counts, n_bits, top_k,
                       sorted_sel, perm, token_index, route_pos);
  } else {
    hipLaunchKernelGGL(sort_scatter_kernel<int32_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                       (const int32_t*)sel, n_routes, n_experts, chunk, n_chunks, counts, n_bits, top_k,
                       sorted_sel, perm, token_index, route_pos);
  }
  return hipGetLastError();
}

hipError_t launch_expert_offsets(const int32_t* sorted_sel, int64_t n_routes, int32_t n_experts,
                                 int64_t* offsets, hipStream_t stream) {
  const int threads = 256;
  hipLaunchKernelGGL(expert_offsets_kernel, dim3((n_experts + threads - 1) / threads), dim3(threads), 0, stream,
                     sorted_sel, n_routes, n_experts, offsets);
  return hipGetLastError();
}

}  // namespace cvmm
