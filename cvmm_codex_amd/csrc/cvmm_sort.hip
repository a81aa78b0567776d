// Selector preparation: stable counting sort of routes by expert.
//
// Replaces the ATen sort of cvmm_prepare_sel / cvmm_prepare_sel2
// (cvmm.py:24-27, cvmm.py:1796-1803) and the offsets binary search
// (cvmm_expert_offsets_kernel, cvmm.py:315-335).
//
// Two launches over chunks of routes:
//   1. histogram   counts[chunk][bucket]      (LDS atomics, bucket E = invalid id)
//   2. scatter     every workgroup first derives its own output positions from
//                  the histogram rows: bucket totals over all chunks, their
//                  exclusive scan (the bucket bases), plus this bucket's counts
//                  in earlier chunks; workgroup 0 also writes the inclusive
//                  per-expert offsets the GEMM schedulers read.  Then the chunk
//                  walks its routes in index order; a route's rank among equal
//                  keys of its wave comes from ballots over the key bits, waves
//                  of a workgroup take turns, so the order is stable (equal
//                  experts keep route order).
// The chunk size keeps (E + 1) * n_chunks, the counts each workgroup reads,
// at most 64K.
#include <atomic>

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_keys.h"

namespace cvmm {

constexpr int kSortThreads = 256;
constexpr int32_t kSortFastBuckets = 8192;  // buckets whose totals fit beside the positions in LDS
// >= 4 rounds of 256 routes per workgroup: fewer chunks keep the count matrix
// every scatter workgroup reads small (measured: ff_up 19.5 us with 256-route
// chunks, 17.6 us with 1024)
constexpr int64_t kSortMinChunk = 1024;

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
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) counts[b * (int64_t)(n_experts + 1) + e] = hist[e];
}

// The histogram launch fused with the int32 copy of the ids that selector
// preparation takes anyway: chunk b's ids are copied and counted by bucket
// (int64 ids by their low 32 bits, the value the copy keeps).
template <typename IdxT>
__global__ __launch_bounds__(kSortThreads) void copy_ids_count_kernel(
    const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
    int32_t* __restrict__ out, int32_t* __restrict__ counts) {
  extern __shared__ int32_t hist[];  // n_experts + 1
  const int64_t b = blockIdx.x;
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) hist[e] = 0;
  __syncthreads();
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  for (int64_t i = lo + threadIdx.x; i < hi; i += kSortThreads) {
    const int32_t v = (int32_t)sel[i];
    out[i] = v;
    atomicAdd(&hist[bucket_of(v, n_experts)], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= n_experts; e += kSortThreads) counts[b * (int64_t)(n_experts + 1) + e] = hist[e];
}

// Exclusive scan, in place, of the n values a[0, n) in LDS (whole workgroup).
__device__ void block_exclusive_scan(int32_t* a, int32_t n) {
  __shared__ int64_t wave_total[kSortThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t seg = (n + kSortThreads - 1) / kSortThreads;
  const int32_t lo = min(tid * seg, n), hi = min(lo + seg, n);
  int64_t sum = 0;
  for (int32_t i = lo; i < hi; ++i) sum += a[i];
  const int64_t incl = wave_incl_scan(sum);
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  int64_t run = incl - sum;
  for (int w = 0; w < wave; ++w) run += wave_total[w];
  for (int32_t i = lo; i < hi; ++i) {
    const int32_t v = a[i];
    a[i] = (int32_t)run;
    run += v;
  }
  __syncthreads();
}

// Ids of the first kSortPrefetch rounds of a chunk, loaded before the
// count-matrix pass so that their latency overlaps it.
constexpr int kSortPrefetch = 4;

// Stable scatter of one chunk: within every 256-route round, lanes with equal
// buckets are ranked by a ballot per bucket bit and the waves take their
// positions in order, so equal ids keep their input order.  `pos` holds this
// chunk's next output position per bucket; `pre` the prefetched ids.
template <typename IdxT>
__device__ void scatter_chunk(const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
                              int32_t n_bits, int64_t top_k, int32_t* pos, int32_t* __restrict__ sorted_sel,
                              int64_t* __restrict__ perm, int64_t* __restrict__ token_index,
                              int32_t* __restrict__ route_pos, int64_t b, const IdxT (&pre)[kSortPrefetch]) {
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  int round = 0;
  for (int64_t base = lo; base < hi; base += kSortThreads, ++round) {
    const int64_t i = base + threadIdx.x;
    const bool valid = i < hi;
    IdxT key = (IdxT)0;
    if (round < kSortPrefetch) {
#pragma unroll
      for (int r = 0; r < kSortPrefetch; ++r)
        if (r == round) key = pre[r];
    } else if (valid) {
      key = sel[i];
    }
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
      lds_barrier();  // pos[] is handed to the next wave; the stores may still be in flight
    }
  }
}

// Routes per wave of the turn-free scatter: a quarter of the chunk, whole
// 64-route rounds.
__host__ __device__ inline int64_t scatter_wave_span(int64_t n) { return ((n + 3) / 4 + 63) / 64 * 64; }

// Stable scatter of one chunk without turns between the waves: wave w owns
// the routes [lo + w * span, lo + (w + 1) * span).  It counts them per
// bucket (64 at a time: one ballot per bucket bit ranks the lanes of a
// bucket, the lowest lane adds the count), an exclusive scan over the four
// waves gives every wave its first output position per bucket, and each
// wave then writes its routes.  Equal buckets keep route order: a wave's
// routes precede the next wave's, and a wave goes through its rounds and
// lanes in route order.  Two barriers per chunk, where the turns of
// scatter_chunk take one per wave and 256-route round.  `pos`: the chunk's
// first output position per bucket; `wpos`: 4 x (E + 1) LDS ints; `pre`: the
// wave's first rounds' ids.
template <typename IdxT>
__device__ void scatter_chunk_waves(const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
                                    int32_t n_bits, int64_t top_k, const int32_t* pos, int32_t* wpos,
                                    int32_t* __restrict__ sorted_sel, int64_t* __restrict__ perm,
                                    int64_t* __restrict__ token_index, int32_t* __restrict__ route_pos, int64_t b,
                                    const IdxT (&pre)[kSortPrefetch]) {
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int32_t nb = n_experts + 1;
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  const int64_t span = scatter_wave_span(hi - lo);
  const int64_t w_lo = lo + wave * span;
  const int64_t w_hi = min(w_lo + span, hi);
  int32_t* mine = wpos + wave * nb;
  for (int32_t e = lane; e < nb; e += 64) mine[e] = 0;
  // route indices are < 2^31; a top_k at least that large puts every route in token 0
  const bool huge_k = top_k >= (int64_t(1) << 31);
  const FastDiv by_k = make_fast_div_dev(huge_k ? 1 : top_k);

  // one 64-route round: the route's key, bucket, rank among its bucket's
  // lanes and the bucket's lane count
  auto round_of = [&](int r, int64_t base, IdxT& key, int32_t& bucket, int& rank, int& cnt) {
    const int64_t i = base + lane;
    const bool valid = i < w_hi;
    key = (IdxT)0;
    if (r < kSortPrefetch) {
#pragma unroll
      for (int q = 0; q < kSortPrefetch; ++q)
        if (q == r) key = pre[q];
    } else if (valid) {
      key = sel[i];
    }
    bucket = valid ? bucket_of(key, n_experts) : 0;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < n_bits; ++bit) {
      const bool set = (bucket >> bit) & 1;
      const uint64_t bb = __ballot(set);
      peers &= set ? bb : ~bb;
    }
    rank = valid ? __popcll(peers & lt_mask) : -1;
    cnt = __popcll(peers);
  };

  // counts need no ranks: one LDS add per route
  int r = 0;
  for (int64_t base = w_lo; base < w_hi; base += 64, ++r) {
    const int64_t i = base + lane;
    if (i < w_hi) {
      IdxT key = (IdxT)0;
      if (r < kSortPrefetch) {
#pragma unroll
        for (int q = 0; q < kSortPrefetch; ++q)
          if (q == r) key = pre[q];
      } else {
        key = sel[i];
      }
      atomicAdd(&mine[bucket_of(key, n_experts)], 1);
    }
  }
  lds_barrier();
  for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) {
    int32_t run = pos[e];
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) {
      const int32_t c = wpos[w * nb + e];
      wpos[w * nb + e] = run;
      run += c;
    }
  }
  lds_barrier();
  r = 0;
  for (int64_t base = w_lo; base < w_hi; base += 64, ++r) {
    IdxT key;
    int32_t bucket;
    int rank, cnt;
    round_of(r, base, key, bucket, rank, cnt);
    if (rank >= 0) {
      const int64_t i = base + lane;
      const int32_t p0 = mine[bucket];
      const int64_t p = (int64_t)p0 + rank;
      sorted_sel[p] = (int32_t)key;
      perm[p] = i;
      if (token_index != nullptr) token_index[p] = huge_k ? 0 : by_k.div(i);
      if (route_pos != nullptr) route_pos[i] = (int32_t)p;
      // after the wave's reads of this round (LDS operations of a wave run in order)
      if (rank == 0) mine[bucket] = p0 + cnt;
    }
  }
}

// The chunks that scatter through LDS (scatter_chunk_local): up to this many
// buckets (4 x (E + 1) positions in the dynamic LDS) and routes (a key and a
// route offset each in the launch's 33 KB tile buffer), in selections of at
// least this many routes.  Measured against the direct scatter (same box,
// sort + cast per step): switch_v (524288 routes, 256 experts) 40.4 -> 33.2
// us, switch_o 35.0 -> 31.8 us, ff_up (65536 routes, 64 chunks: the
// scatter's latency, not its stores, is the limit) 16.1 -> 17.0 us.
constexpr int32_t kSortLocalBuckets = 2048;
constexpr int64_t kSortLocalChunk = kCastTileFloats / 2;
constexpr int64_t kSortLocalMinRoutes = 1 << 18;

// The same stable order through LDS: the rounds place each route at its
// local position (the chunk's routes bucket by bucket, equal buckets in
// route order) with its key and offset, writing route_pos on the way (route
// order, coalesced); then the threads walk the local positions and write
// sorted_sel, perm and token_index: each bucket's run of the chunk goes to
// consecutive output positions, where the direct scatter stores one 4- or
// 8-byte value per route and output at a scattered position (a partial line
// written back per store).  lbase = the chunk's first local position of each
// bucket, lpos its running copy, gpos the chunk's first output position.
template <typename IdxT>
__device__ void scatter_chunk_local(const IdxT* __restrict__ sel, int64_t n_routes, int32_t n_experts, int64_t chunk,
                                    int32_t n_bits, int64_t top_k, const int32_t* gpos, int32_t* lpos,
                                    const int32_t* lbase, int32_t* l_key, int32_t* l_route,
                                    int32_t* __restrict__ sorted_sel, int64_t* __restrict__ perm,
                                    int64_t* __restrict__ token_index, int32_t* __restrict__ route_pos, int64_t b,
                                    const IdxT (&pre)[kSortPrefetch]) {
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t lo = b * chunk;
  const int64_t hi = min(lo + chunk, n_routes);
  int round = 0;
  for (int64_t base = lo; base < hi; base += kSortThreads, ++round) {
    const int64_t i = base + threadIdx.x;
    const bool valid = i < hi;
    IdxT key = (IdxT)0;
    if (round < kSortPrefetch) {
#pragma unroll
      for (int r = 0; r < kSortPrefetch; ++r)
        if (r == round) key = pre[r];
    } else if (valid) {
      key = sel[i];
    }
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
        const int32_t p0 = lpos[bucket];
        const int32_t lp = p0 + rank;
        if (rank == 0) lpos[bucket] = p0 + cnt;
        l_key[lp] = (int32_t)key;
        l_route[lp] = (int32_t)(i - lo);
        if (route_pos != nullptr) route_pos[i] = gpos[bucket] + (lp - lbase[bucket]);
      }
      lds_barrier();  // lpos[] and the local order are handed on through LDS
    }
  }
  const int32_t n = (int32_t)(hi - lo);
  for (int32_t lp = threadIdx.x; lp < n; lp += kSortThreads) {
    const int32_t key = l_key[lp];
    const int32_t e = bucket_of(key, n_experts);
    const int64_t p = (int64_t)gpos[e] + (lp - lbase[e]);
    const int64_t i = lo + l_route[lp];
    sorted_sel[p] = key;
    perm[p] = i;
    if (token_index != nullptr) token_index[p] = i / top_k;
  }
}

// Dynamic LDS of a scatter workgroup: its positions (and totals, local
// positions and bases), plus, for the scatter launch of its own, the local
// order (the launch that casts beside it lends the cast's tile instead).
size_t scatter_lds_bytes(int32_t n_experts) {
  const int32_t nb = n_experts + 1;
  // positions, then totals / local positions / local bases, or the
  // turn-free scatter's 4 x nb wave positions (over the totals, which are
  // dead by then)
  if (nb <= kSortLocalBuckets) return (size_t)5 * nb * sizeof(int32_t);
  return (size_t)(nb <= kSortFastBuckets ? 2 : 1) * nb * sizeof(int32_t);
}
static size_t scatter_kernel_lds_bytes(int32_t n_experts) {
  return scatter_lds_bytes(n_experts) + (n_experts + 1 <= kSortLocalBuckets ? kCastTileFloats * sizeof(float) : 0);
}

// Whether the scatter fits in one launch with the cast (its positions beside
// the cast's 33 KB tile, within the 160 KB of LDS a workgroup may take).
bool sort_cast_fusable(int32_t n_experts) {
  return scatter_lds_bytes(n_experts) + kCastTileFloats * sizeof(float) + 1024 <= 160 * 1024;
}

template <typename IdxT>
struct ScatterArgs {
  const IdxT* sel;
  int64_t n_routes;
  int32_t n_experts;
  int64_t chunk, n_chunks;
  const int32_t* counts;
  int32_t n_bits;
  int64_t top_k;
  int32_t* sorted_sel;
  int64_t* perm;
  int64_t* token_index;
  int32_t* route_pos;
  int64_t* offsets;
  int32_t* n_invalid;
  // not NULL: `counts` already holds each chunk's count of every bucket in
  // the earlier chunks and tot[e] the bucket totals (sort_colscan_kernel)
  const int32_t* tot;
};

// Chunk b: output positions from the histogram rows, then the stable scatter.
// sh: n_experts + 1 positions (+ n_experts + 1 totals when <= kSortFastBuckets).
template <typename IdxT>
__device__ void scatter_block(const ScatterArgs<IdxT>& a, int32_t* sh, int64_t b, float* tile) {
  const int64_t n_routes = a.n_routes, chunk = a.chunk, n_chunks = a.n_chunks, top_k = a.top_k;
  const int32_t n_experts = a.n_experts, n_bits = a.n_bits;
  const int32_t* __restrict__ counts = a.counts;
  int64_t* __restrict__ offsets = a.offsets;
  int32_t* __restrict__ n_invalid = a.n_invalid;
  int32_t* pos = sh;  // running output positions of this chunk
  const int32_t nb = n_experts + 1;
  // through LDS (scatter_chunk_local): the chunk's own count of each bucket
  // goes to lbase (then its exclusive scan) beside pos and the totals
  const bool local = nb <= kSortLocalBuckets && chunk <= kSortLocalChunk && n_routes >= kSortLocalMinRoutes;
  // the turn-free scatter (scatter_chunk_waves) where its wave positions fit
  const bool waves = !local && nb <= kSortLocalBuckets;
  int32_t* lpos = sh + 2 * nb;
  int32_t* lbase = sh + 3 * nb;
  // the first rounds' ids, loaded before the count-matrix pass so that their
  // latency overlaps it: 256-route rounds in thread order, or the wave's own
  // 64-route rounds
  IdxT pre[kSortPrefetch];
  {
    const int64_t lo = b * chunk, hi = min(lo + chunk, n_routes);
    const int64_t w_lo = lo + (threadIdx.x >> 6) * scatter_wave_span(hi - lo);
    const int64_t w_hi = min(w_lo + scatter_wave_span(hi - lo), hi);
#pragma unroll
    for (int r = 0; r < kSortPrefetch; ++r) {
      const int64_t i = waves ? w_lo + r * 64 + lane_id() : lo + r * kSortThreads + threadIdx.x;
      pre[r] = a.sel[i < hi ? i : hi - 1];  // unconditional (see the count pass); masked by index later
    }
  }
  if (a.tot != nullptr) {
    // the column scan did the count-matrix pass: this chunk's row and the
    // bucket totals only
    int32_t* tot = sh + nb;
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) {
      tot[e] = a.tot[e];
      pos[e] = counts[b * (int64_t)nb + e];
      if (local) lbase[e] = (b + 1 < n_chunks ? counts[(b + 1) * (int64_t)nb + e] : a.tot[e]) - pos[e];
    }
    __syncthreads();
    if (b == 0 && threadIdx.x == 0 && n_invalid != nullptr) *n_invalid = tot[n_experts];
    block_exclusive_scan(tot, nb);  // tot[e] = first output position of bucket e
    if (b == 0) {
      for (int32_t e = threadIdx.x; e < n_experts; e += kSortThreads) offsets[e] = tot[e + 1];
    }
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) pos[e] += tot[e];
  } else if (nb <= kSortFastBuckets) {
    // All threads stride over the whole count matrix (loads batched 32 deep);
    // consecutive elements belong to distinct buckets, so the LDS adds of one
    // wave instruction do not collide.
    int32_t* tot = sh + nb;
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) {
      pos[e] = tot[e] = 0;
      if (local) lbase[e] = 0;
    }
    lds_barrier();  // (the prefetched ids may still be in flight)
    const int32_t n = (int32_t)(n_chunks * nb);
    const FastDiv by_nb = make_fast_div_dev(nb);
    constexpr int U = 32;
    for (int32_t i0 = threadIdx.x; i0 < n; i0 += U * kSortThreads) {
      int32_t v[U];
      // unconditional loads (a clamped index, masked below): a load under a
      // branch makes the compiler wait for it before the next one
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int32_t i = i0 + u * kSortThreads;
        v[u] = counts[i < n ? i : n - 1];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int32_t i = i0 + u * kSortThreads;
        if (i < n) {
          const int32_t c = (int32_t)by_nb.div(i), e = i - c * nb;
          atomicAdd(&tot[e], v[u]);
          if (c < b) atomicAdd(&pos[e], v[u]);
          if (local && c == b) lbase[e] = v[u];
        }
      }
    }
    lds_barrier();
    if (b == 0 && threadIdx.x == 0 && n_invalid != nullptr) *n_invalid = tot[n_experts];
    block_exclusive_scan(tot, nb);  // tot[e] = first output position of bucket e
    if (b == 0) {
      // inclusive offsets (the reference's cumsum)
      for (int32_t e = threadIdx.x; e < n_experts; e += kSortThreads) offsets[e] = tot[e + 1];
    }
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) pos[e] += tot[e];
  } else {
    // many buckets: per-bucket column sums, then the earlier chunks again
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) {
      int32_t t = 0;
      for (int64_t c = 0; c < n_chunks; ++c) t += counts[c * nb + e];
      pos[e] = t;
    }
    __syncthreads();
    if (b == 0 && threadIdx.x == 0 && n_invalid != nullptr) *n_invalid = pos[n_experts];
    block_exclusive_scan(pos, nb);
    if (b == 0) {
      for (int32_t e = threadIdx.x; e < n_experts; e += kSortThreads) offsets[e] = pos[e + 1];
    }
    __syncthreads();  // the offsets above read pos before it is moved to this chunk
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) {
      int32_t pre = 0;
      for (int64_t c = 0; c < b; ++c) pre += counts[c * nb + e];
      pos[e] += pre;
    }
  }
  __syncthreads();
  if (local) {
    block_exclusive_scan(lbase, nb);
    for (int32_t e = threadIdx.x; e < nb; e += kSortThreads) lpos[e] = lbase[e];
    __syncthreads();
    int32_t* l_key = reinterpret_cast<int32_t*>(tile);
    scatter_chunk_local(a.sel, n_routes, n_experts, chunk, n_bits, top_k, pos, lpos, lbase, l_key,
                        l_key + kSortLocalChunk, a.sorted_sel, a.perm, a.token_index, a.route_pos, b, pre);
    return;
  }
  if (waves) {
    scatter_chunk_waves(a.sel, n_routes, n_experts, chunk, n_bits, top_k, pos, sh + nb, a.sorted_sel, a.perm,
                        a.token_index, a.route_pos, b, pre);
    return;
  }
  scatter_chunk(a.sel, n_routes, n_experts, chunk, n_bits, top_k, pos, a.sorted_sel, a.perm, a.token_index,
                a.route_pos, b, pre);
}

template <typename IdxT>
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(const ScatterArgs<IdxT> a) {
  extern __shared__ int32_t sh[];
  const int32_t nb = a.n_experts + 1;
  // the local order after the positions (scatter_kernel_lds_bytes)
  scatter_block(a, sh, blockIdx.x, reinterpret_cast<float*>(sh + (nb <= kSortLocalBuckets ? 4 * nb : 0)));
}

// The scatter and the per-step weight cast in one launch: workgroups
// [0, n_chunks) scatter, the rest cast 64 x 64 weight tiles.  The scatter
// (a few workgroups, latency-bound) runs in the shadow of the cast.
template <typename IdxT, typename OutT>
__global__ __launch_bounds__(kSortThreads) void sort_scatter_cast_kernel(const ScatterArgs<IdxT> a,
                                                                         const CastArgs<OutT> c) {
  extern __shared__ int32_t sh[];
  __shared__ float tile[kCastTileFloats];  // the cast's tile, or the scatter's local order
  if ((int64_t)blockIdx.x < a.n_chunks) {
    scatter_block(a, sh, blockIdx.x, tile);
  } else {
    cast_block(c, (int64_t)blockIdx.x - a.n_chunks, tile);
  }
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

static std::atomic<int64_t> g_sort_chunk{0};
void set_sort_chunk(int64_t routes) { g_sort_chunk.store(routes); }

int64_t sort_chunk_size(int64_t n_routes, int32_t n_experts) {
  const int64_t knob = g_sort_chunk.load();
  if (knob > 0) return (knob + kSortThreads - 1) / kSortThreads * kSortThreads;
  // >= kSortMinChunk routes; (E + 1) * n_chunks <= 64K.  A sort of fewer than
  // 8 such chunks takes 8 chunks of at least one round (256 routes): its
  // launch is latency-bound, and a chunk's waves go through their routes in
  // rounds of 64.
  int64_t c = (n_routes * (int64_t)(n_experts + 1) + 65535) / 65536;
  if (c < kSortMinChunk) c = n_routes < 8 * kSortMinChunk ? std::max<int64_t>((n_routes + 7) / 8, kSortThreads)
                                                          : kSortMinChunk;
  return (c + kSortThreads - 1) / kSortThreads * kSortThreads;
}

// Count matrices at least this large (chunks x buckets, with >= 64 buckets)
// are scanned once by sort_colscan_kernel instead of by every scatter
// workgroup (each of which would otherwise read all of it: 65K entries at
// 524288 routes over 256 experts).
constexpr int64_t kSortColscanMin = 16384;
constexpr int kColscanWaves = 16;  // chunk segments per bucket
constexpr int kColscanBatch = 16;  // loads in flight per lane

bool sort_use_colscan(int64_t n_chunks, int32_t n_experts) {
  const int64_t nb = (int64_t)n_experts + 1;
  return nb >= 64 && nb <= kSortFastBuckets && n_chunks * nb >= kSortColscanMin;
}

// In place: counts[c][e] becomes sum_{c' < c} counts[c'][e]; tot[e] = the sum
// over all chunks.  Workgroup = 64 buckets (lanes) x 16 chunk segments
// (waves); each lane reads its segment in batches of 16 independent loads,
// the waves' segment sums are scanned through LDS, and a second pass writes
// the running prefixes.
__global__ __launch_bounds__(64 * kColscanWaves) void sort_colscan_kernel(int32_t* __restrict__ counts,
                                                                          int64_t n_chunks, int32_t nb,
                                                                          int32_t* __restrict__ tot) {
  __shared__ int32_t part[kColscanWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int32_t e = blockIdx.x * 64 + lane;
  const int64_t q = (n_chunks + kColscanWaves - 1) / kColscanWaves;
  const int64_t c0 = min((int64_t)w * q, n_chunks), c1 = min(c0 + q, n_chunks);
  int32_t sum = 0;
  if (e < nb) {
    for (int64_t cb = c0; cb < c1; cb += kColscanBatch) {
      int32_t v[kColscanBatch];
#pragma unroll
      for (int u = 0; u < kColscanBatch; ++u) v[u] = cb + u < c1 ? counts[(cb + u) * nb + e] : 0;
#pragma unroll
      for (int u = 0; u < kColscanBatch; ++u) sum += v[u];
    }
  }
  part[w][lane] = sum;
  __syncthreads();
  int32_t run = 0;
  for (int v = 0; v < w; ++v) run += part[v][lane];
  if (e < nb) {
    for (int64_t cb = c0; cb < c1; cb += kColscanBatch) {
      int32_t v[kColscanBatch];
#pragma unroll
      for (int u = 0; u < kColscanBatch; ++u) v[u] = cb + u < c1 ? counts[(cb + u) * nb + e] : 0;
#pragma unroll
      for (int u = 0; u < kColscanBatch; ++u) {
        if (cb + u < c1) counts[(cb + u) * nb + e] = run;
        run += v[u];
      }
    }
    if (w == kColscanWaves - 1) tot[e] = run;
  }
}

// counts (align_up to 256) + bucket totals (align_up to 256), then 256 bytes
// whose last 4 hold the router's invalid-id counter.
size_t sort_counts_bytes(int64_t n_chunks, int32_t n_experts) {
  return align_up((size_t)(n_experts + 1) * n_chunks * sizeof(int32_t), 256);
}
size_t sort_workspace_bytes(int64_t n_routes, int32_t n_experts) {
  const int64_t chunk = sort_chunk_size(n_routes, n_experts);
  const int64_t n_chunks = n_routes > 0 ? (n_routes + chunk - 1) / chunk : 1;
  return sort_counts_bytes(n_chunks, n_experts) + align_up((size_t)(n_experts + 1) * sizeof(int32_t), 256) + 256;
}

// The column scan when the matrix is large enough; returns the totals to pass
// to the scatter (NULL: the scatter scans the matrix itself).
static const int32_t* launch_colscan(int32_t* counts, int64_t n_chunks, int32_t n_experts, hipStream_t stream) {
  if (!sort_use_colscan(n_chunks, n_experts)) return nullptr;
  const int32_t nb = n_experts + 1;
  int32_t* tot = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(counts) + sort_counts_bytes(n_chunks, n_experts));
  hipLaunchKernelGGL(sort_colscan_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64 * kColscanWaves), 0, stream, counts,
                     n_chunks, nb, tot);
  return tot;
}

// Dynamic LDS above 64 KB (up to 128 KB: the scatter's positions at 32767
// experts) is requested explicitly for the kernel that takes it.
template <typename K>
static hipError_t allow_lds(K kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes);
}

template <typename IdxT>
void launch_scatter_cast(const ScatterArgs<IdxT>& a, const CastRequest& cr, size_t lds, hipStream_t stream) {
  const int64_t grid = a.n_chunks + cast_blocks(cr.n_experts, cr.d_in, cr.d_out);
  allow_lds(sort_scatter_cast_kernel<IdxT, bf16_t>, lds);
  allow_lds(sort_scatter_cast_kernel<IdxT, f16_t>, lds);
  if (cr.out_dtype == kBF16) {
    const CastArgs<bf16_t> c =
        make_cast_args<bf16_t>(cr.keys, cr.se, cr.si, cr.n_experts, cr.d_in, cr.d_out, cr.kt, cr.kn, cr.layout);
    hipLaunchKernelGGL((sort_scatter_cast_kernel<IdxT, bf16_t>), dim3((unsigned)grid), dim3(kSortThreads), lds, stream,
                       a, c);
  } else {
    const CastArgs<f16_t> c =
        make_cast_args<f16_t>(cr.keys, cr.se, cr.si, cr.n_experts, cr.d_in, cr.d_out, cr.kt, cr.kn, cr.layout);
    hipLaunchKernelGGL((sort_scatter_cast_kernel<IdxT, f16_t>), dim3((unsigned)grid), dim3(kSortThreads), lds, stream,
                       a, c);
  }
}

hipError_t launch_copy_ids_count(const void* sel, bool sel_is_int64, int64_t n_routes, int32_t n_experts,
                                 int32_t* out, void* ws, hipStream_t stream) {
  if (n_routes <= 0) return hipSuccess;
  const int64_t chunk = sort_chunk_size(n_routes, n_experts);
  const int64_t n_chunks = (n_routes + chunk - 1) / chunk;
  const size_t lds = (size_t)(n_experts + 1) * sizeof(int32_t);
  int32_t* counts = (int32_t*)ws;
  if (sel_is_int64) {
    const hipError_t e = allow_lds(copy_ids_count_kernel<int64_t>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(copy_ids_count_kernel<int64_t>, dim3((unsigned)n_chunks), dim3(kSortThreads), lds, stream,
                       (const int64_t*)sel, n_routes, n_experts, chunk, out, counts);
  } else {
    const hipError_t e = allow_lds(copy_ids_count_kernel<int32_t>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(copy_ids_count_kernel<int32_t>, dim3((unsigned)n_chunks), dim3(kSortThreads), lds, stream,
                       (const int32_t*)sel, n_routes, n_experts, chunk, out, counts);
  }
  return hipGetLastError();
}

// `counts_ready`: the workspace already holds these ids' count matrix for
// n_experts (launch_copy_ids_count); the histogram launch is skipped.
hipError_t launch_sort_routes(const void* sel, bool sel_is_int64, int64_t n_routes, int32_t n_experts,
                              int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                              int64_t* offsets, int32_t* route_pos, int32_t* n_invalid_out, void* ws,
                              hipStream_t stream, const CastRequest* cast, bool counts_ready) {
  const int64_t chunk = sort_chunk_size(n_routes, n_experts);
  const int64_t n_chunks = (n_routes + chunk - 1) / chunk;
  int32_t* counts = (int32_t*)ws;
  const size_t lds = (size_t)(n_experts + 1) * sizeof(int32_t);
  const size_t lds_scatter = cast == nullptr ? scatter_kernel_lds_bytes(n_experts) : scatter_lds_bytes(n_experts);
  {
    hipError_t e = sel_is_int64 ? allow_lds(sort_hist_kernel<int64_t>, lds) : allow_lds(sort_hist_kernel<int32_t>, lds);
    if (e == hipSuccess)
      e = sel_is_int64 ? allow_lds(sort_scatter_kernel<int64_t>, lds_scatter)
                       : allow_lds(sort_scatter_kernel<int32_t>, lds_scatter);
    if (e != hipSuccess) return e;
  }
  int n_bits = 0;
  while ((1ll << n_bits) <= (int64_t)n_experts) ++n_bits;  // buckets 0..E
  if (!counts_ready) {
    if (sel_is_int64)
      hipLaunchKernelGGL(sort_hist_kernel<int64_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                         (const int64_t*)sel, n_routes, n_experts, chunk, n_chunks, counts);
    else
      hipLaunchKernelGGL(sort_hist_kernel<int32_t>, dim3(n_chunks), dim3(kSortThreads), lds, stream,
                         (const int32_t*)sel, n_routes, n_experts, chunk, n_chunks, counts);
  }
  const int32_t* tot = launch_colscan(counts, n_chunks, n_experts, stream);
  if (sel_is_int64) {
    const ScatterArgs<int64_t> a{(const int64_t*)sel, n_routes, n_experts, chunk, n_chunks, counts, n_bits, top_k,
                                 sorted_sel, perm, token_index, route_pos, offsets, n_invalid_out, tot};
    if (cast == nullptr)
      hipLaunchKernelGGL(sort_scatter_kernel<int64_t>, dim3(n_chunks), dim3(kSortThreads), lds_scatter, stream, a);
    else
      launch_scatter_cast(a, *cast, lds_scatter, stream);
  } else {
    const ScatterArgs<int32_t> a{(const int32_t*)sel, n_routes, n_experts, chunk, n_chunks, counts, n_bits, top_k,
                                 sorted_sel, perm, token_index, route_pos, offsets, n_invalid_out, tot};
    if (cast == nullptr)
      hipLaunchKernelGGL(sort_scatter_kernel<int32_t>, dim3(n_chunks), dim3(kSortThreads), lds_scatter, stream, a);
    else
      launch_scatter_cast(a, *cast, lds_scatter, stream);
  }
  return hipGetLastError();
}

hipError_t launch_sort_scatter(const int64_t* sel, int64_t n_routes, int32_t n_experts, int64_t chunk, int64_t top_k,
                               int32_t* counts, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid_out, hipStream_t stream) {
  if (n_routes <= 0) return hipSuccess;
  const int64_t n_chunks = (n_routes + chunk - 1) / chunk;
  const size_t lds_scatter = scatter_kernel_lds_bytes(n_experts);
  {
    const hipError_t e = allow_lds(sort_scatter_kernel<int64_t>, lds_scatter);
    if (e != hipSuccess) return e;
  }
  int n_bits = 0;
  while ((1ll << n_bits) <= (int64_t)n_experts) ++n_bits;  // buckets 0..E
  const int32_t* tot = launch_colscan(counts, n_chunks, n_experts, stream);
  const ScatterArgs<int64_t> a{sel, n_routes, n_experts, chunk, n_chunks, counts, n_bits, top_k,
                               sorted_sel, perm, token_index, route_pos, offsets, n_invalid_out, tot};
  hipLaunchKernelGGL(sort_scatter_kernel<int64_t>, dim3(n_chunks), dim3(kSortThreads), lds_scatter, stream, a);
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
