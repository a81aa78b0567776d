// Pieces shared by the routed GEMM kernels: the in-kernel tile scheduler, the
// per-row route metadata and the epilogue (all driven by GemmParams).
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

constexpr int kGemmThreads = 256;

// The launcher's tile order for the k-looped kernels (ring, tiled): token
// major when every gathered A row feeds many routes (the SwitchHead products,
// 64 routes per token) -- tile j of every expert covers the same token range,
// so one XCD's workgroups share those rows in L2.  At top-8 fan-out the extra
// weight traffic (every XCD reads every expert's weights) costs more than it
// saves, and the small-K kernels, whose weights dominate, lose either way
// (measured on the benchmark shapes).
inline int32_t resolve_token_major(const GemmParams& p) {
  if (p.token_major >= 0) return p.token_major;
  return (p.n_experts <= kTokenMajorMaxExperts && p.a_rows > 0 && p.n_routes >= 32 * p.a_rows) ? 1 : 0;
}

template <int BM>
struct RouteMeta {
  int64_t arow[BM];   // A row of tile row r, -1 if none
  int64_t orow[BM];   // output row, -1 if none
  int64_t widx[BM];   // routing-weight / dgate index
  int64_t dgrow[BM];  // x row for the routing-weight gradient
  float w[BM];        // rounded routing weight (1 if unweighted)
  int32_t expert;
  int64_t row0;
  int32_t rows;
};

// Find the (expert, first route, row count) of m-tile `tile`: expert e owns
// ceil(count_e / BM) consecutive tiles.  Wave 0 scans the offsets 64 experts at
// a time; returns false (uniformly) when `tile` is past the last tile.
template <int BM>
__device__ bool gemm_schedule_tile(const GemmParams& p, int64_t tile, RouteMeta<BM>& m) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // ---- schedule: which expert / routes does m-tile `tile` cover? -----------
  if (wave == 0 && p.token_major > 0) {
    // Token-major order: all tiles with index j within their expert, in
    // expert order, then index j + 1.  Routes of an expert are sorted by
    // token, so tile j of every expert covers about the same token range and
    // neighbouring workgroups (one XCD) gather the same activation rows.
    // C(j) = sum_e min(nt_e, j) tiles come before index j; binary search.
    constexpr int G = kTokenMajorMaxExperts / 64;
    if (lane == 0) m.expert = -1;
    int64_t st[G], en[G], nt[G], ntmax = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int32_t e = g * 64 + lane;
      st[g] = en[g] = nt[g] = 0;
      if (e < p.n_experts) {
        int64_t end = p.offsets[e];
        int64_t start = e > 0 ? p.offsets[e - 1] : 0;
        end = end < 0 ? 0 : (end > p.n_routes ? p.n_routes : end);
        start = start < 0 ? 0 : (start > p.n_routes ? p.n_routes : start);
        if (end < start) end = start;
        st[g] = start;
        en[g] = end;
        nt[g] = (end - start + BM - 1) / BM;
      }
      ntmax = nt[g] > ntmax ? nt[g] : ntmax;
    }
    for (int o = 32; o > 0; o >>= 1) {
      const int64_t v = __shfl_xor(ntmax, o, 64);
      ntmax = v > ntmax ? v : ntmax;
    }
    auto before = [&](int64_t j) {
      int64_t s = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) s += nt[g] < j ? nt[g] : j;
      return __shfl(wave_incl_scan(s), 63, 64);
    };
    const int64_t n_tiles = before(ntmax);
    if (lane == 0 && tile >= n_tiles) m.row0 = n_tiles;  // past the last tile: the tile count
    if (tile < n_tiles) {
      int64_t lo = 0, hi = ntmax;  // before(lo) <= tile < before(hi)
      while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (before(mid) <= tile) lo = mid;
        else hi = mid;
      }
      int64_t r = tile - before(lo);  // rank among the experts with more than lo tiles
      const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const bool has = nt[g] > lo;
        const uint64_t b = __ballot(has);
        const int64_t cnt = __popcll(b);
        if (r >= 0 && r < cnt && has && (int64_t)__popcll(b & lt_mask) == r) {
          m.expert = g * 64 + lane;
          const int64_t r0 = st[g] + lo * BM;
          m.row0 = r0;
          m.rows = (int32_t)((en[g] - r0) < BM ? (en[g] - r0) : BM);
        }
        r -= cnt;
      }
    }
  } else if (wave == 0) {
    if (lane == 0) m.expert = -1;
    int64_t carry = 0;
    for (int32_t base = 0; base < p.n_experts; base += 64) {
      const int32_t e = base + lane;
      int64_t start = 0, end = 0;
      if (e < p.n_experts) {
        end = p.offsets[e];
        start = e > 0 ? p.offsets[e - 1] : 0;
        end = end < 0 ? 0 : (end > p.n_routes ? p.n_routes : end);
        start = start < 0 ? 0 : (start > p.n_routes ? p.n_routes : start);
        if (end < start) end = start;
      }
      const int64_t nt = (end - start + BM - 1) / BM;
      const int64_t incl = wave_incl_scan(nt) + carry;
      const int64_t excl = incl - nt;
      if (e < p.n_experts && tile >= excl && tile < incl) {
        m.expert = e;
        const int64_t r0 = start + (tile - excl) * BM;
        m.row0 = r0;
        m.rows = (int32_t)((end - r0) < BM ? (end - r0) : BM);
      }
      carry = __shfl(incl, 63, 64);
      if (tile < carry) break;
    }
    if (lane == 0 && m.expert < 0) m.row0 = carry;  // past the last tile: the tile count
  }
  __syncthreads();
  return m.expert >= 0;
}

// The route metadata of every row of the tile gemm_schedule_tile found (NT:
// the workgroup's thread count).
template <int BM, int NT = kGemmThreads>
__device__ void gemm_route_meta(const GemmParams& p, RouteMeta<BM>& m) {
  const int tid = threadIdx.x;
  const int64_t row0 = m.row0;
  const int32_t rows = m.rows;
  for (int r = tid; r < BM; r += NT) {
    int64_t ar = -1, orow = -1, widx = -1, dgr = -1;
    float wv = 1.f;
    if (r < rows) {
      const int64_t q = row0 + r;
      const int64_t ai = p.a_idx[q] / p.a_div;
      if (ai >= 0 && ai < p.a_rows) ar = ai;
      const int64_t oi = p.o_idx != nullptr ? p.o_idx[q] / p.o_div : q;
      if (oi >= 0 && oi < p.out_rows) orow = oi;
      if (p.w_idx != nullptr) {
        const int64_t wi = p.w_idx[q];
        if (wi >= 0 && wi < p.n_routes) widx = wi;
      }
      if (p.w != nullptr && widx >= 0) wv = round_to(load_as_f32(p.w, p.w_dtype, widx), p.w_round);
      if (p.dg != nullptr) {
        const int64_t di = p.dg_x_idx[q];
        if (di >= 0 && di < p.dg_x_rows) dgr = di;
      }
    }
    m.arow[r] = ar;
    m.orow[r] = orow;
    m.widx[r] = widx;
    m.w[r] = wv;
    m.dgrow[r] = dgr;
  }
  __syncthreads();
}

// Both: the tile, then its rows' route metadata.
template <int BM, int NT = kGemmThreads>
__device__ bool gemm_schedule(const GemmParams& p, int64_t tile, RouteMeta<BM>& m) {
  if (!gemm_schedule_tile<BM>(p, tile, m)) return false;
  gemm_route_meta<BM, NT>(p, m);
  return true;
}

// Called by a workgroup past the last m-tile (gemm_schedule returned false,
// leaving the tile count in m.row0), for the routes no tile covers -- expert
// id outside [0, E), sorted at or past offsets[E - 1]: when the call asks
// for it, zero the columns [c0, c1) of their output rows (and GELU
// pre-activation rows); and zero their routing-weight gradient partials
// dg_tile .. dg_tile + dg_count - 1 (dg_tile >= 0 when the caller covers
// exactly those partials' columns), so the partials need no fill before the
// launch.  Surplus m-tile j of the
// n_surplus launched takes every n_surplus-th such route; a launch of
// ceil(R / BM) + min(E, R) m-tiles has at least one surplus m-tile whenever
// such routes exist.
template <int BM, int NT = kGemmThreads>
__device__ void zero_unrouted_cols(const GemmParams& p, const RouteMeta<BM>& m, int64_t tile, int64_t m_tiles,
                                   int64_t c0, int64_t c1, int64_t dg_tile, int dg_count = 1) {
  const bool zero_out = p.zero_unrouted && p.out != nullptr;
  const bool zero_dg = p.dg != nullptr && dg_tile >= 0;
  if (!zero_out && !zero_dg) return;
  const int64_t j = tile - m.row0, n_surplus = m_tiles - m.row0;
  if (j < 0 || n_surplus <= 0) return;
  int64_t q0 = p.offsets[p.n_experts - 1];
  q0 = q0 < 0 ? 0 : q0;
  if (c1 > p.N) c1 = p.N;
  for (int64_t q = q0 + j; q < p.n_routes; q += n_surplus) {
    if (zero_dg && threadIdx.x == 0) {
      const int64_t wi = p.w_idx[q];
      if (wi >= 0 && wi < p.n_routes)
        for (int t = 0; t < dg_count; ++t) p.dg[wi * p.dg_ntiles + dg_tile + t] = 0.f;
    }
    if (!zero_out) continue;
    const int64_t oi = p.o_idx != nullptr ? p.o_idx[q] / p.o_div : q;
    if (oi < 0 || oi >= p.out_rows) continue;
    for (int64_t c = c0 + threadIdx.x; c < c1; c += NT) {
      store_from_f32(p.out, p.out_dtype, oi * p.out_ld + c, 0.f);
      if (p.act != 0 && p.aux != nullptr) store_from_f32(p.aux, p.out_dtype, oi * p.out_ld + c, 0.f);
    }
  }
}

// Epilogue over the fp32 tile of rows [0, rows) and columns
// [n0, n0 + BN): value stores (or fp32 atomics) and the routing-weight
// gradient partial of this n tile.
template <int BM, int BN, int C_LD>
__device__ void gemm_epilogue(const GemmParams& p, const float* C0, const float* C1, int half,
                              const RouteMeta<BM>& m, int64_t n0, int64_t ntile) {
  // fp32 tile row r lives at (r < half ? C0 : C1) + (r % half) * C_LD
  auto crow = [&](int r) { return (r < half ? C0 : C1) + (r % half) * C_LD; };
  const int tid = threadIdx.x;
  const int32_t rows = m.rows;
  const bool has_w = p.w != nullptr;
  if (p.out == nullptr) {
    // only the routing-weight gradient is wanted
  } else if (p.epi == kEpiStore) {
    constexpr int TPR = BN / 8;
    constexpr int RPP = kGemmThreads / TPR;
    const int cg = tid % TPR;
    const bool ovec = p.out_dtype != kF32 && p.out_ld % 8 == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
    for (int r = tid / TPR; r < rows; r += RPP) {
      const int64_t orow = m.orow[r];
      if (orow < 0) continue;
      const float wv = m.w[r];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float c = round_to(crow(r)[cg * 8 + j], p.val_dtype);
        if (has_w) {
          c = c * wv;
          if (p.prod_dtype >= 0) c = round_to(c, p.prod_dtype);
        }
        v[j] = c;
      }
      const int64_t nb = n0 + cg * 8;
      const int64_t off = orow * p.out_ld + nb;
      if (ovec && nb + 8 <= p.N) {
        Chunk16 ch;
        if (p.out_dtype == kBF16) {
#pragma unroll
          for (int j = 0; j < 8; ++j) ch.b[j] = (bf16_t)v[j];
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) ch.h[j] = (f16_t)v[j];
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.out) + off) = ch.u;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (nb + j < p.N) store_from_f32(p.out, p.out_dtype, off + j, v[j]);
      }
    }
  } else {  // kEpiAtomic: consecutive lanes -> consecutive columns of one row
    float* out = reinterpret_cast<float*>(p.out);
    const int col = tid % BN;
    const int64_t n = n0 + col;
    if (n < p.N) {
      for (int r = tid / BN; r < rows; r += kGemmThreads / BN) {
        const int64_t orow = m.orow[r];
        if (orow < 0) continue;
        float c = round_to(crow(r)[col], p.val_dtype);
        if (has_w) {
          c = c * m.w[r];
          if (p.prod_dtype >= 0) c = round_to(c, p.prod_dtype);
        }
        unsafeAtomicAdd(out + orow * p.out_ld + n, c);
      }
    }
  }

  if (p.dg != nullptr) {  // routing-weight gradient partial over this n tile
    constexpr int TPR = BN / 8;
    constexpr int RPP = kGemmThreads / TPR;
    const int cg = tid % TPR;
    for (int r0 = 0; r0 < BM; r0 += RPP) {
      const int r = r0 + tid / TPR;
      float s = 0.f;
      const int64_t xr = r < rows ? m.dgrow[r] : -1;
      if (xr >= 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t n = n0 + cg * 8 + j;
          if (n < p.N)
            s += round_to(crow(r)[cg * 8 + j], p.dg_val_dtype) *
                 load_as_f32(p.dg_x, p.dg_x_dtype, xr * p.dg_x_ld + n);
        }
      }
      // fixed-order butterfly over the TPR lanes of the row (deterministic)
#pragma unroll
      for (int d = 1; d < TPR; d <<= 1) s += __shfl_xor(s, d, 64);
      // every covered route writes its partial (0 without an x row): the
      // partials are not zero-filled before the launch
      if (cg == 0 && r < rows && m.widx[r] >= 0)
        p.dg[m.widx[r] * p.dg_ntiles + ntile] = s;
    }
  }
}


}  // namespace cvmm
