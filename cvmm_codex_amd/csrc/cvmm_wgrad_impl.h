// Per-expert weight gradient dW[e] = X_e^T * G_e, the reduction axis being the
// expert's routes.  Replaces cvmm_grouped_bwd_w_gather_x_kernel
// (cvmm.py:481-538), cvmm_grouped_bwd_w_weighted_kernel (cvmm.py:541-604) and
// the split-K atomic cvmm_backward_kernel3 (cvmm.py:607-805).
//
// Work items are (expert, route chunk of `split` routes) x (BM x BN tile of
// dW).  A chunk never crosses an expert boundary.  Experts with one chunk store
// their tile directly; for hot experts every chunk writes an fp32 partial and
// the last chunk to arrive (device-scope counter) adds the partials in chunk
// order -- the result does not depend on arrival order (deterministic), unlike
// the reference's fp32 atomics.
//
// Both operands are gathered rows of route-major matrices (x rows and dY
// rows), so they are transposed into k-contiguous LDS tiles: each thread loads
// 4 routes x 8 columns (16-byte loads) and writes 8 rows of 4 k-values.
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_mfma.h"

namespace cvmm {

constexpr int kWgThreads = 256;

template <typename T>
__device__ __forceinline__ void load8_f32(const T* __restrict__ row, int64_t m, int64_t M, bool vec, float (&v)[8]) {
  if (vec && m + 8 <= M) {
    if constexpr (sizeof(T) == 4) {
      const float4 lo = *reinterpret_cast<const float4*>(row + m);
      const float4 hi = *reinterpret_cast<const float4*>(row + m + 4);
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
      v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    } else {
      const uint4 raw = *reinterpret_cast<const uint4*>(row + m);
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = to_f32(e[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (m + j < M) ? to_f32(row[m + j]) : 0.f;
  }
}

// 4 k-values of one LDS row, written as OpT (8 bytes for 16-bit, 16 for fp32).
template <typename OpT>
__device__ __forceinline__ void store4(OpT* dst, float a, float b, float c, float d) {
  if constexpr (sizeof(OpT) == 4) {
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
  } else {
    union { uint2 u; OpT e[4]; } w;
    w.e[0] = from_f32<OpT>(a); w.e[1] = from_f32<OpT>(b);
    w.e[2] = from_f32<OpT>(c); w.e[3] = from_f32<OpT>(d);
    *reinterpret_cast<uint2*>(dst) = w.u;
  }
}

template <typename OpT, typename XT, typename GT, int BM, int BN>
__global__ __launch_bounds__(kWgThreads, 2) void wgrad_kernel(const WgradParams p) {
  using Cfg = TileCfg<OpT, BM, BN>;
  constexpr int BK = Cfg::BK;                     // routes per LDS stage
  constexpr int XU = (BK / 4) * (BM / 8);         // x units (4 routes x 8 m)
  constexpr int GU = (BK / 4) * (BN / 8);
  constexpr int XPT = (XU + kWgThreads - 1) / kWgThreads;
  constexpr int GPT = (GU + kWgThreads - 1) / kWgThreads;
  constexpr int OP = DTypeOf<OpT>::value;

  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM];
  __shared__ int64_t s_xr[3][BK];
  __shared__ int64_t s_gr[3][BK];
  __shared__ float s_w[3][BK];
  __shared__ int32_t s_expert, s_nch, s_last;
  __shared__ int64_t s_lo, s_hi, s_slot, s_base_slot;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int64_t tiles = tiles_m * tiles_n;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t slot_id = id / tiles;
  const int64_t tile = id % tiles;
  const int64_t m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;

  // ---- schedule: (expert, chunk) of this slot -----------------------------------
  if (wave == 0) {
    if (lane == 0) s_expert = -1;
    int64_t carry = 0, carry_multi = 0;
    for (int32_t base = 0; base < p.n_experts; base += 64) {
      const int32_t e = base + lane;
      int64_t start = 0, end = 0, nch = 0;
      if (e < p.n_experts) {
        end = p.offsets[e];
        start = e > 0 ? p.offsets[e - 1] : 0;
        end = end < 0 ? 0 : (end > p.n_routes ? p.n_routes : end);
        start = start < 0 ? 0 : (start > p.n_routes ? p.n_routes : start);
        if (end < start) end = start;
        nch = (end - start + p.split - 1) / p.split;
        if (nch < 1) nch = 1;  // empty experts still write their (zero) gradient
      }
      const int64_t multi = nch > 1 ? nch : 0;
      const int64_t incl = wave_incl_scan(nch) + carry;
      const int64_t incl_m = wave_incl_scan(multi) + carry_multi;
      const int64_t excl = incl - nch;
      if (e < p.n_experts && slot_id >= excl && slot_id < incl) {
        const int64_t c = slot_id - excl;
        s_expert = e;
        s_nch = (int32_t)nch;
        s_lo = start + c * p.split;
        s_hi = (start + (c + 1) * p.split) < end ? start + (c + 1) * p.split : end;
        s_base_slot = incl_m - multi;
        s_slot = s_base_slot + c;
      }
      carry = __shfl(incl, 63, 64);
      carry_multi = __shfl(incl_m, 63, 64);
      if (slot_id < carry) break;
    }
  }
  __syncthreads();
  const int32_t expert = s_expert;
  if (expert < 0) return;
  const int64_t lo = s_lo, hi = s_hi;
  const int32_t nch = s_nch;
  const int64_t n_stages = (hi - lo + BK - 1) / BK;

  auto meta_load = [&](int64_t stage) {
    const int slot = (int)(stage % 3);
    if (tid < BK) {
      const int64_t q = lo + stage * BK + tid;
      int64_t xr = -1, gr = -1;
      float w = 1.f;
      if (q < hi) {
        const int64_t xi = p.x_idx[q];
        if (xi >= 0 && xi < p.x_rows) xr = xi;
        const int64_t gi = p.g_idx[q] / p.g_div;
        if (gi >= 0 && gi < p.g_rows) gr = gi;
        if (p.w != nullptr) {
          const int64_t wi = p.w_idx[q];
          w = (wi >= 0 && wi < p.n_routes) ? round_to(load_as_f32(p.w, p.w_dtype, wi), OP) : 0.f;
        }
      }
      if (xr < 0 || gr < 0) { xr = -1; gr = -1; }
      s_xr[slot][tid] = xr;
      s_gr[slot][tid] = gr;
      s_w[slot][tid] = w;
    }
  };

  OpT* As0 = reinterpret_cast<OpT*>(smem);
  OpT* Bs0 = As0 + Cfg::A_ELEMS;
  OpT* As1 = As0 + Cfg::STAGE_ELEMS;
  OpT* Bs1 = As1 + Cfg::A_ELEMS;
  const XT* xb = reinterpret_cast<const XT*>(p.x);
  const GT* gb = reinterpret_cast<const GT*>(p.g);
  const bool x_vec = p.x_vec != 0, g_vec = p.g_vec != 0;
  const bool weighted = p.w != nullptr;

  float rx[XPT][4][8];
  float rg[GPT][4][8];

  auto data_load = [&](int64_t stage) {
    const int slot = (int)(stage % 3);
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int u = tid + j * kWgThreads;
      if (u < XU) {
        const int mg = u % (BM / 8), kg = u / (BM / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t xr = s_xr[slot][kg * 4 + r];
          if (xr >= 0) load8_f32(xb + xr * p.x_ld, m0 + mg * 8, p.M, x_vec, rx[j][r]);
          else {
#pragma unroll
            for (int c = 0; c < 8; ++c) rx[j][r][c] = 0.f;
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      const int u = tid + j * kWgThreads;
      if (u < GU) {
        const int ng = u % (BN / 8), kg = u / (BN / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t gr = s_gr[slot][kg * 4 + r];
          if (gr >= 0) {
            load8_f32(gb + gr * p.g_ld, n0 + ng * 8, p.N, g_vec, rg[j][r]);
            if (weighted) {
              const float w = s_w[slot][kg * 4 + r];
#pragma unroll
              for (int c = 0; c < 8; ++c) rg[j][r][c] = round_to(round_to(rg[j][r][c], OP) * w, OP);
            }
          } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) rg[j][r][c] = 0.f;
          }
        }
      }
    }
  };

  auto store_stage = [&](OpT* As, OpT* Bs) {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int u = tid + j * kWgThreads;
      if (u < XU) {
        const int mg = u % (BM / 8), kg = u / (BM / 8);
#pragma unroll
        for (int c = 0; c < 8; ++c)
          store4<OpT>(As + (mg * 8 + c) * Cfg::LDS_ROW + kg * 4, rx[j][0][c], rx[j][1][c], rx[j][2][c], rx[j][3][c]);
      }
    }
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      const int u = tid + j * kWgThreads;
      if (u < GU) {
        const int ng = u % (BN / 8), kg = u / (BN / 8);
#pragma unroll
        for (int c = 0; c < 8; ++c)
          store4<OpT>(Bs + (ng * 8 + c) * Cfg::LDS_ROW + kg * 4, rg[j][0][c], rg[j][1][c], rg[j][2][c], rg[j][3][c]);
      }
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;

  if (n_stages > 0) {
    meta_load(0);
    if (n_stages > 1) meta_load(1);
    __syncthreads();
    data_load(0);
    store_stage(As0, Bs0);
    __syncthreads();
    for (int64_t s = 0; s < n_stages; ++s) {
      const bool odd = s & 1;
      if (s + 2 < n_stages) meta_load(s + 2);
      if (s + 1 < n_stages) data_load(s + 1);
      mfma_stage<OpT, Cfg>(acc, odd ? As1 : As0, odd ? Bs1 : Bs0, wm, wn, lane);
      if (s + 1 < n_stages) store_stage(odd ? As0 : As1, odd ? Bs0 : Bs1);
      __syncthreads();
    }
  }

  // ---- epilogue: fp32 tile in LDS, then direct store or deterministic reduce ----
  float* Cs = reinterpret_cast<float*>(smem);
  acc_to_lds<Cfg>(acc, Cs, wm, wn, lane);
  __syncthreads();

  constexpr int TPR = BN / 8;
  constexpr int RPP = kWgThreads / TPR;
  const int cg = tid % TPR;
  const bool dw_vec = p.dw_sn == 1 && p.dw_dtype == kF32 && p.dw_sm % 4 == 0 && p.dw_se % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(p.dw) & 15) == 0;
  auto write_dw = [&](int r, const float (&v)[8]) {
    const int64_t m = m0 + r;
    if (m >= p.M) return;
    const int64_t nb = n0 + cg * 8;
    const int64_t off = (int64_t)expert * p.dw_se + m * p.dw_sm;
    if (dw_vec && nb + 8 <= p.N) {
      float* d = reinterpret_cast<float*>(p.dw) + off + nb;
      *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (nb + j < p.N) store_from_f32(p.dw, p.dw_dtype, off + (nb + j) * p.dw_sn, v[j]);
    }
  };

  if (nch == 1) {
    for (int r = tid / TPR; r < BM; r += RPP) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = Cs[r * Cfg::C_LD + cg * 8 + j];
      write_dw(r, v);
    }
    return;
  }

  // partial tile of this chunk -> workspace (tile-contiguous fp32), handed
  // over by the split-K protocol of cvmm_common.h (splitk_*)
  const int64_t slot = s_slot;
  if (slot >= p.max_slots) return;  // cannot happen: workspace sized for 2R/split slots
  auto pack2 = [](float a, float b) {
    return (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  };
  uint64_t* mine = reinterpret_cast<uint64_t*>(p.partial + (slot * tiles + tile) * (int64_t)(BM * BN));
  for (int r = tid / TPR; r < BM; r += RPP) {
    uint64_t* d = mine + (r * BN + cg * 8) / 2;
    const float* s = Cs + r * Cfg::C_LD + cg * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __hip_atomic_store(d + j, pack2(s[2 * j], s[2 * j + 1]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  splitk_published();
  __syncthreads();
  if (tid == 0) s_last = splitk_arrive(p.counters + (int64_t)expert * tiles + tile, nch);
  __syncthreads();
  if (!s_last) return;
  splitk_acquired();
  // this expert's slots are consecutive; add them in chunk order
  const int64_t base_slot = s_base_slot;
  for (int r = tid / TPR; r < BM; r += RPP) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int32_t c = 0; c < nch; ++c) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(
          p.partial + ((base_slot + c) * tiles + tile) * (int64_t)(BM * BN) + r * BN + cg * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t w = __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v[2 * j] += __uint_as_float((uint32_t)w);
        v[2 * j + 1] += __uint_as_float((uint32_t)(w >> 32));
      }
    }
    write_dw(r, v);
  }
}

template <typename OpT, typename XT, typename GT, int BM, int BN>
hipError_t launch_wgrad_t(const WgradParams& p, hipStream_t stream) {
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int64_t grid = p.grid_chunks * tiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL((wgrad_kernel<OpT, XT, GT, BM, BN>), dim3((unsigned)grid), dim3(kWgThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename OpT>
hipError_t launch_wgrad_op(const WgradParams& p, hipStream_t stream) {
  const int32_t op = DTypeOf<OpT>::value;
  const bool x_f32 = p.x_dtype == kF32, g_f32 = p.g_dtype == kF32;
  if (!(x_f32 || p.x_dtype == op) || !(g_f32 || p.g_dtype == op)) return hipErrorInvalidValue;
  int bm, bn;
  wgrad_tile(p.M, p.N, &bm, &bn);
#define CVMM_WG_TILES(XTy, GTy)                                                            \
  if (bm == 256) return launch_wgrad_t<OpT, XTy, GTy, 256, 64>(p, stream);                 \
  if (bm == 64) return launch_wgrad_t<OpT, XTy, GTy, 64, 256>(p, stream);                  \
  return launch_wgrad_t<OpT, XTy, GTy, 128, 128>(p, stream)
  if constexpr (DTypeOf<OpT>::value == kF32) {
    CVMM_WG_TILES(float, float);
  } else {
    if (x_f32 && g_f32) { CVMM_WG_TILES(float, float); }
    if (x_f32 && !g_f32) { CVMM_WG_TILES(float, OpT); }
    if (!x_f32 && g_f32) { CVMM_WG_TILES(OpT, float); }
    CVMM_WG_TILES(OpT, OpT);
  }
#undef CVMM_WG_TILES
}

}  // namespace cvmm
