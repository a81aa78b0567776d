// Weight gradient fast path (16-bit operands, gfx950).
//
// dW[e] = X_e^T G_e reduces over the expert's routes, and both operands are
// route-major rows (x rows and dY rows).  Each LDS stage holds 64 routes of
// both operands in their natural layout -- [route][m] and [route][n] -- moved
// by global_load_lds DMA (16 bytes per lane, rows gathered by route index).
// The MFMA fragments need 8 consecutive routes per lane, which
// ds_read_b64_tr_b16 provides directly: within each 16-lane group, lane L
// points at route k0 + L/4, column c0 + 4*(L%4); lane i then receives the 4
// values of column c0 + i for routes k0..k0+3.  Two such reads give the 8
// routes of a 16x16x32 operand fragment.  So there are no transposing LDS
// writes (the bank-conflict bottleneck of the general kernel).
//
// LDS rows of 256 B (128 columns) are swizzled at 16-byte granularity,
//   physical chunk = chunk ^ (2 * ((row & 3) | (((row >> 3) & 1) << 2))),
// keeping each 32-byte read segment whole and spreading the 16 routes one
// transpose read touches over distinct banks.  128-byte rows (64 columns) use
//   chunk ^ (2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1))).
//
// Weighted gradients scale dY rows by their routing weight (rounded to the op
// type at the same points as cvmm.py:590-599); those rows go through registers
// instead of DMA so the scale is applied before they reach LDS.
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_mfma.h"

namespace cvmm {

static __device__ uint4 g_cvmm_wg_zero_page[256];

template <int N>
__device__ __forceinline__ void wg_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wg_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

typedef short wg_v4i16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint2 ds_read_tr16(const char* p) {
  wg_v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) wg_v4i16*)p);
  return __builtin_bit_cast(uint2, v);
}

// k-major operand tile: 64 route rows of COLS 16-bit values.
template <int COLS>
struct KmTile {
  static constexpr int ROWB = COLS * 2;
  static constexpr int CPR = COLS / 8;           // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;           // rows per 1 KB DMA instruction
  static constexpr int INSTS = 64 / RPI;         // DMA instructions per stage
  static constexpr int PER_WAVE = INSTS / 4;
  static constexpr int BYTES = 64 * ROWB;
  static_assert(CPR == 8 || CPR == 16 || CPR == 32, "64, 128 or 256 columns");
  __device__ static __forceinline__ int swz(int row) {
    if constexpr (CPR >= 16) return 2 * ((row & 3) | (((row >> 3) & 1) << 2));
    else return 2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1));
  }
  // byte offset of (row, 16-bit column col) with col % 4 == 0
  __device__ static __forceinline__ int off(int row, int col) {
    const int c = col >> 3;
    return row * ROWB + ((c ^ swz(row)) << 4) + ((col & 7) << 1);
  }
};

template <typename OpT, int BM, int BN>
struct Wg2Cfg {
  using TA = KmTile<BM>;
  using TB = KmTile<BN>;
  static constexpr int STAGE = TA::BYTES + TB::BYTES;
  static constexpr int WN = BN / 64, WM = BM / 64;
  static_assert(WM * WN == 4, "4 waves of 64x64");
  static constexpr int C_LD = BN + 4;
  static constexpr int C_HALF = BM / 2;
  static constexpr int C_HALF_BYTES = C_HALF * C_LD * 4;
  static constexpr int STAGE_BYTES = STAGE > C_HALF_BYTES ? STAGE : C_HALF_BYTES;
  // weighted dY rows through registers: 16-byte chunks per thread per stage
  static constexpr int GCH = 64 * TB::CPR / 256;
};

template <typename OpT, int BM, int BN, bool WEIGHTED>
__global__ __launch_bounds__(256, 2) void wgrad_v2_kernel(const WgradParams p) {
  using Cfg = Wg2Cfg<OpT, BM, BN>;
  using TA = typename Cfg::TA;
  using TB = typename Cfg::TB;
  constexpr int OP = DTypeOf<OpT>::value;
  __shared__ __attribute__((aligned(1024))) char stage0[Cfg::STAGE_BYTES];
  __shared__ __attribute__((aligned(1024))) char stage1[Cfg::STAGE_BYTES];
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

  // ---- schedule: (expert, route chunk) of this slot (as in the general kernel)
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
        if (nch < 1) nch = 1;
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
  const int64_t n_stages = (hi - lo + 63) / 64;

  const char* zero = reinterpret_cast<const char*>(g_cvmm_wg_zero_page);
  const char* xb = reinterpret_cast<const char*>(p.x);
  const char* gb = reinterpret_cast<const char*>(p.g);

  // ---- per-lane DMA geometry: instruction j of this wave -> (row, logical chunk)
  int a_row[TA::PER_WAVE], a_col[TA::PER_WAVE];
#pragma unroll
  for (int j = 0; j < TA::PER_WAVE; ++j) {
    const int row = (wave * TA::PER_WAVE + j) * TA::RPI + lane / TA::CPR;
    a_row[j] = row;
    a_col[j] = (((lane % TA::CPR) ^ TA::swz(row)) * 8);
  }
  int b_row[TB::PER_WAVE], b_col[TB::PER_WAVE];
#pragma unroll
  for (int j = 0; j < TB::PER_WAVE; ++j) {
    const int row = (wave * TB::PER_WAVE + j) * TB::RPI + lane / TB::CPR;
    b_row[j] = row;
    b_col[j] = (((lane % TB::CPR) ^ TB::swz(row)) * 8);
  }

  // Route rows of a stage: lane t of every wave resolves route lo + 64*stage + t
  // (coalesced index loads, one division per route); DMA lanes then fetch the
  // row of the route they copy with a cross-lane shuffle.  -1 = no route.
  // Row indices fit int32 (the C ABI rejects more than 2^31 - 1 routes).
  struct StageRoutes {
    int32_t xr, gr;
    float w;
  };
  auto load_routes = [&](int64_t stage, StageRoutes& sr) {
    const int64_t q = lo + stage * 64 + lane;
    sr.xr = -1;
    sr.gr = -1;
    sr.w = 0.f;
    if (q < hi) {
      const int64_t xi = p.x_idx[q];
      const int64_t graw = p.g_idx[q];
      const int64_t gi = (graw >= 0 && graw < 0x7fffffffll) ? p.g_fdiv.div(graw) : -1;
      if (xi >= 0 && xi < p.x_rows && gi >= 0 && gi < p.g_rows) {
        sr.xr = (int32_t)xi;
        sr.gr = (int32_t)gi;
        if constexpr (WEIGHTED) {
          const int64_t wi = p.w_idx[q];
          sr.w = (wi >= 0 && wi < p.n_routes) ? round_to(load_as_f32(p.w, p.w_dtype, wi), OP) : 0.f;
        }
      }
    }
  };

  constexpr int GCH = WEIGHTED ? Cfg::GCH : 1;
  uint4 g_val[GCH];
  float g_w[GCH];

  auto issue = [&](const StageRoutes& sr, char* st) {
#pragma unroll
    for (int j = 0; j < TA::PER_WAVE; ++j) {
      const int32_t xr = __shfl(sr.xr, a_row[j], 64);
      const int64_t col = m0 + a_col[j];
      const char* src = (xr >= 0 && col < p.M) ? xb + ((int64_t)xr * p.x_ld + col) * 2 : zero;
      wg_dma16(src, st + (wave * TA::PER_WAVE + j) * 1024);
    }
    if constexpr (!WEIGHTED) {
#pragma unroll
      for (int j = 0; j < TB::PER_WAVE; ++j) {
        const int32_t gr = __shfl(sr.gr, b_row[j], 64);
        const int64_t col = n0 + b_col[j];
        const char* src = (gr >= 0 && col < p.N) ? gb + ((int64_t)gr * p.g_ld + col) * 2 : zero;
        wg_dma16(src, st + TA::BYTES + (wave * TB::PER_WAVE + j) * 1024);
      }
    }
  };

  // weighted dY: global -> registers (issued with the DMA), scaled into LDS after the MFMAs
  auto g_load = [&](const StageRoutes& sr) {
    if constexpr (WEIGHTED) {
#pragma unroll
      for (int j = 0; j < GCH; ++j) {
        const int u = tid + j * 256;
        const int row = u / TB::CPR;
        const int32_t gr = __shfl(sr.gr, row, 64);
        g_w[j] = __shfl(sr.w, row, 64);
        const int64_t col = n0 + (u % TB::CPR) * 8;
        g_val[j] = (gr >= 0 && col < p.N) ? *reinterpret_cast<const uint4*>(gb + ((int64_t)gr * p.g_ld + col) * 2)
                                          : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto g_store = [&](char* st) {
    if constexpr (WEIGHTED) {
#pragma unroll
      for (int j = 0; j < GCH; ++j) {
        const int u = tid + j * 256;
        Chunk16 c;
        c.u = g_val[j];
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = round_to(to_f32(reinterpret_cast<const OpT*>(&c)[q]) * g_w[j], OP);
        *reinterpret_cast<uint4*>(st + TA::BYTES + TB::off(u / TB::CPR, (u % TB::CPR) * 8)) = pack_chunk<OpT>(v);
      }
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int L = lane & 15, grp = lane >> 4;
  // A lane reads route row ks*32 + grp*8 + h*4 + L/4, columns blk*16 + 4*(L%4).
  // The swizzle only sees row bits 0-1 (from L) and bit 3 (grp & 1), so it is a
  // per-lane constant; (ks, h) become immediate offsets.
  const int trow = grp * 8 + (L >> 2);
  const int lane_lo = ((L & 1) << 3) + (((L >> 1) & 1) << 4);
  const int a_base = trow * TA::ROWB + lane_lo;
  const int b_base = TA::BYTES + trow * TB::ROWB + lane_lo;
  int a_chunk[4], b_chunk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a_chunk[i] = (((wm * 8 + 2 * i) ^ TA::swz(trow)) << 4);
    b_chunk[i] = (((wn * 8 + 2 * i) ^ TB::swz(trow)) << 4);
  }

  auto compute = [&](const char* st) {
    const char* pa = st + a_base;
    const char* pb = st + b_base;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 lo2 = ds_read_tr16(pa + a_chunk[i] + (ks * 32) * TA::ROWB);
        const uint2 hi2 = ds_read_tr16(pa + a_chunk[i] + (ks * 32 + 4) * TA::ROWB);
        a[i] = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint2 lo2 = ds_read_tr16(pb + b_chunk[j] + (ks * 32) * TB::ROWB);
        const uint2 hi2 = ds_read_tr16(pb + b_chunk[j] + (ks * 32 + 4) * TB::ROWB);
        b[j] = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MfmaOp<OpT>::step(acc[i][j], a[i], b[j]);
    }
  };

  if (n_stages > 0) {
    StageRoutes r_cur, r_nxt;
    load_routes(0, r_cur);
    wg_wait_vmcnt<0>();
    issue(r_cur, stage0);
    g_load(r_cur);
    if (n_stages > 1) load_routes(1, r_nxt);
    wg_wait_vmcnt<0>();
    g_store(stage0);
    for (int64_t s = 0; s < n_stages; s += 2) {
      // ---- even stage: read stage0, fill stage1 (routes in r_nxt)
      wg_wait_vmcnt<0>();
      __syncthreads();
      if (s + 1 < n_stages) {
        issue(r_nxt, stage1);
        g_load(r_nxt);
      }
      if (s + 2 < n_stages) load_routes(s + 2, r_cur);
      compute(stage0);
      if (s + 1 >= n_stages) break;
      if constexpr (WEIGHTED) {
        wg_wait_vmcnt<0>();
        g_store(stage1);
      }
      // ---- odd stage: read stage1, fill stage0 (routes in r_cur)
      wg_wait_vmcnt<0>();
      __syncthreads();
      if (s + 2 < n_stages) {
        issue(r_cur, stage0);
        g_load(r_cur);
      }
      if (s + 3 < n_stages) load_routes(s + 3, r_nxt);
      compute(stage1);
      if constexpr (WEIGHTED) {
        if (s + 2 < n_stages) {
          wg_wait_vmcnt<0>();
          g_store(stage0);
        }
      }
    }
  }
  __syncthreads();

  // ---- accumulators -> fp32 LDS tile (rows [0, BM/2) in stage0, rest in stage1)
  float* C0 = reinterpret_cast<float*>(stage0);
  float* C1 = reinterpret_cast<float*>(stage1);
  auto crow = [&](int r) { return (r < Cfg::C_HALF ? C0 : C1) + (r % Cfg::C_HALF) * Cfg::C_LD; };
  {
    const int col = lane & 15;
    const int rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) crow(wm * 64 + i * 16 + rq + v)[wn * 64 + j * 16 + col] = acc[i][j][v];
  }
  __syncthreads();

  constexpr int TPR = BN / 8;
  constexpr int RPP = 256 / TPR;
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
      const float* src = crow(r) + cg * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = src[j];
      write_dw(r, v);
    }
    return;
  }

  // multi-chunk expert: fp32 partial -> workspace, last arriver sums in chunk order
  const int64_t slot = s_slot;
  if (slot >= p.max_slots) return;  // cannot happen: workspace holds 2R/split + 1 slots
  float* mine = p.partial + (slot * tiles + tile) * (int64_t)(BM * BN);
  for (int r = tid / TPR; r < BM; r += RPP) {
    float* d = mine + r * BN + cg * 8;
    const float* src = crow(r) + cg * 8;
    *reinterpret_cast<float4*>(d) = make_float4(src[0], src[1], src[2], src[3]);
    *reinterpret_cast<float4*>(d + 4) = make_float4(src[4], src[5], src[6], src[7]);
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    int32_t* ctr = p.counters + (int64_t)expert * tiles + tile;
    const int32_t prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == nch - 1);
    if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int64_t base_slot = s_base_slot;
  for (int r = tid / TPR; r < BM; r += RPP) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int32_t c = 0; c < nch; ++c) {
      const float* src = p.partial + ((base_slot + c) * tiles + tile) * (int64_t)(BM * BN) + r * BN + cg * 8;
      const float4 a = *reinterpret_cast<const float4*>(src);
      const float4 b = *reinterpret_cast<const float4*>(src + 4);
      v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
      v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
    }
    write_dw(r, v);
  }
}

template <typename OpT, int BM, int BN>
hipError_t launch_wgrad_v2_t(const WgradParams& p, hipStream_t stream) {
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int64_t grid = p.grid_chunks * tiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.w != nullptr)
    hipLaunchKernelGGL((wgrad_v2_kernel<OpT, BM, BN, true>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((wgrad_v2_kernel<OpT, BM, BN, false>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <typename OpT>
hipError_t launch_wgrad_v2_op(const WgradParams& p, hipStream_t stream) {
  int bm, bn;
  wgrad_tile(p.M, p.N, &bm, &bn);
  if (bm == 256) return launch_wgrad_v2_t<OpT, 256, 64>(p, stream);
  if (bm == 64) return launch_wgrad_v2_t<OpT, 64, 256>(p, stream);
  return launch_wgrad_v2_t<OpT, 128, 128>(p, stream);
}

}  // namespace cvmm
