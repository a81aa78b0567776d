// Routed GEMM fast path (16-bit operands, both k-contiguous): the forward reads
// x rows and the transposed bf16 weight copy [E][d_out][d_in]; the input
// gradient reads dY rows and the bf16 weight copy [E][d_in][d_out].
//
// Staging: global_load_lds (16 bytes per lane, gfx950) moves every 16-byte
// chunk straight from global memory into LDS -- no staging registers, no
// conversion.  One wave instruction fills 1 KB = 8 rows of 128 bytes (BK = 64
// 16-bit values); the lane -> chunk assignment applies the LDS swizzle
//   physical chunk = logical chunk ^ (row & 7)
// under which the MFMA fragment reads (lane l: row l % 16, chunk l / 16) are
// bank-conflict free on gfx950 (SQ_LDS_BANK_CONFLICT = 0 in a ds_read_b128
// probe; the variant that also flips on row bit 3 measured 4 conflict cycles
// per read).  Rows outside the tile, invalid
// indices and k beyond K read a zero page.  Two LDS buffers alternate.
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_mfma.h"
#include "cvmm_gemm_common.h"

namespace cvmm {

// 4 KB of zeros in device memory (zero-initialised at load, one copy per code
// object): the source of every DMA chunk that lies outside an operand.
static __device__ uint4 g_cvmm_zero_page[256];

__device__ __forceinline__ int lds_swz(int row) { return row & 7; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <typename OpT, int BM, int BN>
struct NtCfg {
  static constexpr int BK = 64;                 // 16-bit values per LDS row (128 B)
  static constexpr int ROWB = 128;
  static constexpr int A_BYTES = BM * ROWB;
  static constexpr int B_BYTES = BN * ROWB;
  static constexpr int NA = BM / 32;            // DMA instructions per wave per stage (A)
  static constexpr int NB = BN / 32;
  static constexpr int WN = BN / 64, WM = BM / 64;
  static_assert(WM * WN == 4, "4 waves of 64x64");
  static constexpr int C_LD = BN + 4;
  static constexpr int C_HALF = BM / 2;         // epilogue rows held per stage buffer
  static constexpr int C_HALF_BYTES = C_HALF * C_LD * 4;
  static constexpr int STAGE_BYTES = (A_BYTES + B_BYTES > C_HALF_BYTES) ? A_BYTES + B_BYTES : C_HALF_BYTES;
};

template <typename OpT, int BM, int BN, int Role>
__global__ __launch_bounds__(kGemmThreads, 2) void routed_gemm_nt_kernel(const GemmParams p) {
  using Cfg = NtCfg<OpT, BM, BN>;
  // Two LDS objects (double buffer).  The loop is unrolled by two so every
  // access names its buffer statically: the compiler's wait-count pass then
  // sees that the DMA into one buffer does not alias the reads of the other
  // and keeps the DMA in flight across the MFMA work.
  __shared__ __attribute__((aligned(1024))) char stage0[Cfg::STAGE_BYTES];
  __shared__ __attribute__((aligned(1024))) char stage1[Cfg::STAGE_BYTES];
  __shared__ RouteMeta<BM> meta;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tile = id / n_ntiles;
  const int64_t ntile = id % n_ntiles;
  const int64_t n0 = ntile * BN;

  if (!gemm_schedule<BM>(p, tile, meta)) {
    zero_unrouted_cols<BM>(p, meta, tile, gridDim.x / n_ntiles, n0, n0 + BN, ntile);
    return;
  }
  const int32_t expert = meta.expert;

  // ---- per-lane DMA sources (fixed across k stages) --------------------------
  // wave instruction j covers rows 8*(wave*NA + j) .. +7; lane -> (row, physical chunk)
  const char* zero = reinterpret_cast<const char*>(g_cvmm_zero_page);
  const char* a_src[Cfg::NA];
  int a_k8[Cfg::NA];
#pragma unroll
  for (int j = 0; j < Cfg::NA; ++j) {
    const int row = 8 * (wave * Cfg::NA + j) + (lane >> 3);
    const int lc = (lane & 7) ^ lds_swz(row);
    const int64_t ar = meta.arow[row];
    a_k8[j] = lc * 8;
    a_src[j] = ar >= 0 ? reinterpret_cast<const char*>(p.a) + (ar * p.a_ld + lc * 8) * 2 : nullptr;
  }
  const char* b_src[Cfg::NB];
  int b_k8[Cfg::NB];
#pragma unroll
  for (int j = 0; j < Cfg::NB; ++j) {
    const int row = 8 * (wave * Cfg::NB + j) + (lane >> 3);
    const int lc = (lane & 7) ^ lds_swz(row);
    const int64_t gn = n0 + row;
    b_k8[j] = lc * 8;
    b_src[j] = gn < p.N ? reinterpret_cast<const char*>(p.b) + ((int64_t)expert * p.b_se + gn * p.b_sn + lc * 8) * 2
                        : nullptr;
  }

  auto issue = [&](int64_t kt, char* sa) {
    const int64_t k0 = kt * Cfg::BK;
    char* sb = sa + Cfg::A_BYTES;
#pragma unroll
    for (int j = 0; j < Cfg::NA; ++j) {
      const char* src = (a_src[j] != nullptr && k0 + a_k8[j] < p.K) ? a_src[j] + k0 * 2 : zero;
      dma16(src, sa + (wave * Cfg::NA + j) * 1024);
    }
#pragma unroll
    for (int j = 0; j < Cfg::NB; ++j) {
      const char* src = (b_src[j] != nullptr && k0 + b_k8[j] < p.K) ? b_src[j] + k0 * 2 : zero;
      dma16(src, sb + (wave * Cfg::NB + j) * 1024);
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int fr = lane & 15, fq = lane >> 4;
  // fragment byte offsets inside a stage (rows of this wave, per k-step chunk)
  int a_off[4][2], b_off[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ra = wm * 64 + i * 16 + fr;
    const int rb = wn * 64 + i * 16 + fr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + fq;
      a_off[i][ks] = ra * Cfg::ROWB + ((c ^ lds_swz(ra)) << 4);
      b_off[i][ks] = Cfg::A_BYTES + rb * Cfg::ROWB + ((c ^ lds_swz(rb)) << 4);
    }
  }

  auto compute = [&](const char* st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const uint4*>(st + a_off[i][ks]);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const uint4*>(st + b_off[j][ks]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MfmaOp<OpT>::step(acc[i][j], a[i], b[j]);
    }
  };

  const int64_t nk = (p.K + Cfg::BK - 1) / Cfg::BK;
  issue(0, stage0);
  for (int64_t kt = 0; kt < nk; kt += 2) {
    wait_vmcnt<0>();
    __syncthreads();
    if (kt + 1 < nk) issue(kt + 1, stage1);
    compute(stage0);
    if (kt + 1 >= nk) break;
    wait_vmcnt<0>();
    __syncthreads();
    if (kt + 2 < nk) issue(kt + 2, stage0);
    compute(stage1);
  }
  __syncthreads();

  // ---- accumulators -> fp32 LDS tile: rows [0, BM/2) in stage0, the rest in stage1
  float* C0 = reinterpret_cast<float*>(stage0);
  float* C1 = reinterpret_cast<float*>(stage1);
  {
    const int col = lane & 15;
    const int rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = wm * 64 + i * 16 + rq + v;
          float* C = r < Cfg::C_HALF ? C0 : C1;
          C[(r % Cfg::C_HALF) * Cfg::C_LD + wn * 64 + j * 16 + col] = acc[i][j][v];
        }
  }
  __syncthreads();
  gemm_epilogue<BM, BN, Cfg::C_LD>(p, C0, C1, Cfg::C_HALF, meta, n0, ntile);
}

// N-loop variant for small K (few k stages per tile): one workgroup walks the
// n-tiles [nt_begin, nt_end) of its m-tile as one continuous stream of
// (n-tile, k-stage) DMA stages, so the schedule, route metadata and pipeline
// ramp are paid once per m-tile instead of once per output tile.  The MFMA
// operands are swapped (C^T = W-tile x A-tile^T): each lane then holds 4
// consecutive output columns of one row and stores them straight from
// registers (8 bytes), leaving LDS to the next stage's DMA.  Plain stores only
// (no routing-weight gradient, no atomics); N % 8 == 0.
template <typename OpT, int BM, int BN, int Role>
__global__ __launch_bounds__(kGemmThreads, 2) void routed_gemm_nloop_kernel(const GemmParams p, int32_t ng) {
  using Cfg = NtCfg<OpT, BM, BN>;
  __shared__ __attribute__((aligned(1024))) char stage0[Cfg::A_BYTES + Cfg::B_BYTES];
  __shared__ __attribute__((aligned(1024))) char stage1[Cfg::A_BYTES + Cfg::B_BYTES];
  __shared__ RouteMeta<BM> meta;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t n_groups = (n_ntiles + ng - 1) / ng;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tile = id / n_groups;
  const int64_t nt_begin = (id % n_groups) * ng;
  const int64_t nt_end = nt_begin + ng < n_ntiles ? nt_begin + ng : n_ntiles;

  if (!gemm_schedule<BM>(p, tile, meta)) {
    zero_unrouted_cols<BM>(p, meta, tile, gridDim.x / n_groups, nt_begin * BN, nt_end * BN, -1);
    return;
  }
  const int32_t expert = meta.expert;

  const char* zero = reinterpret_cast<const char*>(g_cvmm_zero_page);
  const char* a_src[Cfg::NA];
  int a_k8[Cfg::NA];
#pragma unroll
  for (int j = 0; j < Cfg::NA; ++j) {
    const int row = 8 * (wave * Cfg::NA + j) + (lane >> 3);
    const int lc = (lane & 7) ^ lds_swz(row);
    const int64_t ar = meta.arow[row];
    a_k8[j] = lc * 8;
    a_src[j] = ar >= 0 ? reinterpret_cast<const char*>(p.a) + (ar * p.a_ld + lc * 8) * 2 : nullptr;
  }
  int b_row[Cfg::NB], b_lc8[Cfg::NB];
#pragma unroll
  for (int j = 0; j < Cfg::NB; ++j) {
    const int row = 8 * (wave * Cfg::NB + j) + (lane >> 3);
    b_row[j] = row;
    b_lc8[j] = ((lane & 7) ^ lds_swz(row)) * 8;
  }
  const char* b_expert = reinterpret_cast<const char*>(p.b) + (int64_t)expert * p.b_se * 2;

  const int64_t nk = (p.K + Cfg::BK - 1) / Cfg::BK;
  const int64_t n_stages = (nt_end - nt_begin) * nk;

  auto issue = [&](int64_t s, char* sa) {
    const int64_t nt = nt_begin + s / nk;
    const int64_t k0 = (s % nk) * Cfg::BK;
    char* sb = sa + Cfg::A_BYTES;
#pragma unroll
    for (int j = 0; j < Cfg::NA; ++j) {
      const char* src = (a_src[j] != nullptr && k0 + a_k8[j] < p.K) ? a_src[j] + k0 * 2 : zero;
      dma16(src, sa + (wave * Cfg::NA + j) * 1024);
    }
#pragma unroll
    for (int j = 0; j < Cfg::NB; ++j) {
      const int64_t gn = nt * BN + b_row[j];
      const char* src = (gn < p.N && k0 + b_lc8[j] < p.K) ? b_expert + (gn * p.b_sn + b_lc8[j] + k0) * 2 : zero;
      dma16(src, sb + (wave * Cfg::NB + j) * 1024);
    }
  };

  // MFMA "A" = weight rows (n), "B" = activation rows (m):  D[n][m] = C[m][n]
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int fr = lane & 15, fq = lane >> 4;
  int act_off[4][2], w_off[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ra = wm * 64 + i * 16 + fr;
    const int rb = wn * 64 + i * 16 + fr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + fq;
      act_off[i][ks] = ra * Cfg::ROWB + ((c ^ lds_swz(ra)) << 4);
      w_off[i][ks] = Cfg::A_BYTES + rb * Cfg::ROWB + ((c ^ lds_swz(rb)) << 4);
    }
  }

  // per-lane output rows (4 m-blocks) and routing weights, fixed over n-tiles
  int64_t orow[4];
  float wv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = wm * 64 + j * 16 + fr;
    orow[j] = m < meta.rows ? meta.orow[m] : -1;
    wv[j] = meta.w[m];
  }
  const bool has_w = p.w != nullptr;

  f32x4_t acc[4][4];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  auto compute = [&](const char* st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 wf[4], af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wf[i] = *reinterpret_cast<const uint4*>(st + w_off[i][ks]);
#pragma unroll
      for (int j = 0; j < 4; ++j) af[j] = *reinterpret_cast<const uint4*>(st + act_off[j][ks]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MfmaOp<OpT>::step(acc[i][j], wf[i], af[j]);
    }
  };
  // lane holds C[m = wm*64 + j*16 + fr][n = wn*64 + i*16 + 4*fq + v]
  auto store_tile = [&](int64_t nt) {
    const int64_t nbase = nt * BN + wn * 64 + 4 * fq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (orow[j] < 0) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = nbase + i * 16;
        if (n >= p.N) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float c = round_to(acc[i][j][q], p.val_dtype);
          if (has_w) {
            c = c * wv[j];
            if (p.prod_dtype >= 0) c = round_to(c, p.prod_dtype);
          }
          v[q] = c;
        }
        const int64_t off = orow[j] * p.out_ld + n;
        if (p.out_dtype == kF32) {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + off) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          union { uint2 u; bf16_t b[4]; f16_t h[4]; } pk;
          if (p.out_dtype == kBF16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) pk.b[q] = (bf16_t)v[q];
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) pk.h[q] = (f16_t)v[q];
          }
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + off) = pk.u;
        }
      }
    }
  };

  zero_acc();
  issue(0, stage0);
  for (int64_t s = 0; s < n_stages; s += 2) {
    wait_vmcnt<0>();
    __syncthreads();
    if (s + 1 < n_stages) issue(s + 1, stage1);
    compute(stage0);
    if ((s + 1) % nk == 0) {
      store_tile(nt_begin + s / nk);
      zero_acc();
    }
    if (s + 1 >= n_stages) break;
    wait_vmcnt<0>();
    __syncthreads();
    if (s + 2 < n_stages) issue(s + 2, stage0);
    compute(stage1);
    if ((s + 2) % nk == 0) {
      store_tile(nt_begin + (s + 1) / nk);
      zero_acc();
    }
  }
}

template <typename OpT, int BM, int BN>
hipError_t launch_routed_gemm_nloop_t(const GemmParams& p, int32_t ng, hipStream_t stream) {
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t n_groups = (n_ntiles + ng - 1) / ng;
  const int64_t grid = p.grid_tiles * n_groups;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.role == 0)
    hipLaunchKernelGGL((routed_gemm_nloop_kernel<OpT, BM, BN, 0>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                       stream, p, ng);
  else
    hipLaunchKernelGGL((routed_gemm_nloop_kernel<OpT, BM, BN, 1>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                       stream, p, ng);
  return hipGetLastError();
}

template <typename OpT, int BM, int BN>
hipError_t launch_routed_gemm_nt_t(const GemmParams& p_in, hipStream_t stream) {
  GemmParams p = p_in;
  p.token_major = resolve_token_major(p);
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t grid = p.grid_tiles * n_ntiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.role == 0)
    hipLaunchKernelGGL((routed_gemm_nt_kernel<OpT, BM, BN, 0>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((routed_gemm_nt_kernel<OpT, BM, BN, 1>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                       stream, p);
  return hipGetLastError();
}

template <typename OpT>
hipError_t launch_routed_gemm_nt_op(const GemmParams& p, hipStream_t stream) {
  if (p.N <= 64) return launch_routed_gemm_nt_t<OpT, 256, 64>(p, stream);
  // one k stage per tile (K <= 64): walk all n-tiles of an m-tile in one
  // workgroup (plain stores only).  Measured: switch_o forward 2.07 -> 1.51 ms;
  // with two k stages (K = 128, ff_up grad-input) the tiled kernel is faster.
  const int64_t nk = (p.K + 63) / 64;
  const int64_t n_ntiles = (p.N + 127) / 128;
  if (nk == 1 && n_ntiles > 1 && p.epi == kEpiStore && p.dg == nullptr && p.out != nullptr && p.N % 8 == 0 &&
      p.out_ld % 8 == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0)
    return launch_routed_gemm_nloop_t<OpT, 128, 128>(p, (int32_t)n_ntiles, stream);
  return launch_routed_gemm_nt_t<OpT, 128, 128>(p, stream);
}

}  // namespace cvmm
