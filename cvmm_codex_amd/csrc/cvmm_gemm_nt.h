// Routed GEMM fast path (16-bit operands, both k-contiguous): the forward reads
// x rows and the transposed bf16 weight copy [E][d_out][d_in]; the input
// gradient reads dY rows and the bf16 weight copy [E][d_in][d_out].
//
// Staging: global_load_lds (16 bytes per lane, gfx950) moves every 16-byte
// chunk straight from global memory into LDS -- no staging registers, no
// conversion.  One wave instruction fills 1 KB = 8 rows of 128 bytes (BK = 64
// 16-bit values); the lane -> chunk assignment applies the LDS swizzle
//   physical chunk = logical chunk ^ ((row & 7) ^ ((row >> 3) & 1))
// so the MFMA fragment reads (16 rows x one 16-byte chunk per lane group) hit
// distinct banks both per 8 and per 16 lanes.  Rows outside the tile, invalid
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

__device__ __forceinline__ int lds_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

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

template <typename OpT, int BM, int BN>
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

  if (!gemm_schedule<BM>(p, tile, meta)) return;
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

template <typename OpT, int BM, int BN>
hipError_t launch_routed_gemm_nt_t(const GemmParams& p, hipStream_t stream) {
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t grid = p.grid_tiles * n_ntiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL((routed_gemm_nt_kernel<OpT, BM, BN>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename OpT>
hipError_t launch_routed_gemm_nt_op(const GemmParams& p, hipStream_t stream) {
  if (p.N <= 64) return launch_routed_gemm_nt_t<OpT, 256, 64>(p, stream);
  return launch_routed_gemm_nt_t<OpT, 128, 128>(p, stream);
}

}  // namespace cvmm
