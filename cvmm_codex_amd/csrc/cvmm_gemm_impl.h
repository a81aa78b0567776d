// Routed grouped GEMM for the CVMM forward (cvmm_kernel, cvmm.py:101-243) and
// the input gradient (cvmm_grouped_bwd_x_kernel cvmm.py:363-421,
// cvmm_weighted_route_bwd_x_kernel cvmm.py:1008-1105).
//
// Scheduling: routes are expert-sorted; expert e owns ceil(count_e / BM)
// m-tiles, so no tile straddles two experts (the reference recomputes a full
// tile per expert present in it).  Wave 0 of every workgroup finds its
// (expert, first route) with a wave-wide prefix scan over the per-expert tile
// counts read from the offsets array -- no host sync and no extra launch.
//
// Data path per K stage (128-byte LDS rows, double buffered):
//   A: BM gathered rows  -> As[m][k]   (16-byte loads, converted to the op type)
//   B: BK x BN of W_e    -> Bs[n][k]   (transposed on the way in when W is
//                                       n-contiguous, i.e. the forward)
//   4 waves x (4x4) v_mfma_f32_16x16x32_bf16 (or f16 / 4x f32 16x16x4)
// Epilogue through an fp32 LDS tile: coalesced row stores (scatter to the
// route's output row) or fp32 atomics into token rows (fused top-k combine),
// plus the optional routing-weight gradient row dot product.
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "cvmm_mfma.h"
#include "cvmm_gemm_common.h"

namespace cvmm {

enum BMode : int { kBNContig = 0, kBKContig = 1 };

template <typename OpT, typename AT, typename BT, int BM, int BN, int BMODE>
__global__ __launch_bounds__(kGemmThreads, 2) void routed_gemm_kernel(const GemmParams p) {
  using Cfg = TileCfg<OpT, BM, BN>;
  constexpr int EPC = Cfg::EPC;
  constexpr int BK = Cfg::BK;
  constexpr int KCH = Cfg::KCH;
  constexpr int UA = BM * KCH / kGemmThreads;                          // A chunks per thread
  constexpr int UBN = ((BN / 4) * KCH + kGemmThreads - 1) / kGemmThreads;  // n-contig B units
  constexpr int UBK = BN * KCH / kGemmThreads;                         // k-contig B chunks
  static_assert(UA * kGemmThreads == BM * KCH, "A tile split");
  static_assert(UBK * kGemmThreads == BN * KCH, "B tile split");

  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM];
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

  OpT* As0 = reinterpret_cast<OpT*>(smem);
  OpT* Bs0 = As0 + Cfg::A_ELEMS;
  OpT* As1 = As0 + Cfg::STAGE_ELEMS;
  OpT* Bs1 = As1 + Cfg::A_ELEMS;

  // A: gathered row pointers of this thread's chunks
  const AT* a_base = reinterpret_cast<const AT*>(p.a);
  const AT* aptr[UA];
  int a_m[UA], a_kc[UA];
#pragma unroll
  for (int j = 0; j < UA; ++j) {
    const int u = tid + j * kGemmThreads;
    a_m[j] = u / KCH;
    a_kc[j] = u % KCH;
    const int64_t ar = meta.arow[a_m[j]];
    aptr[j] = ar >= 0 ? a_base + ar * p.a_ld : nullptr;
  }
  const BT* b_e = reinterpret_cast<const BT*>(p.b) + (int64_t)expert * p.b_se;
  const bool a_vec = p.a_vec != 0;
  const bool b_vec = p.b_vec != 0;

  uint4 ra[UA];
  // k-contiguous B: one chunk per unit;  n-contiguous: EPC x 4 values per unit
  uint4 rbk[BMODE == kBKContig ? UBK : 1];
  float rbn[BMODE == kBNContig ? UBN : 1][EPC][4];

  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < UA; ++j) {
      if (aptr[j] != nullptr) ra[j] = load_chunk<OpT>(aptr[j], k0 + a_kc[j] * EPC, p.K, a_vec);
      else ra[j] = make_uint4(0, 0, 0, 0);
    }
    if constexpr (BMODE == kBKContig) {
#pragma unroll
      for (int j = 0; j < UBK; ++j) {
        const int u = tid + j * kGemmThreads;
        const int kc = u % KCH, n = u / KCH;
        const int64_t gn = n0 + n;
        if (gn < p.N) {
          const BT* row = b_e + gn * p.b_sn;
          if (p.b_sk == 1) {
            rbk[j] = load_chunk<OpT>(row, k0 + kc * EPC, p.K, b_vec);
          } else {
            float v[EPC];
#pragma unroll
            for (int i = 0; i < EPC; ++i) {
              const int64_t k = k0 + kc * EPC + i;
              v[i] = k < p.K ? to_f32(row[k * p.b_sk]) : 0.f;
            }
            rbk[j] = pack_chunk<OpT>(v);
          }
        } else {
          rbk[j] = make_uint4(0, 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < UBN; ++j) {
        const int u = tid + j * kGemmThreads;
        const int n4 = u % (BN / 4), kc = u / (BN / 4);
        if (kc < KCH) {
          const int64_t gn = n0 + n4 * 4;
#pragma unroll
          for (int i = 0; i < EPC; ++i) {
            const int64_t k = k0 + kc * EPC + i;
            const BT* src = b_e + k * p.b_sk + gn * p.b_sn;
            if (k < p.K && b_vec && gn + 4 <= p.N) {
              if constexpr (sizeof(BT) == 4) {
                const float4 v = *reinterpret_cast<const float4*>(src);
                rbn[j][i][0] = v.x; rbn[j][i][1] = v.y; rbn[j][i][2] = v.z; rbn[j][i][3] = v.w;
              } else {
                const uint2 raw = *reinterpret_cast<const uint2*>(src);
                const BT* e4 = reinterpret_cast<const BT*>(&raw);
#pragma unroll
                for (int q = 0; q < 4; ++q) rbn[j][i][q] = to_f32(e4[q]);
              }
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                rbn[j][i][q] = (k < p.K && gn + q < p.N) ? to_f32(src[q * p.b_sn]) : 0.f;
            }
          }
        }
      }
    }
  };

  auto store_stage = [&](OpT* As, OpT* Bs) {
#pragma unroll
    for (int j = 0; j < UA; ++j)
      *reinterpret_cast<uint4*>(As + a_m[j] * Cfg::LDS_ROW + a_kc[j] * EPC) = ra[j];
    if constexpr (BMODE == kBKContig) {
#pragma unroll
      for (int j = 0; j < UBK; ++j) {
        const int u = tid + j * kGemmThreads;
        const int kc = u % KCH, n = u / KCH;
        *reinterpret_cast<uint4*>(Bs + n * Cfg::LDS_ROW + kc * EPC) = rbk[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < UBN; ++j) {
        const int u = tid + j * kGemmThreads;
        const int n4 = u % (BN / 4), kc = u / (BN / 4);
        if (kc < KCH) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v[EPC];
#pragma unroll
            for (int i = 0; i < EPC; ++i) v[i] = rbn[j][i][q];
            *reinterpret_cast<uint4*>(Bs + (n4 * 4 + q) * Cfg::LDS_ROW + kc * EPC) = pack_chunk<OpT>(v);
          }
        }
      }
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int64_t nk = (p.K + BK - 1) / BK;
  load_stage(0);
  store_stage(As0, Bs0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const bool odd = kt & 1;
    if (kt + 1 < nk) load_stage((kt + 1) * BK);
    mfma_stage<OpT, Cfg>(acc, odd ? As1 : As0, odd ? Bs1 : Bs0, wm, wn, lane);
    if (kt + 1 < nk) store_stage(odd ? As0 : As1, odd ? Bs0 : Bs1);
    __syncthreads();
  }

  // ---- epilogue ----------------------------------------------------------------
  float* Cs = reinterpret_cast<float*>(smem);
  acc_to_lds<Cfg>(acc, Cs, wm, wn, lane);
  __syncthreads();

  gemm_epilogue<BM, BN, Cfg::C_LD>(p, Cs, Cs + (BM / 2) * Cfg::C_LD, BM / 2, meta, n0, ntile);
}

template <typename OpT, typename AT, typename BT, int BM, int BN>
hipError_t launch_routed_gemm_t(const GemmParams& p, hipStream_t stream) {
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t grid = p.grid_tiles * n_ntiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.b_sn == 1 || p.b_sk != 1) {
    hipLaunchKernelGGL((routed_gemm_kernel<OpT, AT, BT, BM, BN, kBNContig>), dim3((unsigned)grid),
                       dim3(kGemmThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((routed_gemm_kernel<OpT, AT, BT, BM, BN, kBKContig>), dim3((unsigned)grid),
                       dim3(kGemmThreads), 0, stream, p);
  }
  return hipGetLastError();
}

// Instantiate the supported storage combinations for one op type.
template <typename OpT>
hipError_t launch_routed_gemm_op(const GemmParams& p, hipStream_t stream) {
  const int32_t op = DTypeOf<OpT>::value;
  const bool a_f32 = p.a_dtype == kF32, b_f32 = p.b_dtype == kF32;
  if (!(a_f32 || p.a_dtype == op) || !(b_f32 || p.b_dtype == op)) return hipErrorInvalidValue;
  const bool narrow = p.N <= 64;
#define CVMM_GEMM_CASE(ATy, BTy)                                                                  \
  return narrow ? launch_routed_gemm_t<OpT, ATy, BTy, 256, 64>(p, stream)                         \
                : launch_routed_gemm_t<OpT, ATy, BTy, 128, 128>(p, stream)
  if constexpr (DTypeOf<OpT>::value == kF32) {
    CVMM_GEMM_CASE(float, float);
  } else {
    if (a_f32 && b_f32) { CVMM_GEMM_CASE(float, float); }
    if (a_f32 && !b_f32) { CVMM_GEMM_CASE(float, OpT); }
    if (!a_f32 && b_f32) { CVMM_GEMM_CASE(OpT, float); }
    CVMM_GEMM_CASE(OpT, OpT);
  }
#undef CVMM_GEMM_CASE
}

}  // namespace cvmm
