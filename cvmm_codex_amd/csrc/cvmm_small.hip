// Small fp32 problems (C1-sized: a few thousand routes): the routed product
// (cvmm_kernel, cvmm.py:101-243, and the grad-input orientation,
// cvmm.py:363-421) and the weight gradient (cvmm.py:481-538) with tiles small
// enough to put a workgroup on most CUs.  The MFMA kernels' 256x64 / 128x128
// tiles give such a problem a few dozen workgroups, each a long dependent
// K loop; here a workgroup owns 16 routes x 64 columns (or a 64 x 64 block of
// one expert's weight gradient) and plain fp32 FMAs do the arithmetic, which
// at these sizes waits on loads, not on the ALUs.
//
// Routed product: thread (row tid / 16, columns 4 (tid % 16) + [0, 4)) sums
// over k in 64-wide chunks staged in LDS, up to four chunks loaded in one
// round (A rows gathered through the route index, B from the expert's matrix
// in either orientation); the products are
// stored as the routed GEMM stores them (rounded to val_dtype, per-route
// output rows), and the workgroups past the last m-tile zero the rows of
// out-of-range routes as there.
//
// Weight gradient: one workgroup per (expert, 64-row block of d_in, 64-column
// block of d_out), thread owning a 4 x 4 block; the expert's routes are
// staged 128 at a time (their indices, then all their rows' loads in one
// round) and summed in their sorted order, so every launch gives the same
// bits.  Where those blocks number fewer than the CUs, 32 x 32 blocks with
// each round's routes split over the four waves (wgrad_small32_kernel).
#include "cvmm_gemm_common.h"

namespace cvmm {

constexpr int kSmBM = 16, kSmBN = 64, kSmBK = 64;

// VEC: 16-byte loads (16-byte aligned operands, row strides and K, N
// multiples of 4).  The expert's weight chunk of the first round is loaded
// as soon as the tile's expert is known, before the route rows' metadata
// (whose loads the activation loads wait for).
template <int KC, bool VEC>
__global__ __launch_bounds__(256) void routed_small_kernel(const GemmParams p) {
  // KC chunks of 64 k in LDS at once: their loads are issued together
  __shared__ __attribute__((aligned(16))) float As[kSmBM][KC * kSmBK];  // float4 stores
  __shared__ __attribute__((aligned(16))) float Bs[KC * kSmBK][kSmBN + 4];  // rows padded: k-major fills
  __shared__ RouteMeta<kSmBM> meta;
  const int tid = threadIdx.x;
  const int64_t n_ntiles = (p.N + kSmBN - 1) / kSmBN;
  const int64_t tile = blockIdx.x / n_ntiles;
  const int64_t n0 = (blockIdx.x % n_ntiles) * kSmBN;
  const int64_t m_tiles = gridDim.x / n_ntiles;
  if (!gemm_schedule_tile<kSmBM>(p, tile, meta)) {
    zero_unrouted_cols<kSmBM>(p, meta, tile, m_tiles, n0, n0 + kSmBN, -1);
    return;
  }
  const int64_t e = meta.expert;
  const float* a = static_cast<const float*>(p.a);
  const float* b = static_cast<const float*>(p.b) + e * p.b_se;
  const int tm = tid >> 4, tn = (tid & 15) * 4;
  const bool k_unit = p.b_sk == 1 && p.b_sn != 1;
  // B chunk c of round k0: 64 k x 64 n, consecutive threads along the
  // matrix's unit-stride dimension (VEC: 4 values of it per thread)
  constexpr int NB = VEC ? 4 : 16;  // loads per thread per chunk
  float4 bv[KC][NB / (VEC ? 1 : 4)];
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = tid + i * 256;  // 1024 pieces of 4
          const int kk = k_unit ? (idx & 15) * 4 : (idx >> 4);
          const int nn = k_unit ? (idx >> 4) : (idx & 15) * 4;
          const int64_t k = k0 + c * kSmBK + kk, n = n0 + nn;
          bv[c][i] = (k < p.K && n < p.N) ? *reinterpret_cast<const float4*>(b + k * p.b_sk + n * p.b_sn)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int idx = tid + i * 256;
          const int kk = k_unit ? (idx & 63) : (idx >> 6);
          const int nn = k_unit ? (idx >> 6) : (idx & 63);
          const int64_t k = k0 + c * kSmBK + kk, n = n0 + nn;
          reinterpret_cast<float*>(&bv[c][0])[i] = (k < p.K && n < p.N) ? b[k * p.b_sk + n * p.b_sn] : 0.f;
        }
      }
    }
  };
  auto store_b = [&]() {
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = tid + i * 256;
          if (k_unit) {
            const int kk = (idx & 15) * 4, nn = idx >> 4;
            Bs[c * kSmBK + kk][nn] = bv[c][i].x;
            Bs[c * kSmBK + kk + 1][nn] = bv[c][i].y;
            Bs[c * kSmBK + kk + 2][nn] = bv[c][i].z;
            Bs[c * kSmBK + kk + 3][nn] = bv[c][i].w;
          } else {
            *reinterpret_cast<float4*>(&Bs[c * kSmBK + (idx >> 4)][(idx & 15) * 4]) = bv[c][i];
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int idx = tid + i * 256;
          const int kk = k_unit ? (idx & 63) : (idx >> 6);
          const int nn = k_unit ? (idx >> 6) : (idx & 63);
          Bs[c * kSmBK + kk][nn] = reinterpret_cast<const float*>(&bv[c][0])[i];
        }
      }
    }
  };
  load_b(0);
  gemm_route_meta<kSmBM>(p, meta);
  const int64_t ar = meta.arow[tm];  // A: thread (row tm, k 4 (tid % 16) + 64 c + [0, 4))
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 0; k0 < p.K; k0 += KC * kSmBK) {
    if (k0 > 0) load_b(k0);
    float4 av[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int64_t k = k0 + c * kSmBK + tn;
      if constexpr (VEC) {
        av[c] = (ar >= 0 && k < p.K) ? *reinterpret_cast<const float4*>(a + ar * p.a_ld + k)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float* v = reinterpret_cast<float*>(&av[c]);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (ar >= 0 && k + q < p.K) ? a[ar * p.a_ld + k + q] : 0.f;
      }
    }
#pragma unroll
    for (int c = 0; c < KC; ++c) *reinterpret_cast<float4*>(&As[tm][c * kSmBK + tn]) = av[c];
    store_b();
    __syncthreads();
#pragma unroll 8
    for (int k = 0; k < KC * kSmBK; ++k) {
      const float x = As[tm][k];
      const float4 w = *reinterpret_cast<const float4*>(&Bs[k][tn]);
      acc[0] += x * w.x;
      acc[1] += x * w.y;
      acc[2] += x * w.z;
      acc[3] += x * w.w;
    }
    __syncthreads();
  }
  const int64_t orow = meta.orow[tm];
  if (orow < 0) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t n = n0 + tn + q;
    if (n < p.N) store_from_f32(p.out, p.out_dtype, orow * p.out_ld + n, round_to(acc[q], p.val_dtype));
  }
}

// routes of one expert staged per round: their indices, then all their rows'
// loads issued together
constexpr int kSmRoutes = 128;

__global__ __launch_bounds__(256) void wgrad_small_kernel(const WgradParams p) {
  __shared__ __attribute__((aligned(16))) float Xs[kSmRoutes][64];
  __shared__ __attribute__((aligned(16))) float Gs[kSmRoutes][64];
  __shared__ int64_t s_x[kSmRoutes], s_g[kSmRoutes];
  const int tid = threadIdx.x;
  const int64_t n_mb = (p.M + 63) / 64, n_nb = (p.N + 63) / 64;
  const int64_t e = blockIdx.x / (n_mb * n_nb);
  const int64_t blk = blockIdx.x % (n_mb * n_nb);
  const int64_t m0 = (blk / n_nb) * 64, n0 = (blk % n_nb) * 64;
  int64_t lo = e > 0 ? p.offsets[e - 1] : 0, hi = p.offsets[e];
  lo = lo < 0 ? 0 : (lo > p.n_routes ? p.n_routes : lo);
  hi = hi < lo ? lo : (hi > p.n_routes ? p.n_routes : hi);
  const float* x = static_cast<const float*>(p.x);
  const float* g = static_cast<const float*>(p.g);
  const int tm = (tid >> 4) * 4, tn = (tid & 15) * 4;
  float acc[4][4] = {};
  for (int64_t q0 = lo; q0 < hi; q0 += kSmRoutes) {
    if (tid < kSmRoutes) {
      const int64_t q = q0 + tid;
      int64_t xr = -1, gr = -1;
      if (q < hi) {
        const int64_t xi = p.x_idx[q], gi = p.g_idx[q] / p.g_div;
        if (xi >= 0 && xi < p.x_rows && gi >= 0 && gi < p.g_rows) {
          xr = xi;
          gr = gi;
        }
      }
      s_x[tid] = xr;
      s_g[tid] = gr;
    }
    __syncthreads();
    const int nr = (int)((hi - q0) < kSmRoutes ? (hi - q0) : kSmRoutes);
    constexpr int kPer = kSmRoutes * 64 / 256;  // values per thread of each operand
    float xv[kPer], gv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + i * 256, r = idx >> 6, c = idx & 63;
      const int64_t xr = s_x[r], gr = s_g[r];
      xv[i] = (xr >= 0 && m0 + c < p.M) ? x[xr * p.x_ld + m0 + c] : 0.f;
      gv[i] = (gr >= 0 && n0 + c < p.N) ? g[gr * p.g_ld + n0 + c] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + i * 256, r = idx >> 6, c = idx & 63;
      Xs[r][c] = xv[i];
      Gs[r][c] = gv[i];
    }
    __syncthreads();
    for (int r = 0; r < nr; ++r) {
      const float4 xq = *reinterpret_cast<const float4*>(&Xs[r][tm]);
      const float4 gq = *reinterpret_cast<const float4*>(&Gs[r][tn]);
      const float xa[4] = {xq.x, xq.y, xq.z, xq.w}, ga[4] = {gq.x, gq.y, gq.z, gq.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += xa[i] * ga[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + tm + i, n = n0 + tn + j;
      if (m < p.M && n < p.N) store_from_f32(p.dw, p.dw_dtype, e * p.dw_se + m * p.dw_sm + n * p.dw_sn, acc[i][j]);
    }
}

// The weight gradient in 32 x 32 blocks, for problems whose 64 x 64 blocks
// would leave most CUs idle (fewer blocks than CUs): four times the
// workgroups, and the routes of each round split into contiguous quarters,
// one per wave, every lane keeping a 4 x 4 block of its wave's sums.  The
// four partial blocks are added in wave order at the end, so every launch
// gives the same bits.  VEC: 16-byte loads of the staged rows (aligned rows,
// M and N multiples of 4).
constexpr int kSm32Routes = 256;

template <bool VEC>
__global__ __launch_bounds__(256) void wgrad_small32_kernel(const WgradParams p) {
  __shared__ __attribute__((aligned(16))) float Xs[kSm32Routes][32];
  __shared__ __attribute__((aligned(16))) float Gs[kSm32Routes][32];
  __shared__ int64_t s_x[kSm32Routes], s_g[kSm32Routes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n_mb = (p.M + 31) / 32, n_nb = (p.N + 31) / 32;
  const int64_t e = blockIdx.x / (n_mb * n_nb);
  const int64_t blk = blockIdx.x % (n_mb * n_nb);
  const int64_t m0 = (blk / n_nb) * 32, n0 = (blk % n_nb) * 32;
  int64_t lo = e > 0 ? p.offsets[e - 1] : 0, hi = p.offsets[e];
  lo = lo < 0 ? 0 : (lo > p.n_routes ? p.n_routes : lo);
  hi = hi < lo ? lo : (hi > p.n_routes ? p.n_routes : hi);
  const float* x = static_cast<const float*>(p.x);
  const float* g = static_cast<const float*>(p.g);
  const int tm = (lane >> 3) * 4, tn = (lane & 7) * 4;
  float acc[4][4] = {};
  for (int64_t q0 = lo; q0 < hi; q0 += kSm32Routes) {
    {
      const int64_t q = q0 + tid;
      int64_t xr = -1, gr = -1;
      if (q < hi) {
        const int64_t xi = p.x_idx[q], gi = p.g_idx[q] / p.g_div;
        if (xi >= 0 && xi < p.x_rows && gi >= 0 && gi < p.g_rows) {
          xr = xi;
          gr = gi;
        }
      }
      s_x[tid] = xr;
      s_g[tid] = gr;
    }
    __syncthreads();
    const int nr = (int)((hi - q0) < kSm32Routes ? (hi - q0) : kSm32Routes);
    if constexpr (VEC) {
      // row r = idx / 8, columns 4 (idx % 8) + [0, 4)
      constexpr int kPer = kSm32Routes * 8 / 256;
      float4 xv[kPer], gv[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256, r = idx >> 3, c = (idx & 7) * 4;
        const int64_t xr = s_x[r], gr = s_g[r];
        // (a zero rvalue, not a named one: a select between the load and a
        // local object would make it a generic-address load)
        xv[i] = (xr >= 0 && m0 + c < p.M) ? *reinterpret_cast<const float4*>(x + xr * p.x_ld + m0 + c)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
        gv[i] = (gr >= 0 && n0 + c < p.N) ? *reinterpret_cast<const float4*>(g + gr * p.g_ld + n0 + c)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256, r = idx >> 3, c = (idx & 7) * 4;
        *reinterpret_cast<float4*>(&Xs[r][c]) = xv[i];
        *reinterpret_cast<float4*>(&Gs[r][c]) = gv[i];
      }
    } else {
      // one operand at a time (32 values per thread in flight)
      constexpr int kPer = kSm32Routes * 32 / 256;
      float v[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256, r = idx >> 5, c = idx & 31;
        const int64_t xr = s_x[r];
        v[i] = (xr >= 0 && m0 + c < p.M) ? x[xr * p.x_ld + m0 + c] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256;
        Xs[idx >> 5][idx & 31] = v[i];
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256, r = idx >> 5, c = idx & 31;
        const int64_t gr = s_g[r];
        v[i] = (gr >= 0 && n0 + c < p.N) ? g[gr * p.g_ld + n0 + c] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * 256;
        Gs[idx >> 5][idx & 31] = v[i];
      }
    }
    __syncthreads();
    const int qn = (nr + 3) / 4;
    const int r0 = wave * qn, r1 = (r0 + qn) < nr ? (r0 + qn) : nr;
#pragma unroll 4
    for (int r = r0; r < r1; ++r) {
      const float4 xq = *reinterpret_cast<const float4*>(&Xs[r][tm]);
      const float4 gq = *reinterpret_cast<const float4*>(&Gs[r][tn]);
      const float xa[4] = {xq.x, xq.y, xq.z, xq.w}, ga[4] = {gq.x, gq.y, gq.z, gq.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += xa[i] * ga[j];
    }
    __syncthreads();
  }
  // the four waves' partial blocks (16 KB, in the staging area), summed in
  // wave order
  float* part = &Xs[0][0];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<float4*>(part + wave * 1024 + (tm + i) * 32 + tn) =
        make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
  __syncthreads();
#pragma unroll
  for (int o = tid; o < 1024; o += 256) {
    const int64_t m = m0 + (o >> 5), n = n0 + (o & 31);
    float s = part[o];
    s += part[1024 + o];
    s += part[2048 + o];
    s += part[3072 + o];
    if (m < p.M && n < p.N) store_from_f32(p.dw, p.dw_dtype, e * p.dw_se + m * p.dw_sm + n * p.dw_sn, s);
  }
}

// ---------------------------------------------------------------------------
// eligibility and launchers
// ---------------------------------------------------------------------------
// fp32 storage and op, plain stores (no routing weight, no routing-weight
// gradient, no activation), and few enough outputs that the MFMA kernels'
// tiles would leave most CUs idle.
bool small_gemm_eligible(const GemmParams& p, int32_t op) {
  return op == kF32 && p.a_dtype == kF32 && p.b_dtype == kF32 && p.epi == kEpiStore && p.w == nullptr &&
         p.dg == nullptr && p.act == 0 && p.out != nullptr && p.n_routes * p.N <= (1ll << 20) &&
         p.n_routes <= (1ll << 20);
}

hipError_t launch_routed_small(const GemmParams& p, hipStream_t stream) {
  const int64_t m_tiles = (p.n_routes + kSmBM - 1) / kSmBM + (p.n_experts < p.n_routes ? p.n_experts : p.n_routes);
  const int64_t grid = m_tiles * ((p.N + kSmBN - 1) / kSmBN);
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  // 16-byte loads: aligned operands, and the unit-stride dimension of each
  // (k of A; k or n of B) a multiple of 4 in extent and in the other strides
  const bool k_unit = p.b_sk == 1 && p.b_sn != 1;
  const bool vec = (reinterpret_cast<uintptr_t>(p.a) % 16) == 0 && (reinterpret_cast<uintptr_t>(p.b) % 16) == 0 &&
                   p.a_ld % 4 == 0 && p.K % 4 == 0 && p.b_se % 4 == 0 &&
                   (k_unit ? p.b_sn % 4 == 0 : (p.b_sn == 1 && p.b_sk % 4 == 0 && p.N % 4 == 0));
  // every k chunk of a short K in one round of loads (K <= 256), else
  // rounds of four chunks
#define CVMM_SMALL(KC)                                                                                    \
  do {                                                                                                    \
    if (vec) hipLaunchKernelGGL((routed_small_kernel<KC, true>), dim3((unsigned)grid), dim3(256), 0, stream, p); \
    else hipLaunchKernelGGL((routed_small_kernel<KC, false>), dim3((unsigned)grid), dim3(256), 0, stream, p);    \
  } while (0)
  if (p.K <= kSmBK) CVMM_SMALL(1);
  else if (p.K <= 2 * kSmBK) CVMM_SMALL(2);
  else CVMM_SMALL(4);
#undef CVMM_SMALL
  return hipGetLastError();
}

// fp32, unweighted, and a small problem: each workgroup loops over one
// expert's routes, so the routes per expert stay bounded too.
bool small_wgrad_eligible(const WgradParams& p, int32_t op) {
  return op == kF32 && p.x_dtype == kF32 && p.g_dtype == kF32 && p.w == nullptr && p.n_routes <= 32768 &&
         p.M * p.N <= (1ll << 20);
}

hipError_t launch_wgrad_small(const WgradParams& p, hipStream_t stream) {
  const int64_t grid = (int64_t)p.n_experts * ((p.M + 63) / 64) * ((p.N + 63) / 64);
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (grid < 256) {
    // fewer 64 x 64 blocks than CUs: 32 x 32 blocks, routes split over waves
    const int64_t grid32 = (int64_t)p.n_experts * ((p.M + 31) / 32) * ((p.N + 31) / 32);
    const bool vec = (reinterpret_cast<uintptr_t>(p.x) % 16) == 0 && (reinterpret_cast<uintptr_t>(p.g) % 16) == 0 &&
                     p.x_ld % 4 == 0 && p.g_ld % 4 == 0 && p.M % 4 == 0 && p.N % 4 == 0;
    if (vec) hipLaunchKernelGGL(wgrad_small32_kernel<true>, dim3((unsigned)grid32), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(wgrad_small32_kernel<false>, dim3((unsigned)grid32), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(wgrad_small_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace cvmm
