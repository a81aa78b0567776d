// Routed GEMM with a DMA ring for a long inner dimension (K > 128, 16-bit
// operands): the ff_up forward (K = d_in = 1024, N = 128), the ff_down input
// gradient (K = 1024, N = 128), the SwitchHead V forward / O input gradient
// (K = 2048, N = 64) and both FFN-stack projections (K = 2048 / 512, N = 512
// / 2048).  A workgroup is four waves (one 128- or 160-row tile of 128
// columns, or 256 x 64) or eight (256 x 256).
//
// The k loop streams slices (BK = 64 or 32 values of k for every A row and B
// row of the tile) through a ring of STAGES LDS buffers, STAGES - 1 of them
// in flight:
//  * wait for the next slice with a constant vmcnt: only DMA is in flight in
//    the loop, D instructions per slice and lane, retiring in order;
//  * one barrier, then the buffer every wave has finished reading is refilled;
//  * MFMA with operands swapped (C^T = W x A^T) so that a lane ends with 4
//    consecutive output columns of one row; two lane swaps make that 8
//    columns, stored as one 16-byte write.
// Gathered A rows are read in 128-byte pieces with BK = 64 (whole L2 lines:
// a probe of gathered 64-byte pieces from a 16 MiB activation measured 5.2
// TB/s against 10.3 TB/s for 128-byte pieces).
// With read-ahead (RA, BK = 32) the fragments of slice s + 1 are read into a
// second register set while the MFMAs of slice s run; that needs ~200 VGPRs,
// so it is used where two workgroups per CU are the limit anyway (256 x 64).
// Slices past K are loaded from the zero page, so every iteration issues the
// same DMA count and the waits are the same constant.
// The weighted input gradient also yields the routing-weight gradient
// (dgate_r = sum_n rnd(acc) * x_r[n], cvmm.py:1101): the DG variant sums each
// tile row over its n tile in a fixed order (a lane's 16 columns, the row's 4
// lanes, the waves through LDS) and stores one partial per n tile; a later
// pass adds the n tiles in order.
//
// LDS rows are 64 or 128 bytes.  The MFMA fragment reads (lane l: row l % 16,
// chunk l / 16) are free of bank conflicts with chunk ^ ((r >> 1) & 3) for
// 64-byte rows and chunk ^ (r & 7) for 128-byte rows: an inline-asm
// ds_read_b128 probe on gfx950 measured SQ_LDS_BANK_CONFLICT = 0 for both,
// and 16.8 M conflict cycles for 64-byte rows with chunk ^ (r & 3),
// chunk ^ ((r >> 2) & 3) or no swizzle.
#pragma once

#include <type_traits>

#include "cvmm_gemm_panel.h"

namespace cvmm {

template <int BM, int BN, int STAGES, int BK_, int NW = 4>
struct RingCfg {
  static constexpr int BK = BK_;                       // 16-bit values per k slice
  static constexpr int ROWB = BK * 2;                  // bytes per LDS row
  static constexpr int CPR = ROWB / 16;                // 16-byte chunks per row
  static constexpr int KSS = BK / 32;                  // MFMA k steps per slice
  static_assert(BK == 32 || BK == 64, "64- or 128-byte rows");
  static constexpr int A_BYTES = BM * ROWB;
  static constexpr int B_BYTES = BN * ROWB;
  static constexpr int SLICE_BYTES = A_BYTES + B_BYTES;
  static constexpr int NT = NW * 64;                   // threads per workgroup
  static constexpr int D = SLICE_BYTES / (NW * 1024);  // DMA instructions per wave per slice
  static constexpr int WN = BN / 64, WM = NW / WN;     // wave grid: 64 columns per wave
  static constexpr int WROWS = BM / WM;                // rows per wave: 64, 80 or 128
  static constexpr int MB = WROWS / 16;                // 16-row MFMA blocks per wave
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(WM * WN == NW && WM * WROWS == BM && WROWS % 16 == 0, "waves of whole 16-row blocks");
  static_assert(SLICE_BYTES % (NW * 1024) == 0, "whole DMA instructions per wave");
  static_assert(STAGES >= 2 && STAGES <= 5, "ring depth");
  static_assert((STAGES - 2) * D < 64, "vmcnt range");
};

// 64-byte rows: chunk ^ ((r >> 1) & 3); 128-byte rows: chunk ^ (r & 7).
template <int CPR>
__device__ __forceinline__ int ring_swz(int row) {
  if constexpr (CPR == 4) return (row >> 1) & 3;
  else return row & 7;
}

// lgkmcnt(0) tied to the registers of the fragment reads of one k step (NB
// B fragments, NA A fragments): no use of them is scheduled before the wait.
template <int NB, int NA>
__device__ __forceinline__ void lds_wait_tied_n(lds_u32x4 (&x)[NB], lds_u32x4 (&y)[NA]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[0]), "+v"(y[0]));
#pragma unroll
  for (int i = 1; i < NB; ++i) asm volatile("" : "+v"(x[i]));
#pragma unroll
  for (int i = 1; i < NA; ++i) asm volatile("" : "+v"(y[i]));
}

// lgkmcnt(0) tied to the registers of one k step's transposed B reads (two
// 8-byte reads per 16-column block) and its A fragment reads.
template <int NA>
__device__ __forceinline__ void lds_wait_tied_tr(lds_u32x2 (&x)[4][2], lds_u32x4 (&y)[NA]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[0][0]), "+v"(y[0]));
  asm volatile("" : "+v"(x[0][1]));
#pragma unroll
  for (int i = 1; i < 4; ++i) asm volatile("" : "+v"(x[i][0]), "+v"(x[i][1]));
#pragma unroll
  for (int i = 1; i < NA; ++i) asm volatile("" : "+v"(y[i]));
}

// BNC: the weights are n-contiguous in memory (B[k][n] rows of N values, as
// the other orientation's copy holds them).  Their slices then sit in LDS as
// BK rows of BN columns, and ds_read_b64_tr_b16 hands each lane 4 k values of
// one column per read; two reads make the 8 consecutive k values of an MFMA
// operand (the weight gradient's transposed reads).  One weight copy then
// serves both products of a step.
template <typename OpT, typename OutT, int BM, int BN, int STAGES, int OCC, bool RA, int Role, int BK, bool DG = false,
          bool BNC = false, int NW = 4>
__global__ __launch_bounds__(NW * 64, OCC) void routed_gemm_ring_kernel(const GemmParams p) {
  using Cfg = RingCfg<BM, BN, STAGES, BK, NW>;
  constexpr int MB = Cfg::MB, WR = Cfg::WROWS;
  constexpr int ROWB_B = BNC ? BN * 2 : Cfg::ROWB;  // bytes per LDS row of a B slice
  constexpr int CPR_B = ROWB_B / 16;
  constexpr int A_INSTS = Cfg::A_BYTES / 1024;     // DMA instructions of a slice's A rows
  static_assert(Cfg::A_BYTES % 1024 == 0, "A and B rows in separate DMA instructions");
  static_assert(!BNC || CPR_B == 8 || CPR_B == 16 || CPR_B == 32, "128- to 512-byte B rows");
  static_assert(!RA || Cfg::KSS == 1, "read-ahead keeps one k step per slice");
  __shared__ __attribute__((aligned(1024))) char ring[STAGES * Cfg::SLICE_BYTES];
  __shared__ RouteMeta<BM> meta;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tile = id / n_ntiles;
  const int64_t ntile = id % n_ntiles;
  const int64_t n0 = ntile * BN;

  if (!gemm_schedule<BM, Cfg::NT>(p, tile, meta)) {
    // the routing-weight gradient's partials: one per 128 columns (per tile
    // where BN = 64)
    constexpr int kDgPer = BN > 128 ? BN / 128 : 1;
    zero_unrouted_cols<BM, Cfg::NT>(p, meta, tile, gridDim.x / n_ntiles, n0, n0 + BN, ntile * kDgPer, kDgPer);
    return;
  }
  const int32_t expert = meta.expert;

  // ---- per-lane DMA sources: instruction j of wave w fills LDS bytes
  // [(w * D + j) * 1024, +1024) of a slice; A rows first, then B rows ([n][k]
  // rows of BK values, or with BNC [k][n] rows of BN values)
  const char* zero = reinterpret_cast<const char*>(g_cvmm_zero_page);
  const char* src[Cfg::D];
  int kc[Cfg::D];  // k of this lane's chunk within a slice: its first element, or (BNC B) its row
#pragma unroll
  for (int j = 0; j < Cfg::D; ++j) {
    const int q = (wave * Cfg::D + j) * 64 + lane;  // 16-byte chunk index within the slice
    if (wave * Cfg::D + j < A_INSTS) {
      const int row = q / Cfg::CPR;
      const int c = (q % Cfg::CPR) ^ ring_swz<Cfg::CPR>(row);
      kc[j] = c * 8;
      const int64_t ar = meta.arow[row];
      src[j] = ar >= 0 ? reinterpret_cast<const char*>(p.a) + (ar * p.a_ld + c * 8) * 2 : nullptr;
    } else if constexpr (!BNC) {
      const int row = q / Cfg::CPR;
      const int c = (q % Cfg::CPR) ^ ring_swz<Cfg::CPR>(row);
      kc[j] = c * 8;
      const int64_t gn = n0 + (row - BM);
      src[j] = gn < p.N ? reinterpret_cast<const char*>(p.b) + ((int64_t)expert * p.b_se + gn * p.b_sn + c * 8) * 2
                        : nullptr;
    } else {
      const int qb = q - A_INSTS * 64;
      const int krow = qb / CPR_B;
      const int c = (qb % CPR_B) ^ tr_row_swz<CPR_B>(krow);
      kc[j] = krow;
      const int64_t gn = n0 + c * 8;
      src[j] = gn < p.N ? reinterpret_cast<const char*>(p.b) + ((int64_t)expert * p.b_se + krow * p.b_sk + gn) * 2
                        : nullptr;
    }
  }
  // bytes a chunk's source moves per k: 2 along a row, a row stride for BNC B
  const int64_t b_adv = BNC ? p.b_sk * 2 : 2;
  auto issue = [&](int64_t s, char* buf) {
    const int64_t k0 = s * Cfg::BK;
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      const int64_t adv = wave * Cfg::D + j < A_INSTS ? 2 : b_adv;
      const char* sp = (src[j] != nullptr && k0 + kc[j] < p.K) ? src[j] + k0 * adv : zero;
      dma16(sp, buf + (wave * Cfg::D + j) * 1024);
    }
  };

  // ---- fragments: lane reads row (l % 16) of each 16-row block, chunk l / 16
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int fr = lane & 15, fq = lane >> 4;
  // B fragment of n-block i, k step kk: lane l holds B[n = 16 i + l % 16]
  // [k = 32 kk + 8 (l / 16) .. + 8].  [n][k] rows: one 16-byte read.  BNC
  // [k][n] rows: two transposed reads of rows 8 (l / 16) + (l % 16) / 4 and
  // + 4, at column 4 (l % 4) of the 16-column block.
  int a_off[Cfg::KSS][MB], b_off[Cfg::KSS][4];  // per k step of a slice
#pragma unroll
  for (int kk = 0; kk < Cfg::KSS; ++kk) {
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int ra = wm * WR + j * 16 + fr;
      a_off[kk][j] = ra * Cfg::ROWB + (((kk * 4 + fq) ^ ring_swz<Cfg::CPR>(ra)) << 4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (BNC) {
        const int r = kk * 32 + fq * 8 + (fr >> 2);
        const int lane_lo = ((fr & 1) << 3) + (((fr >> 1) & 1) << 4);
        b_off[kk][i] = Cfg::A_BYTES + r * ROWB_B + lane_lo + (((wn * 8 + 2 * i) ^ tr_row_swz<CPR_B>(r)) << 4);
      } else {
        const int rb = BM + wn * 64 + i * 16 + fr;
        b_off[kk][i] = rb * Cfg::ROWB + (((kk * 4 + fq) ^ ring_swz<Cfg::CPR>(rb)) << 4);
      }
    }
  }
  f32x4_t acc[4][MB];  // acc[i][j]: n-block i, m-block j (C^T orientation)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  using BFrag = std::conditional_t<BNC, lds_u32x2[4][2], lds_u32x4[4]>;
  auto read_frags = [&](const char* buf, lds_u32x4 (&af)[MB], BFrag& bf, int kk = 0) {
    if constexpr (BNC) {
      const uint32_t base = lds_addr(buf);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf[i][0] = lds_read_tr<0>(base + b_off[kk][i]);
        bf[i][1] = lds_read_tr<4 * ROWB_B>(base + b_off[kk][i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) bf[i] = lds_read128(buf + b_off[kk][i]);
    }
#pragma unroll
    for (int j = 0; j < MB; ++j) af[j] = lds_read128(buf + a_off[kk][j]);
  };
  auto wait_frags = [&](BFrag& bf, lds_u32x4 (&af)[MB]) {
    if constexpr (BNC) lds_wait_tied_tr(bf, af);
    else lds_wait_tied_n(bf, af);
  };
  auto mfma = [&](lds_u32x4 (&af)[MB], BFrag& bf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 b;
      if constexpr (BNC) b = make_uint4(bf[i][0].x, bf[i][0].y, bf[i][1].x, bf[i][1].y);
      else b = as_uint4(bf[i]);
#pragma unroll
      for (int j = 0; j < MB; ++j) MfmaOp<OpT>::step(acc[i][j], b, as_uint4(af[j]));
    }
  };

  // DG (16-bit x with 8-byte aligned rows, ring_eligible): every x piece
  // this lane needs for the routing-weight gradient (MB rows x 4 blocks of 4
  // columns, 8 bytes each) is requested early, so the gathers' latency
  // overlaps the last MFMAs (or at least the output stores).  Waves of 8 row
  // blocks (256 x 256 tiles) have no registers for them: their sums load
  // the pieces where they use them.
  constexpr bool XPRE = MB <= 5;
  uint2 xpre[XPRE ? MB : 1][4];
  auto load_x = [&]() {
    if constexpr (!XPRE) return;
    const int64_t nw = n0 + wn * 64;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int64_t xr = meta.dgrow[wm * WR + j * 16 + fr];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = nw + i * 16 + 4 * fq;
        xpre[j][i] = xr >= 0 && n < p.N
                         ? *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.dg_x) + xr * p.dg_x_ld + n)
                         : make_uint2(0, 0);
      }
    }
  };

  const int64_t nk = (p.K + Cfg::BK - 1) / Cfg::BK;
  if constexpr (RA) {
    // ---- k loop with fragment read-ahead: the fragments of slice s + 1 are
    // read while the MFMAs of slice s run (two register sets), so a slice's
    // buffer is free once its reads have been waited for: iteration s refills
    // the buffer of slice s with slice s + STAGES.
#pragma unroll
    for (int s0 = 0; s0 < STAGES; ++s0) {
      issue(s0, ring + s0 * Cfg::SLICE_BYTES);
      issue_fence();
    }
    lds_u32x4 a0[MB], a1[MB];
    BFrag b0, b1;
    vm_wait<(STAGES - 1) * Cfg::D>();
    wg_barrier();
    read_frags(ring, a0, b0);
    wait_frags(b0, a0);
    int buf = 0;  // buffer of slice s
    auto step = [&](int64_t s, lds_u32x4 (&ac)[MB], BFrag& bc, lds_u32x4 (&an)[MB], BFrag& bn) {
      const int nxt = buf + 1 == STAGES ? 0 : buf + 1;
      vm_wait<(STAGES - 2) * Cfg::D>();  // slice s + 1 has landed (only DMA is in flight)
      wg_barrier();
      issue(s + STAGES, ring + buf * Cfg::SLICE_BYTES);
      issue_fence();
      read_frags(ring + nxt * Cfg::SLICE_BYTES, an, bn);
      mfma(ac, bc);
      wait_frags(bn, an);
      buf = nxt;
    };
    for (int64_t s = 0; s < nk; s += 2) {
      step(s, a0, b0, a1, b1);
      if (s + 1 >= nk) break;
      step(s + 1, a1, b1, a0, b0);
    }
  } else {
    // ---- k loop: wait for slice s, refill the buffer of slice s - 1 with
    // slice s + STAGES - 1, then read and multiply slice s
#pragma unroll
    for (int s0 = 0; s0 < STAGES - 1; ++s0) {
      issue(s0, ring + s0 * Cfg::SLICE_BYTES);
      issue_fence();
    }
    int cur = 0, refill = STAGES - 1;
    auto multiply = [&]() {
#pragma unroll
      for (int kk = 0; kk < Cfg::KSS; ++kk) {
        lds_u32x4 af[MB];
        BFrag bf;
        read_frags(ring + cur * Cfg::SLICE_BYTES, af, bf, kk);
        wait_frags(bf, af);
        mfma(af, bf);
      }
    };
    // DG: the last slice is peeled (K > 128, so nk >= 2)
    static_assert(!DG || STAGES == 2, "the peeled DG slice leaves no DMA in flight");
    const int64_t n_loop = DG ? nk - 1 : nk;
    for (int64_t s = 0; s < n_loop; ++s) {
      vm_wait<(STAGES - 2) * Cfg::D>();
      wg_barrier();
      issue(s + STAGES - 1, ring + refill * Cfg::SLICE_BYTES);
      issue_fence();
      multiply();
      cur = cur + 1 == STAGES ? 0 : cur + 1;
      refill = refill + 1 == STAGES ? 0 : refill + 1;
    }
    if constexpr (DG) {
      // the last slice: the x pieces take the place of its refill, which
      // would only bring zeros from past K (8-block waves, which load their
      // pieces in the sums, peel it all the same)
      vm_wait<(STAGES - 2) * Cfg::D>();
      wg_barrier();
      load_x();
      issue_fence();
      multiply();
    }
  }
  // slices past K may still be landing in LDS: drain them before the
  // workgroup can end and its LDS be handed to another (the peeled DG loop
  // issues none; its x loads are waited for where they are used)
  if constexpr (RA || !DG) vm_wait<0>();

  // ---- epilogue from registers: lane holds C[m = wm*WR + j*16 + fr]
  // [n = n0 + wn*64 + i*16 + 4*fq + {0..3}]
  const bool has_w = p.w != nullptr;
  // plain: the value is the product rounded once to the output type, which
  // the conversion at the store does by itself
  const bool plain = !has_w && p.val_dtype == DTypeOf<OutT>::value;
  const int64_t nwave = n0 + wn * 64;
  // DG without a peeled last slice (the read-ahead loop): the x pieces now
  if constexpr (DG && RA) load_x();
  // one row piece of 4 x 16 columns: lane values -> 16-byte (or 4 x 16-byte
  // fp32) stores of row rowp
  auto store_row = [&](char* rowp, const float (&v)[4][4]) {
    if constexpr (sizeof(OutT) == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = nwave + i * 16 + 4 * fq;
        if (rowp != nullptr && n < p.N)
          *reinterpret_cast<float4*>(rowp + n * 4) = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
      }
    } else {
      // blocks 2p, 2p+1 -> columns 32p + 8*fq + [0, 8) per lane (two lane swaps)
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        uint32_t a[2], b[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          union { uint32_t u; OutT e[2]; } pa, pb;
          pa.e[0] = (OutT)v[2 * pr][2 * h];
          pa.e[1] = (OutT)v[2 * pr][2 * h + 1];
          pb.e[0] = (OutT)v[2 * pr + 1][2 * h];
          pb.e[1] = (OutT)v[2 * pr + 1][2 * h + 1];
          a[h] = pa.u;
          b[h] = pb.u;
        }
        const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
        const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s0[1], false, false);
        const auto t1 = __builtin_amdgcn_permlane16_swap(s1[0], s1[1], false, false);
        const int64_t n = nwave + pr * 32 + 8 * fq;
        if (rowp != nullptr && n < p.N)
          *reinterpret_cast<uint4*>(rowp + n * 2) = make_uint4(t0[0], t1[0], t0[1], t1[1]);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = wm * WR + j * 16 + fr;
    const int64_t orow = meta.orow[m];
    float v[4][4];
    if (plain) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[i][q] = acc[i][j][q];
    } else {
      const float wv = meta.w[m];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float c = round_to(acc[i][j][q], p.val_dtype);
          if (has_w) {
            c = c * wv;
            if (p.prod_dtype >= 0) c = round_to(c, p.prod_dtype);
          }
          v[i][q] = c;
        }
    }
    char* rowp = orow >= 0 ? reinterpret_cast<char*>(p.out) + orow * p.out_ld * (int64_t)sizeof(OutT) : nullptr;
    if (p.act == 0) {
      store_row(rowp, v);
    } else {
      // GELU: h = the product in the output type (kept for the backward),
      // out = gelu(h) rounded to the output type
      char* auxp = orow >= 0 ? reinterpret_cast<char*>(p.aux) + orow * p.out_ld * (int64_t)sizeof(OutT) : nullptr;
      float y[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float h = (float)(OutT)v[i][q];
          v[i][q] = h;
          y[i][q] = gelu_erf(h);
        }
      store_row(auxp, v);
      store_row(rowp, y);
    }
  }

  if constexpr (DG) {
    // routing-weight gradient partial of this n tile for each tile row:
    // sum_n rnd(acc, dg_val) * x[dgrow][n].  Fixed order: each lane its 16
    // columns (blocks i, then the 4 columns), the 4 lanes of a row (xor 16,
    // then xor 32), then the waves of the tile row in wn order through LDS.
    // (N % 8 == 0: a 4-column piece is wholly inside or outside the row)
    const bool xbf = p.dg_x_dtype == kBF16;
    float part[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int64_t xr = meta.dgrow[wm * WR + j * 16 + fr];
      float sum = 0.f;
      if (xr >= 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (nwave + i * 16 + 4 * fq >= p.N) continue;
          union { uint2 u; bf16_t b[4]; f16_t h[4]; } c;
          if constexpr (XPRE)
            c.u = xpre[j][i];
          else
            c.u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.dg_x) + xr * p.dg_x_ld +
                                                  nwave + i * 16 + 4 * fq);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            sum += round_to(acc[i][j][q], p.dg_val_dtype) * (xbf ? (float)c.b[q] : (float)c.h[q]);
        }
      }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      part[j] = sum;
    }
    if constexpr (Cfg::WN == 1) {
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const int m = wm * WR + j * 16 + fr;
        if (fq == 0 && meta.widx[m] >= 0) p.dg[meta.widx[m] * p.dg_ntiles + ntile] = part[j];
      }
    } else {
      // one partial per 128 columns: the two waves of each 128-column piece
      // summed in wn order (one piece for BN = 128, two for 256 x 256
      // tiles).  Every wave is past its last LDS read of the ring (the DMA
      // drained above): the ring's first bytes take the per-wave partials.
      constexpr int WPP = 2, DGP = Cfg::WN / WPP;
      float* red = reinterpret_cast<float*>(ring);
      wg_barrier();
      if (fq == 0) {
#pragma unroll
        for (int j = 0; j < MB; ++j) red[wn * BM + wm * WR + j * 16 + fr] = part[j];
      }
      __syncthreads();
      if (wn % WPP == 0 && fq == 0) {
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          const int m = wm * WR + j * 16 + fr;
          float sum = red[wn * BM + m];
#pragma unroll
          for (int w = 1; w < WPP; ++w) sum += red[(wn + w) * BM + m];
          if (meta.widx[m] >= 0) p.dg[meta.widx[m] * p.dg_ntiles + ntile * DGP + wn / WPP] = sum;
        }
      }
    }
  }
}

// The ring kernel applies: plain stores (optionally scaled by a per-row
// routing weight, optionally with the routing-weight gradient partials of
// its n tile, of gemm_bn(N) columns, against 16-bit x with 8-byte aligned
// rows), output in the op type or fp32, N a multiple of 8 with 16-byte
// aligned output rows.
inline bool ring_eligible(const GemmParams& p, int32_t op) {
  const size_t esz = p.out_dtype == kF32 ? 4 : 2;
  // weights k-contiguous, or n-contiguous with 16-byte aligned k rows
  const bool b_ok = p.b_sk == 1 || (p.b_sn == 1 && p.b_sk % 8 == 0 && p.b_se % 8 == 0 &&
                                     (reinterpret_cast<uintptr_t>(p.b) & 15) == 0);
  return p.K > 128 && p.epi == kEpiStore && p.out != nullptr && b_ok &&
         (p.dg == nullptr || (p.act == 0 && p.dg_ntiles == (p.N + (p.N <= 64 ? 63 : 127)) / (p.N <= 64 ? 64 : 128) &&
                              (p.dg_x_dtype == kBF16 || p.dg_x_dtype == kF16) &&
                              (reinterpret_cast<uintptr_t>(p.dg_x) & 7) == 0 && p.dg_x_ld % 4 == 0)) &&
         (p.act == 0 || (p.aux != nullptr && (reinterpret_cast<uintptr_t>(p.aux) % 16) == 0)) &&
         (p.out_dtype == op || p.out_dtype == kF32) && p.N % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(p.out) % 16) == 0 && ((size_t)p.out_ld * esz) % 16 == 0;
}

template <typename OpT, typename OutT, int BM, int BN, int STAGES, int OCC, bool RA, int BK, bool BNC, int NW>
hipError_t launch_routed_gemm_ring_b(const GemmParams& p_in, hipStream_t stream) {
  GemmParams p = p_in;
  p.token_major = resolve_token_major(p);
  const int64_t m_tiles = (p.n_routes + BM - 1) / BM + (p.n_experts < p.n_routes ? p.n_experts : p.n_routes);
  const int64_t n_ntiles = (p.N + BN - 1) / BN;
  const int64_t grid = m_tiles * n_ntiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  // the routing-weight gradient only ever comes with the grad-input product
  if (p.role == 0 && p.dg == nullptr)
    hipLaunchKernelGGL((routed_gemm_ring_kernel<OpT, OutT, BM, BN, STAGES, OCC, RA, 0, BK, false, BNC, NW>),
                       dim3((unsigned)grid), dim3(NW * 64), 0, stream, p);
  else if (p.dg == nullptr)
    hipLaunchKernelGGL((routed_gemm_ring_kernel<OpT, OutT, BM, BN, STAGES, OCC, RA, 1, BK, false, BNC, NW>),
                       dim3((unsigned)grid), dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((routed_gemm_ring_kernel<OpT, OutT, BM, BN, STAGES, OCC, RA, 1, BK, true, BNC, NW>),
                       dim3((unsigned)grid), dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

// k-contiguous weights ([n][k] rows), or n-contiguous ones (BNC, b_sn == 1)
template <typename OpT, typename OutT, int BM, int BN, int STAGES, int OCC, bool RA, int BK, int NW = 4>
hipError_t launch_routed_gemm_ring_t(const GemmParams& p, hipStream_t stream) {
  if (p.b_sk == 1) return launch_routed_gemm_ring_b<OpT, OutT, BM, BN, STAGES, OCC, RA, BK, false, NW>(p, stream);
  return launch_routed_gemm_ring_b<OpT, OutT, BM, BN, STAGES, OCC, RA, BK, true, NW>(p, stream);
}

// 128 x 128 tiles: two 32 KB slices of 64 k (128-byte rows: each gathered A
// row is read in whole 128-byte lines) + route metadata = 69 KB of LDS, two
// workgroups per CU.  Measured on the ff_up forward shape with the
// benchmark's spread of expert loads: 35.9 us, against 45.7 us for three
// 16 KB slices of 32 k at three workgroups per CU.
// 256 x 64 tiles: 3 slices of 20 KB + 9 KB = 69 KB, two per CU, read-ahead.
// 160 x 128 tiles (two waves of 80 rows along m: 5 MFMA blocks each; two
// 36 KB slices + metadata = 78 KB, two per CU) unless they cost more than
// 5 % over 128-row tiles in round count x tile height, with the tile count
// estimated as R / BM + E / 2 (an expert's last tile half full on average)
// on 256 CUs x 2 workgroups.  At the ff_up forward shape 128-row tiles need
// 544 tiles on 512 slots -- 32 run as a second round alone -- while 160-row
// tiles need ~442: one round (42.4 -> 32.0 us; the ff_down grad-input 74.6
// -> 50.3 us).  Over many rounds a tile's weight slices serve 25 % more rows
// (the FFN stack's long-K products 522 -> 508 and 540 -> 523 us per
// launch).  A single round of a small product keeps 128-row tiles (more
// workgroups).
inline bool ring_tall_tiles(const GemmParams& p) {
  constexpr int64_t kSlots = 2 * 256;
  const int64_t nt = (p.N + 127) / 128;
  auto rounds = [&](int64_t bm) {
    const int64_t tiles = (p.n_routes + bm - 1) / bm + p.n_experts / 2;
    return (tiles * nt + kSlots - 1) / kSlots;
  };
  return 20 * 160 * rounds(160) <= 21 * 128 * rounds(128);
}

// 256 x 256 tiles of eight waves (2 x 4 waves of 128 x 64; two 64 KB slices
// + metadata = 137 KB, one workgroup per CU): each gathered A row piece
// serves twice the columns of a 128-column tile.  At the FFN stack (K =
// 2048 / 512, N = 512 / 2048, ~4.5-18 dispatch rounds) the forward went 508
// -> 452 us and the grad-input without the routing-weight gradient 548 ->
// 476 us per launch.  Four waves of 128 x 128 (the same tile), 320 x 128,
// 256 x 128 and 128 x 256 of eight waves, and 32-k slices in a 4-slice ring
// all measured slower or no faster.  Taken where N is a multiple of 256 and
// the grid fills at least two rounds of 256 CUs (tile count estimated as R /
// 256 + E / 2).  With the routing-weight gradient each 128-column half of
// the tile writes its own partial, summed as a 128-column tile sums it.
inline bool ring_wide_tiles(const GemmParams& p) {
  if (p.N % 256 != 0 || p.ring_tile == 1 || p.ring_tile == 2) return false;
  if (p.ring_tile == 3) return true;
  const int64_t tiles = ((p.n_routes + 255) / 256 + p.n_experts / 2) * (p.N / 256);
  return tiles >= 2 * 256;
}

template <typename OpT, typename OutT>
hipError_t launch_routed_gemm_ring_out(const GemmParams& p, hipStream_t stream) {
  if (p.N <= 64) return launch_routed_gemm_ring_t<OpT, OutT, 256, 64, 3, 2, true, 32>(p, stream);
  if (ring_wide_tiles(p)) return launch_routed_gemm_ring_t<OpT, OutT, 256, 256, 2, 1, false, 64, 8>(p, stream);
  if (p.ring_tile == 2 || ((p.ring_tile == 0 || p.ring_tile == 3) && ring_tall_tiles(p)))
    return launch_routed_gemm_ring_t<OpT, OutT, 160, 128, 2, 2, false, 64>(p, stream);
  return launch_routed_gemm_ring_t<OpT, OutT, 128, 128, 2, 2, false, 64>(p, stream);
}

// Fast-path dispatch for 16-bit k-contiguous operands: small K -> panel
// kernel, long K -> ring kernel, anything else (routing-weight gradient,
// atomics, unaligned output) -> the tiled kernel.
template <typename OpT>
hipError_t launch_routed_gemm_fast_op(const GemmParams& p, hipStream_t stream) {
  constexpr int32_t op = DTypeOf<OpT>::value;
  if (p.act != 0 && !ring_eligible(p, op)) return hipErrorInvalidValue;  // only the ring kernel applies it
  if (panel_eligible(p, op)) {
    if (p.out_dtype == kF32) return launch_routed_gemm_panel_out<OpT, float>(p, stream);
    return launch_routed_gemm_panel_out<OpT, OpT>(p, stream);
  }
  if (ring_eligible(p, op)) {
    if (p.out_dtype == kF32) return launch_routed_gemm_ring_out<OpT, float>(p, stream);
    return launch_routed_gemm_ring_out<OpT, OpT>(p, stream);
  }
  return launch_routed_gemm_nt_op<OpT>(p, stream);
}

}  // namespace cvmm
