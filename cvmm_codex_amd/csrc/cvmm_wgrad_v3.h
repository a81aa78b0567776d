// Weight gradient fast path (16-bit operands, gfx950): dW[e] = X_e^T G_e.
//
// The reduction runs over the expert's routes, and both operands are gathered
// route rows (an x row and a dY row per route).  A workgroup owns one
// BM x BN tile of dW[e] (x columns m0.., dY columns n0..) and one chunk of the
// expert's routes, and streams that chunk through LDS in slices of 32 routes:
//  * Route table: the chunk's row indices (and rounded routing weights) are
//    resolved once, coalesced, into an LDS table; the DMA lanes of each slice
//    read their row from it.  Chunks longer than the table run in segments.
//  * DMA ring: slices move by global_load_lds (16 bytes per lane, one 1 KB
//    instruction = RPI rows) into a ring of STAGES buffers, STAGES - 1 in
//    flight.  Only DMA is in flight in the loop, so the wait for slice s is the
//    exact vmcnt of the slices issued after it.
//  * Fragments without transposing writes: the slices keep the natural
//    [route][column] layout, and ds_read_b64_tr_b16 hands each lane 4 routes
//    of one column (lane L of a 16-lane group points at route L / 4, column
//    4 * (L % 4)); two reads give the 8 routes of a 16x16x32 MFMA operand.
//  * Operands swapped (dW^T tile = G^T X), so a lane ends holding 4
//    consecutive dW columns of one row, stored as one 16-byte write straight
//    from the accumulators.
//  * Weighted routes (dY scaled by the routing weight, rounded to the op type
//    as cvmm.py:590-599 does) are scaled while the dY fragments are in
//    registers: each lane's 8 routes share one weight per route.
//  * An expert with more routes than the split runs as several chunks; each
//    writes its fp32 partial tile in fragment order, and the last to arrive
//    (per-tile counter) sums them in chunk order -- deterministic -- and
//    stores dW.
//  * Tiles: 128 x 128 (and 256 x 64 / 64 x 256 on a narrow side) at two
//    workgroups per CU, each wave 64 x 64; or, for wide dW, 256 x 256 (or
//    256 x 128 / 128 x 256) at one workgroup per CU, each of four waves up to
//    128 x 128 with its accumulators in AGPRs, or 256 x 256 of eight waves
//    of 128 x 64 (two waves per SIMD: the FFN stack's launch 514 -> 485 us).
//    Every tile sums each dW element over the same slices in the same
//    order, so the tile choice never changes bits.
// Workgroup orders (WgradParams::order): tile-major by default; chunk-major
// and chunk-per-XCD for tuning.
// LDS rows are swizzled at 16-byte granularity so that a transposed read's
// 16 lanes (4 routes x 32 bytes) hit distinct banks:
//   256-byte rows: chunk ^ (2 * ((row & 3) | (((row >> 3) & 1) << 2)))
//   128-byte rows: chunk ^ (2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1)))
// and 512-byte rows use the 256-byte rule within each half.
#pragma once

#include "cvmm_gemm_panel.h"

namespace cvmm {

static __device__ uint4 g_cvmm_wg3_zero_page[64];

// 32 route rows of COLS 16-bit values.
template <int COLS>
struct RouteSlice {
  static constexpr int ROWB = COLS * 2;
  static constexpr int CPR = COLS / 8;        // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per 1 KB DMA instruction
  static constexpr int BYTES = 32 * ROWB;
  static constexpr int INSTS = BYTES / 1024;
  static_assert(CPR == 8 || CPR == 16 || CPR == 32, "64, 128 or 256 columns");
  __device__ static __forceinline__ int swz(int row) { return tr_row_swz<CPR>(row); }
};

// A BM x BN tile on a WM x WN grid of waves; each wave owns JM x IN blocks of
// 16 x 16 (x columns x dY columns).  Four waves of up to 16 blocks (64
// accumulator registers) run two workgroups per CU with 80 KB of LDS each;
// four waves of more blocks run one workgroup per CU -- one wave per SIMD,
// whose 512 registers hold the accumulators in AGPRs -- with all 160 KB;
// eight waves (two per SIMD, 256 registers each) run one workgroup per CU.
template <int BM, int BN, int WM, int WN, int STAGES, bool WEIGHTED>
struct Wg3Cfg {
  using TA = RouteSlice<BM>;                   // x rows: dW rows m0 .. m0 + BM
  using TB = RouteSlice<BN>;                   // dY rows: dW columns n0 .. n0 + BN
  static constexpr int NW = WM * WN, NT = NW * 64;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static constexpr int JM = BM / WM / 16, IN = BN / WN / 16;
  static constexpr int OCC = JM * IN <= 16 ? 2 : 1;  // workgroups per CU
  static_assert(JM * WM * 16 == BM && IN * WN * 16 == BN && JM >= 1 && IN >= 1, "wave grid");
  static constexpr int SLICE = TA::BYTES + TB::BYTES;
  static constexpr int D = (TA::INSTS + TB::INSTS) / NW;  // DMA instructions per wave per slice
  static_assert((TA::INSTS + TB::INSTS) % NW == 0, "whole DMA instructions per wave");
  static_assert((STAGES - 2) * D < 64, "vmcnt range");
  // route table in what is left of the workgroup's share of the 160 KB
  static constexpr int ENTRY = WEIGHTED ? 12 : 8;
  static constexpr int TBL = (((160 / OCC) * 1024 - 512 - STAGES * SLICE) / ENTRY) / 32 * 32;
  static_assert(TBL >= 256, "route table");
};

struct Wg3Sched {
  int32_t expert, nch, last;
  int64_t lo, hi, slot, base_slot;
};

// (expert, route chunk) of work slot `slot_id`: experts in order, each cut
// into chunks of p.split routes (at least one chunk per expert).
__device__ __forceinline__ bool wgrad_schedule(const WgradParams& p, int64_t slot_id, Wg3Sched& s) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    if (lane == 0) s.expert = -1;
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
        s.expert = e;
        s.nch = (int32_t)nch;
        s.lo = start + c * p.split;
        s.hi = (start + (c + 1) * p.split) < end ? start + (c + 1) * p.split : end;
        s.base_slot = incl_m - multi;
        s.slot = s.base_slot + c;
      }
      carry = __shfl(incl, 63, 64);
      carry_multi = __shfl(incl_m, 63, 64);
      if (slot_id < carry) break;
    }
  }
  __syncthreads();
  return s.expert >= 0;
}

// dW contiguous fp32 rows, 16-byte aligned: a lane's 4 columns are one store.
__host__ __device__ inline bool wgrad_dw_vec(const WgradParams& p) {
  return p.dw_sn == 1 && p.dw_dtype == kF32 && p.dw_sm % 4 == 0 && p.dw_se % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(p.dw) & 15) == 0;
}

template <typename OpT, int BM, int BN, int WM, int WN, int STAGES, bool WEIGHTED>
__global__ __launch_bounds__(WM * WN * 64, (BM / WM / 16) * (BN / WN / 16) <= 16 ? 2 : 1) void wgrad_v3_kernel(
    const WgradParams p) {
  using Cfg = Wg3Cfg<BM, BN, WM, WN, STAGES, WEIGHTED>;
  constexpr int JM = Cfg::JM, IN = Cfg::IN;
  using TA = typename Cfg::TA;
  using TB = typename Cfg::TB;
  constexpr int D = Cfg::D;
  constexpr int TBL = Cfg::TBL;
  __shared__ __attribute__((aligned(1024))) char ring[STAGES * Cfg::SLICE];
  __shared__ __attribute__((aligned(16))) int32_t t_x[TBL];
  __shared__ __attribute__((aligned(16))) int32_t t_g[TBL];
  __shared__ __attribute__((aligned(16))) float t_w[WEIGHTED ? TBL : 4];
  __shared__ Wg3Sched sched;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tiles_n = (p.N + BN - 1) / BN;
  const int64_t tiles = ((p.M + BM - 1) / BM) * tiles_n;
  int64_t slot_id, tile;
  if (p.order == kWgOrderChunkXcd) {  // grid = round_up(grid_chunks, 8) * tiles
    const int64_t xcd = blockIdx.x % 8, local = blockIdx.x / 8;
    slot_id = (local / tiles) * 8 + xcd;
    tile = local % tiles;
  } else {
    const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
    slot_id = p.order == kWgOrderTile ? id % p.grid_chunks : id / tiles;
    tile = p.order == kWgOrderTile ? id / p.grid_chunks : id % tiles;
  }
  const int64_t m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;

  if (!wgrad_schedule(p, slot_id, sched)) return;
  const int32_t expert = sched.expert;
  const int64_t lo = sched.lo, hi = sched.hi;
  const int32_t nch = sched.nch;

  // ---- DMA geometry: instruction j of this wave fills slice bytes
  // [(wave * D + j) * 1024, +1024): x rows (TA) first, then dY rows (TB)
  const char* zero = reinterpret_cast<const char*>(g_cvmm_wg3_zero_page);
  const char* xb = reinterpret_cast<const char*>(p.x) + m0 * 2;
  const char* gb = reinterpret_cast<const char*>(p.g) + n0 * 2;
  // Row bases and strides live in registers: nothing in the loop may load
  // from memory, or the compiler's wait for it would also wait for the DMA.
  uint32_t tab[D];         // LDS address of the table entry of this lane's row (slice 0)
  const char* dbase[D];    // row 0 + this lane's 16-byte chunk, nullptr = past the edge
  int64_t dld[D];          // row stride in bytes
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int gi = wave * D + j;
    if (gi < TA::INSTS) {
      const int row = gi * TA::RPI + lane / TA::CPR;
      const int c = (lane % TA::CPR) ^ TA::swz(row);
      tab[j] = lds_addr(t_x + row);
      dbase[j] = m0 + c * 8 < p.M ? xb + c * 16 : nullptr;
      dld[j] = p.x_ld * 2;
    } else {
      const int row = (gi - TA::INSTS) * TB::RPI + lane / TB::CPR;
      const int c = (lane % TB::CPR) ^ TB::swz(row);
      tab[j] = lds_addr(t_g + row);
      dbase[j] = n0 + c * 8 < p.N ? gb + c * 16 : nullptr;
      dld[j] = p.g_ld * 2;
    }
  }
  auto issue = [&](int s, int slot) {
    int32_t r[D];
#pragma unroll
    for (int j = 0; j < D; ++j) r[j] = lds_read_i32<0>(tab[j] + s * 128);
    lgkm_wait_tied(r);
    char* dst = ring + slot * Cfg::SLICE + wave * D * 1024;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const char* src = (r[j] >= 0 && dbase[j] != nullptr) ? dbase[j] + (int64_t)r[j] * dld[j] : zero;
      dma16(src, dst + j * 1024);
    }
  };

  // ---- fragment offsets: lane reads route row grp*8 + L/4 (+4), columns
  // blk*16 + 4*(L%4); the swizzle sees row bits 0, 1, 3 only -> per-lane constant
  const int wm = wave / WN, wn = wave % WN;
  const int L = lane & 15, grp = lane >> 4;
  const int trow = grp * 8 + (L >> 2);
  const int lane_lo = ((L & 1) << 3) + (((L >> 1) & 1) << 4);
  uint32_t xo[JM], go[IN];
#pragma unroll
  for (int j = 0; j < JM; ++j) xo[j] = trow * TA::ROWB + lane_lo + (((wm * 2 * JM + 2 * j) ^ TA::swz(trow)) << 4);
#pragma unroll
  for (int i = 0; i < IN; ++i)
    go[i] = TA::BYTES + trow * TB::ROWB + lane_lo + (((wn * 2 * IN + 2 * i) ^ TB::swz(trow)) << 4);
  const uint32_t ring_a = lds_addr(ring);
  const uint32_t w_a = lds_addr(t_w) + grp * 32;

  f32x4_t acc[IN][JM];  // acc[i][j]: dY column block i, x column block j (dW^T orientation)
#pragma unroll
  for (int i = 0; i < IN; ++i)
#pragma unroll
    for (int j = 0; j < JM; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s, int slot) {
    const uint32_t base = ring_a + slot * Cfg::SLICE;
    lds_u32x2 gf[IN][2], xf[JM][2];
#pragma unroll
    for (int i = 0; i < IN; ++i) {
      gf[i][0] = lds_read_tr<0>(base + go[i]);
      gf[i][1] = lds_read_tr<4 * TB::ROWB>(base + go[i]);
    }
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      xf[j][0] = lds_read_tr<0>(base + xo[j]);
      xf[j][1] = lds_read_tr<4 * TA::ROWB>(base + xo[j]);
    }
    uint4 g4[IN];
    if constexpr (WEIGHTED) {
      lds_u32x4 w8[2];
      w8[0] = lds_read128_at<0>(w_a + s * 128);
      w8[1] = lds_read128_at<16>(w_a + s * 128);
      lgkm_wait_w(w8);
      lgkm_wait_frags_n(gf, xf);
      float wv[8];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        // element copied to a scalar first: __builtin_bit_cast of a vector
        // element expression reads element 0 with this compiler
        const uint32_t lo = w8[0][v], hi = w8[1][v];
        wv[v] = __uint_as_float(lo);
        wv[4 + v] = __uint_as_float(hi);
      }
#pragma unroll
      for (int i = 0; i < IN; ++i) {
        Chunk16 c;
        c.u = make_uint4(gf[i][0].x, gf[i][0].y, gf[i][1].x, gf[i][1].y);
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = to_f32(reinterpret_cast<const OpT*>(&c)[q]) * wv[q];
        g4[i] = pack_chunk<OpT>(v);
      }
    } else {
      lgkm_wait_frags_n(gf, xf);
#pragma unroll
      for (int i = 0; i < IN; ++i) g4[i] = make_uint4(gf[i][0].x, gf[i][0].y, gf[i][1].x, gf[i][1].y);
    }
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      const uint4 x4 = make_uint4(xf[j][0].x, xf[j][0].y, xf[j][1].x, xf[j][1].y);
#pragma unroll
      for (int i = 0; i < IN; ++i) MfmaOp<OpT>::step(acc[i][j], g4[i], x4);
    }
  };

  // ---- segments of up to TBL routes: table, then the slice ring
  for (int64_t seg = lo; seg < hi; seg += TBL) {
    const int n_rt = (int)((hi - seg) < TBL ? (hi - seg) : TBL);
    const int n_st = (n_rt + 31) / 32;
    if (seg != lo) __syncthreads();  // every wave is done with the previous table
    for (int r = tid; r < n_st * 32; r += Cfg::NT) {
      int32_t xr = -1, gr = -1;
      float w = 0.f;
      if (r < n_rt) {
        const int64_t q = seg + r;
        const int64_t xi = p.x_idx[q];
        const int64_t graw = p.g_idx[q];
        const int64_t gi = (graw >= 0 && graw < 0x7fffffffll) ? p.g_fdiv.div(graw) : -1;
        if (xi >= 0 && xi < p.x_rows && gi >= 0 && gi < p.g_rows) {
          xr = (int32_t)xi;
          gr = (int32_t)gi;
          if constexpr (WEIGHTED) {
            const int64_t wi = p.w_idx[q];
            w = (wi >= 0 && wi < p.n_routes) ? round_to(load_as_f32(p.w, p.w_dtype, wi), DTypeOf<OpT>::value) : 0.f;
          }
        }
      }
      t_x[r] = xr;
      t_g[r] = gr;
      if constexpr (WEIGHTED) t_w[r] = w;
    }
    __syncthreads();
#pragma unroll
    for (int s0 = 0; s0 < STAGES - 1; ++s0) {
      if (s0 < n_st) issue(s0, s0);
      issue_fence();
    }
    int cur = 0;
    for (int s = 0; s < n_st; ++s) {
      const int ahead = (n_st - 1 - s) < (STAGES - 2) ? (n_st - 1 - s) : (STAGES - 2);
      vm_wait_slices<D, STAGES - 2>(ahead);  // slice s has landed (this wave's part)
      wg_barrier();                          // ... every wave's part; slot of s - 1 is free
      if (s + STAGES - 1 < n_st) {
        const int refill = cur == 0 ? STAGES - 1 : cur - 1;
        issue(s + STAGES - 1, refill);
        issue_fence();
      }
      compute(s, cur);
      cur = cur + 1 == STAGES ? 0 : cur + 1;
    }
  }
  vm_wait<0>();

  // ---- epilogue: lane holds dW[m = m0 + wm*16*JM + j*16 + L][n = n0 + wn*16*IN + i*16 + 4*grp + {0..3}]
  // one-workgroup-per-CU tiles are launched only for contiguous, aligned
  // fp32 dW (wgrad_dw_vec): their accumulators never take the element path
  constexpr bool VEC_ONLY = Cfg::OCC == 1;
  const bool dw_vec = VEC_ONLY || wgrad_dw_vec(p);
  // Stores are emitted per 16 x 16 block straight from where the block's sum
  // lives (accumulators, or the chunk partials), with the layout test outside
  // the block loops: no block waits in registers for another.
  auto emit = [&](auto&& block) {
    if (dw_vec) {
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        const int64_t m = m0 + wm * 16 * JM + j * 16 + L;
        if (m >= p.M) continue;
        float* row = reinterpret_cast<float*>(p.dw) + (int64_t)expert * p.dw_se + m * p.dw_sm;
#pragma unroll
        for (int i = 0; i < IN; ++i) {
          const int64_t n = n0 + wn * 16 * IN + i * 16 + 4 * grp;
          if (n < p.N) *reinterpret_cast<float4*>(row + n) = block(i, j);
          __builtin_amdgcn_sched_barrier(0);  // block by block: no accumulator hoisted ahead
        }
      }
    } else if constexpr (!VEC_ONLY) {
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        const int64_t m = m0 + wm * 16 * JM + j * 16 + L;
        if (m >= p.M) continue;
        const int64_t off = (int64_t)expert * p.dw_se + m * p.dw_sm;
#pragma unroll
        for (int i = 0; i < IN; ++i) {
          const int64_t n = n0 + wn * 16 * IN + i * 16 + 4 * grp;
          if (n >= p.N) continue;
          const float4 v = block(i, j);
          const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < p.N) store_from_f32(p.dw, p.dw_dtype, off + (n + q) * p.dw_sn, e[q]);
        }
      }
    }
  };
  auto acc_block = [&](int i, int j) { return make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]); };

  if (nch == 1) {
    emit(acc_block);
    return;
  }

  // ---- multi-chunk expert: fp32 partial tile in fragment order -> workspace;
  // the last arriver sums the chunks in chunk order, by the split-K protocol
  // of cvmm_common.h (splitk_*: on gfx942/gfx950 without release/acquire
  // fences, which write back and invalidate the whole L2 of the XCD under the
  // feet of the other workgroups there: the FFN stack's weight gradient took
  // 780 us per launch with them, 720 us without).
  const int64_t slot = sched.slot;
  if (slot >= p.max_slots) return;  // cannot happen: workspace holds 2R/split + 1 slots
  // float4 k of this lane's fragment list = two 8-byte words at 2k, 2k + 1
  auto frag_ptr = [&](int64_t sl) {
    return reinterpret_cast<uint64_t*>(p.partial) +
           2 * (((sl * tiles + tile) * Cfg::NW + wave) * (IN * JM) * 64 + lane);
  };
  auto pack2 = [](float a, float b) {
    return (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  };
  {
    uint64_t* d = frag_ptr(slot);
#pragma unroll
    for (int i = 0; i < IN; ++i)
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        uint64_t* w = d + 2 * (i * JM + j) * 64;
        __hip_atomic_store(w, pack2(acc[i][j][0], acc[i][j][1]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(w + 1, pack2(acc[i][j][2], acc[i][j][3]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_sched_barrier(0);
      }
  }
  splitk_published();
  __syncthreads();
  if (tid == 0) sched.last = splitk_arrive(p.counters + (int64_t)expert * tiles + tile, nch);
  __syncthreads();
  if (!sched.last) return;
  splitk_acquired();
  // each of the wave's blocks: 0 + chunk 0 + chunk 1 + ... in chunk order,
  // GB blocks at a time (GB loads in flight per chunk); flat block index
  // b = i * JM + j, as the partials are laid out
  const uint64_t* src = frag_ptr(sched.base_slot);
  const int64_t stride = 2 * tiles * Cfg::NW * (IN * JM) * 64;  // 8-byte words between chunks
  constexpr int NB = IN * JM, GB = NB < 16 ? NB : 16;
#pragma unroll 1
  for (int g0 = 0; g0 < NB; g0 += GB) {
    float4 t[GB];
#pragma unroll
    for (int b = 0; b < GB; ++b) t[b] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 1
    for (int32_t c = 0; c < nch; ++c) {
      const uint64_t* q = src + c * stride + 2 * g0 * 64;
      float4 v[GB];
#pragma unroll
      for (int b = 0; b < GB; ++b) {
        const uint64_t lo = __hip_atomic_load(q + 2 * b * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t hi = __hip_atomic_load(q + 2 * b * 64 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v[b] = make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                           __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
      }
#pragma unroll
      for (int b = 0; b < GB; ++b) {
        t[b].x += v[b].x;
        t[b].y += v[b].y;
        t[b].z += v[b].z;
        t[b].w += v[b].w;
      }
    }
#pragma unroll
    for (int b = 0; b < GB; ++b) {
      const int i = (g0 + b) / JM, j = (g0 + b) % JM;
      const int64_t m = m0 + wm * 16 * JM + j * 16 + L, n = n0 + wn * 16 * IN + i * 16 + 4 * grp;
      if (m >= p.M || n >= p.N) continue;
      const int64_t off = (int64_t)expert * p.dw_se + m * p.dw_sm;
      if (dw_vec) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.dw) + off + n) = t[b];
      } else if constexpr (!VEC_ONLY) {
        const float e[4] = {t[b].x, t[b].y, t[b].z, t[b].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < p.N) store_from_f32(p.dw, p.dw_dtype, off + (n + q) * p.dw_sn, e[q]);
      }
    }
  }
}

template <typename OpT, int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch_wgrad_v3_t(const WgradParams& p, hipStream_t stream) {
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int64_t chunks = p.order == kWgOrderChunkXcd ? (p.grid_chunks + 7) / 8 * 8 : p.grid_chunks;
  const int64_t grid = chunks * tiles;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  const dim3 block(WM * WN * 64);
  if (p.w != nullptr)
    hipLaunchKernelGGL((wgrad_v3_kernel<OpT, BM, BN, WM, WN, STAGES, true>), dim3((unsigned)grid), block, 0, stream, p);
  else
    hipLaunchKernelGGL((wgrad_v3_kernel<OpT, BM, BN, WM, WN, STAGES, false>), dim3((unsigned)grid), block, 0, stream,
                       p);
  return hipGetLastError();
}

template <typename OpT>
hipError_t launch_wgrad_v3_op(const WgradParams& p, hipStream_t stream) {
  int bm, bn;
  wgrad_fast_tile(p.M, p.N, wgrad_dw_vec(p) ? p.tile_choice : kWgTileBase, &bm, &bn);
  if (bm == 256 && bn == 256 && wgrad_dw_vec(p) && p.tile_choice == kWgTile256x256W8)
    return launch_wgrad_v3_t<OpT, 256, 256, 2, 4, 4>(p, stream);
  if (bm == 256 && bn == 256) return launch_wgrad_v3_t<OpT, 256, 256, 2, 2, 4>(p, stream);
  if (bm == 256 && bn == 128) return launch_wgrad_v3_t<OpT, 256, 128, 2, 2, 4>(p, stream);
  if (bm == 128 && bn == 256) return launch_wgrad_v3_t<OpT, 128, 256, 2, 2, 4>(p, stream);
  if (bm == 256) return launch_wgrad_v3_t<OpT, 256, 64, 4, 1, 3>(p, stream);
  if (bm == 64) return launch_wgrad_v3_t<OpT, 64, 256, 1, 4, 3>(p, stream);
  return launch_wgrad_v3_t<OpT, 128, 128, 2, 2, 4>(p, stream);
}

}  // namespace cvmm
