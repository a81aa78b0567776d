// Routed GEMM for a small inner dimension (K <= 128) and a wide output
// (N % 64 == 0): the shape of the ff_up input gradient (K = d_out = 128,
// N = d_in = 1024), the ff_down forward (K = 128, N = 1024) and the SwitchHead
// products (K = 64, N = 2048).  Such a product is bound by its output stores,
// and a tile holds only one or two k stages, so a tile-per-workgroup kernel
// spends most of its life in the dependent prologue (schedule, route rows,
// first loads) and in draining its stores.
//
// Here one workgroup owns a 128-row m-tile and a run of `tpw` n-tiles:
//  * the activation rows (128 x K) are loaded once, straight into the MFMA
//    fragment registers of the waves that use them;
//  * the weight tiles (BN x K) stream through a ring of three LDS buffers by
//    global_load_lds (16 bytes per lane), two tiles ahead of the MFMA work;
//  * every output value is stored from registers as soon as its tile is done
//    (C^T = W-tile x A^T, so a lane holds 4 consecutive columns of one row;
//    two lane swaps make that 8 columns, one 16-byte store, for 16-bit output).
// Loads and stores retire in order on vmcnt, so the wait for weight tile t
// leaves exactly the later ops in flight: the stores of tiles t-2 and t-1 and
// the DMA of tile t+1.  Every lane issues a fixed number of stores per tile
// (rows outside the tile write to a sink), which keeps those counts exact.
#pragma once

#include "cvmm_gemm_nt.h"

namespace cvmm {

// Sink for the stores of rows outside a tile (contents never read).
static __device__ uint4 g_cvmm_store_sink[64];

// s_waitcnt that constrains only vmcnt (gfx9 encoding: vmcnt[3:0],
// expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in bits [15:14]).  The builtin, unlike
// inline asm, is seen by the compiler's own wait-count pass.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without __syncthreads' memory fences (those make the
// compiler wait for every outstanding store and DMA).  LDS visibility is
// arranged explicitly: a wave waits for its own DMA before the barrier.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }

// 16-byte LDS read issued as inline asm.  The compiler does not see it as an
// LDS access, so its wait-count pass inserts no vmcnt wait for in-flight DMA
// into other LDS buffers (it cannot always tell those apart and then waits
// for all of them); the caller orders it after its own DMA wait and barrier
// and must call lds_wait_tied on the results before using them.
typedef unsigned int lds_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ lds_u32x4 lds_read128(const char* p) {
  lds_u32x4 v;
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
  return v;
}

// lgkmcnt(0) tied to the registers of 8 inline-asm LDS reads, so no use of
// them can be scheduled before the wait.
__device__ __forceinline__ void lds_wait_tied(lds_u32x4 (&x)[4], lds_u32x4 (&y)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]));
}

__device__ __forceinline__ uint4 as_uint4(lds_u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// LDS address of a __shared__ object, for inline-asm LDS accesses.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// A 4-byte LDS load as inline asm, waited for at once (see lds_read128): for
// scalar bookkeeping reads inside DMA loops.
__device__ __forceinline__ int32_t lds_load_i32(const void* p) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return v;
}

typedef unsigned int lds_u32x2 __attribute__((ext_vector_type(2)));

// Inline-asm LDS reads (invisible to the compiler's wait-count pass, see
// lds_read128); results are used only after an lgkmcnt wait tied to them.
template <int OFF>
__device__ __forceinline__ lds_u32x2 lds_read_tr(uint32_t a) {
  lds_u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

__device__ __forceinline__ lds_u32x2 lds_read64(uint32_t a) {
  lds_u32x2 v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(a));
  return v;
}

template <int OFF>
__device__ __forceinline__ int32_t lds_read_i32(uint32_t a) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ lds_u32x4 lds_read128_at(uint32_t a) {
  lds_u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

template <int N>
__device__ __forceinline__ void lgkm_wait_tied(int32_t (&r)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]));
#pragma unroll
  for (int i = 1; i < N; ++i) asm volatile("" : "+v"(r[i]));
}

__device__ __forceinline__ void lgkm_wait_frags(lds_u32x2 (&g)[4][2], lds_u32x2 (&x)[4][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(g[0][0]), "+v"(g[0][1]), "+v"(g[1][0]), "+v"(g[1][1]), "+v"(g[2][0]), "+v"(g[2][1]),
                 "+v"(g[3][0]), "+v"(g[3][1]), "+v"(x[0][0]), "+v"(x[0][1]), "+v"(x[1][0]), "+v"(x[1][1]),
                 "+v"(x[2][0]), "+v"(x[2][1]), "+v"(x[3][0]), "+v"(x[3][1]));
}

// Any number of fragments: the wait, then empty statements that hand each
// fragment on (volatile asm keeps its order, so every use follows the wait).
template <int NG, int NX>
__device__ __forceinline__ void lgkm_wait_frags_n(lds_u32x2 (&g)[NG][2], lds_u32x2 (&x)[NX][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(g[0][0]), "+v"(g[0][1]), "+v"(x[0][0]), "+v"(x[0][1]));
#pragma unroll
  for (int i = 1; i < NG; ++i) asm volatile("" : "+v"(g[i][0]), "+v"(g[i][1]));
#pragma unroll
  for (int i = 1; i < NX; ++i) asm volatile("" : "+v"(x[i][0]), "+v"(x[i][1]));
}

__device__ __forceinline__ void lgkm_wait_w(lds_u32x4 (&w)[2]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(w[0]), "+v"(w[1]));
}

// 16-byte chunk swizzle of [k][column] rows read by ds_read_b64_tr_b16 (lane
// L of a 16-lane group reads 8 bytes of row L / 4 at column 4 * (L % 4); the
// group's 4 rows x 32 bytes land on distinct banks).  The rule sees row bits
// 0, 1 and 3 only, so rows r and r + 4, r + 32 share it.  CPR = chunks per
// row: 16 or 32 (256- or 512-byte rows: the 256-byte rule within each half)
// or 8 (128-byte rows).
template <int CPR>
__device__ __forceinline__ int tr_row_swz(int row) {
  if constexpr (CPR >= 16) return 2 * ((row & 3) | (((row >> 3) & 1) << 2));
  else return 2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1));
}

// 16-byte chunk swizzle of the panel kernel's [n][k] weight tiles, whose
// 16-lane fragment reads take one chunk of 16 consecutive rows: 256-byte rows
// put chunk c of row n at c ^ (n & 15), 128-byte rows (two per 256 bytes) at
// c ^ ((n >> 1) & 7), so those 16 chunks fill 16 distinct 16-byte bank groups.
template <int CPR>
__device__ __forceinline__ int panel_swz(int row) {
  if constexpr (CPR >= 16) return row & 15;
  else return (row >> 1) & 7;
}

// Wait until at most `ahead` slices (D DMA instructions each) are in flight.
template <int D, int K>
__device__ __forceinline__ void vm_wait_slices(int ahead) {
  if constexpr (K == 0) {
    vm_wait<0>();
  } else {
    if (ahead >= K) vm_wait<K * D>();
    else vm_wait_slices<D, K - 1>(ahead);
  }
}

// WM waves along the m-tile (64 rows each), 4 / WM along the n-tile: 128-row
// tiles (2 x 2 waves, three workgroups per CU) or 256-row tiles (4 x 1,
// two per CU, half the weight reads per output row).
template <int KP, int BN, int WM_>
struct PanelCfg {
  static constexpr int WM = WM_, WN = 4 / WM_;
  static constexpr int BM = 64 * WM;
  static constexpr int CPR = KP / 8;                  // 16-byte chunks per weight row
  static constexpr int TILE_BYTES = BN * KP * 2;      // one weight tile in LDS
  static constexpr int D = TILE_BYTES / (4 * 1024);   // DMA instructions per wave per tile
  static constexpr int NI = BN / (16 * WN);           // 16-column blocks per wave (wave: 64 x BN/WN)
  static constexpr int KS = KP / 32;                  // MFMA k steps
  static constexpr int OCC = WM == 2 ? 3 : 2;         // workgroups per CU (LDS 52.8 / 57.5 KB)
  static_assert(CPR == 8 || CPR == 16, "swizzle for 128- or 256-byte rows");
  static_assert(WM == 2 || WM == 4, "128- or 256-row tiles");
};

template <typename OpT, typename OutT, int KP, int BN, int Role, int WM>
__global__ __launch_bounds__(kGemmThreads, (PanelCfg<KP, BN, WM>::OCC)) void routed_gemm_panel_kernel(
    const GemmParams p, int32_t tpw) {
  using Cfg = PanelCfg<KP, BN, WM>;
  // store instructions per lane per tile: one per 16-byte piece
  constexpr int S = sizeof(OutT) == 4 ? 4 * Cfg::NI : 2 * Cfg::NI;
  static_assert(2 * S + Cfg::D < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char ring0[Cfg::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) char ring1[Cfg::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) char ring2[Cfg::TILE_BYTES];
  __shared__ RouteMeta<Cfg::BM> meta;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n_ntiles = p.N / BN;
  const int64_t n_groups = (n_ntiles + tpw - 1) / tpw;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tile = id / n_groups;
  const int64_t nt0 = (id % n_groups) * tpw;
  const int T = (int)((n_ntiles - nt0) < tpw ? (n_ntiles - nt0) : tpw);

  if (!gemm_schedule<Cfg::BM>(p, tile, meta)) {
    zero_unrouted_cols<Cfg::BM>(p, meta, tile, gridDim.x / n_groups, nt0 * BN, (nt0 + T) * BN, -1);
    return;
  }
  const int32_t expert = meta.expert;

  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int fr = lane & 15, fq = lane >> 4;
  const char* zero = reinterpret_cast<const char*>(g_cvmm_zero_page);

  // ---- activation fragments (fixed over the n-tiles), output rows, weights --
  uint4 af[4][Cfg::KS];
  int64_t orow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = wm * 64 + j * 16 + fr;
    const int64_t ar = meta.arow[m];
    orow[j] = meta.orow[m];
#pragma unroll
    for (int ks = 0; ks < Cfg::KS; ++ks) {
      const int k = (ks * 4 + fq) * 8;
      const char* src = (ar >= 0 && k < p.K) ? reinterpret_cast<const char*>(p.a) + (ar * p.a_ld + k) * 2
                                             : zero + lane * 16;
      af[j][ks] = *reinterpret_cast<const uint4*>(src);
    }
  }
  issue_fence();

  // ---- weight tile t -> LDS buffer (row = n, 16-byte chunk c at c ^ panel_swz(n))
  const char* bexp = reinterpret_cast<const char*>(p.b) + (int64_t)expert * p.b_se * 2;
  auto issue = [&](int t, char* buf) {
    const int64_t nb = (nt0 + t) * BN;
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      const int q = (wave * Cfg::D + j) * 64 + lane;
      const int row = q / Cfg::CPR;
      const int c = (q % Cfg::CPR) ^ panel_swz<Cfg::CPR>(row);
      const char* src = c * 8 < p.K ? bexp + ((nb + row) * p.b_sn + c * 8) * 2 : zero + lane * 16;
      dma16(src, buf + (wave * Cfg::D + j) * 1024);
    }
  };

  // ---- MFMA on one weight tile + stores of its outputs ------------------------
  // output row pointers (a sink for rows outside the tile)
  char* rowp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    rowp[j] = orow[j] >= 0 ? reinterpret_cast<char*>(p.out) + orow[j] * p.out_ld * (int64_t)sizeof(OutT) : nullptr;
  char* sink = reinterpret_cast<char*>(g_cvmm_store_sink) + lane * 16;
  auto compute_store = [&](int t, const char* buf) {
    f32x4_t acc[Cfg::NI][4];
#pragma unroll
    for (int i = 0; i < Cfg::NI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < Cfg::KS; ++ks) {
      uint4 bf[Cfg::NI];
#pragma unroll
      for (int i = 0; i < Cfg::NI; ++i) {
        const int n = wn * (BN / Cfg::WN) + i * 16 + fr;
        const int c = ks * 4 + fq;
        bf[i] = *reinterpret_cast<const uint4*>(buf + n * (Cfg::CPR * 16) + ((c ^ panel_swz<Cfg::CPR>(n)) << 4));
      }
#pragma unroll
      for (int i = 0; i < Cfg::NI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MfmaOp<OpT>::step(acc[i][j], bf[i], af[j][ks]);
    }
    // lane holds C[m = wm*64 + j*16 + fr][n = nwave + i*16 + 4*fq + {0..3}]
    const int64_t nwave = (nt0 + t) * BN + wn * (BN / Cfg::WN);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(OutT) == 4) {
#pragma unroll
        for (int i = 0; i < Cfg::NI; ++i) {
          char* dst = rowp[j] != nullptr ? rowp[j] + (nwave + i * 16 + 4 * fq) * 4 : sink;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        }
      } else {
        // 16-bit output: blocks i = 2p, 2p+1 hold columns 32p + [0, 32) of
        // the row in 4-column pieces, lane group fq having piece fq of each.
        // Swapping lanes 32-63 of the first block with lanes 0-31 of the
        // second, then odd 16-lane rows of the first with even rows of the
        // second, leaves group fq with columns 32p + 8*fq + [0, 8): one
        // 16-byte store per lane.
#pragma unroll
        for (int pr = 0; pr < Cfg::NI / 2; ++pr) {
          uint32_t a[2], b[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            union { uint32_t u; OutT e[2]; } pa, pb;
            pa.e[0] = (OutT)acc[2 * pr][j][2 * h];
            pa.e[1] = (OutT)acc[2 * pr][j][2 * h + 1];
            pb.e[0] = (OutT)acc[2 * pr + 1][j][2 * h];
            pb.e[1] = (OutT)acc[2 * pr + 1][j][2 * h + 1];
            a[h] = pa.u;
            b[h] = pb.u;
          }
          uint4 v;
          {
            const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
            const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s0[1], false, false);
            const auto t1 = __builtin_amdgcn_permlane16_swap(s1[0], s1[1], false, false);
            v = make_uint4(t0[0], t1[0], t0[1], t1[1]);
          }
          char* dst = rowp[j] != nullptr ? rowp[j] + (nwave + pr * 32 + 8 * fq) * 2 : sink;
          *reinterpret_cast<uint4*>(dst) = v;
        }
      }
    }
  };

  // ---- wait for weight tile t: the ops issued after it may stay in flight -----
  // issue order: B0 B1 | B2 S0 | B3 S1 | ... (iteration t issues B(t+2), then S(t))
  auto wait_tile = [&](int t) {
    const bool more = t + 1 < T;  // B(t+1) was issued after B(t)
    if (t == 0) {
      if (more) vm_wait<Cfg::D>(); else vm_wait<0>();
    } else if (t == 1) {
      if (more) vm_wait<S + Cfg::D>(); else vm_wait<S>();
    } else {
      if (more) vm_wait<2 * S + Cfg::D>(); else vm_wait<2 * S>();
    }
  };

  issue(0, ring0);
  issue_fence();
  if (T > 1) issue(1, ring1);
  issue_fence();
  // The activation rows scaled by their routing weights (xs_out), from the
  // fragments in registers: rnd_op(rnd_op(w) * a), each row once (row block j
  // of the tile by group j % G of its min(groups, 4) workgroups).  Issued
  // after the first weight DMAs, so the fragment loads' wait leaves those in
  // flight; the extra stores only make the tile waits below stricter.
  if (p.xs_out != nullptr) {
    const int64_t grp = id % n_groups;
    const int64_t G = n_groups < 4 ? n_groups : 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = wm * 64 + j * 16 + fr;
      const int64_t ar = meta.arow[m], wi = meta.widx[m];
      if (grp != j % G || ar < 0 || wi < 0) continue;
      const float sc = round_to(load_as_f32(p.xs_w, p.xs_w_dtype, wi), DTypeOf<OpT>::value);
#pragma unroll
      for (int ks = 0; ks < Cfg::KS; ++ks) {
        const int k = (ks * 4 + fq) * 8;
        if (k >= p.K) continue;
        Chunk16 in, o;
        in.u = af[j][ks];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          reinterpret_cast<OpT*>(&o)[i] = from_f32<OpT>(sc * to_f32(reinterpret_cast<const OpT*>(&in)[i]));
        *reinterpret_cast<uint4*>(static_cast<OpT*>(p.xs_out) + ar * p.K + k) = o.u;
      }
    }
  }
  issue_fence();
  // three statically named buffers: every LDS access names its buffer, so the
  // compiler can tell the in-flight DMA targets from the buffer being read
  for (int t = 0; t < T; t += 3) {
    wait_tile(t);
    wg_barrier();
    if (t + 2 < T) issue(t + 2, ring2);
    issue_fence();
    compute_store(t, ring0);
    issue_fence();
    if (t + 1 >= T) break;

    wait_tile(t + 1);
    wg_barrier();
    if (t + 3 < T) issue(t + 3, ring0);
    issue_fence();
    compute_store(t + 1, ring1);
    issue_fence();
    if (t + 2 >= T) break;

    wait_tile(t + 2);
    wg_barrier();
    if (t + 4 < T) issue(t + 4, ring1);
    issue_fence();
    compute_store(t + 2, ring2);
    issue_fence();
  }
}

// The panel kernel applies: plain stores of the products rounded once to the
// output type (no routing-weight scale, no routing-weight gradient), output in
// the op type or fp32, K <= 128, N a multiple of 64, 8-byte (16-bit output) or
// 16-byte (fp32) aligned output rows.
inline bool panel_eligible(const GemmParams& p, int32_t op) {
  const size_t osz = p.out_dtype == kF32 ? 16 : 8;
  const size_t esz = p.out_dtype == kF32 ? 4 : 2;
  return p.K <= 128 && p.b_sk == 1 && p.act == 0 && p.epi == kEpiStore && p.dg == nullptr && p.w == nullptr &&
         p.out != nullptr &&
         p.val_dtype == p.out_dtype && (p.out_dtype == op || p.out_dtype == kF32) && p.N % 64 == 0 &&
         (reinterpret_cast<uintptr_t>(p.out) % osz) == 0 && ((size_t)p.out_ld * esz) % osz == 0;
}

// n-tiles per workgroup: enough workgroups for about one per slot (occ per
// CU x 256 CUs), n-tiles split evenly over the groups of an m-tile.
// Measured with 128-row tiles (n-tiles per workgroup 2/4/6/8/16): ff_up
// grad-input 70.9 / 52.6 / 50.6 / 47.6 / 49.2 us, ff_down forward 70.7 / 52.1
// / 51.4 / 46.7 / 48.7 us; with 256-row tiles 4/5/6/8/11/16: 44.5 / 48.8 /
// 44.5 / 43.5 / 51.9 / 51.1 us (ff_up; ff_down forward 45.0 -> 43.9 us from
// 6 to 8); the SwitchHead shapes (4352 m-tiles) are best with all n-tiles in
// one group.
inline int32_t panel_tiles_per_wg(int64_t m_tiles, int64_t n_ntiles, int occ) {
  const int64_t slots = occ * 256;
  int64_t groups = (slots + m_tiles - 1) / (m_tiles > 0 ? m_tiles : 1);
  if (groups < 1) groups = 1;
  if (groups > n_ntiles) groups = n_ntiles;
  return (int32_t)((n_ntiles + groups - 1) / groups);
}

template <typename OpT, typename OutT, int KP, int BN, int WM>
hipError_t launch_routed_gemm_panel_t(const GemmParams& p, hipStream_t stream) {
  using Cfg = PanelCfg<KP, BN, WM>;
  // m-tile slots: every expert's last tile may be partial
  const int64_t m_tiles = (p.n_routes + Cfg::BM - 1) / Cfg::BM + (p.n_experts < p.n_routes ? p.n_experts : p.n_routes);
  const int64_t n_ntiles = p.N / BN;
  const int32_t tpw = p.panel_tpw > 0 ? (int32_t)(p.panel_tpw < n_ntiles ? p.panel_tpw : n_ntiles)
                                      : panel_tiles_per_wg(m_tiles, n_ntiles, Cfg::OCC);
  const int64_t n_groups = (n_ntiles + tpw - 1) / tpw;
  const int64_t grid = m_tiles * n_groups;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.role == 0)
    hipLaunchKernelGGL((routed_gemm_panel_kernel<OpT, OutT, KP, BN, 0, WM>), dim3((unsigned)grid),
                       dim3(kGemmThreads), 0, stream, p, tpw);
  else
    hipLaunchKernelGGL((routed_gemm_panel_kernel<OpT, OutT, KP, BN, 1, WM>), dim3((unsigned)grid),
                       dim3(kGemmThreads), 0, stream, p, tpw);
  return hipGetLastError();
}

// 256-row tiles when the average expert fills one (half the weight traffic
// per output row; measured on the ff_up grad-input shape: 43.8 us against
// 48.4 us for 128-row tiles), else 128-row tiles.
template <typename OpT, typename OutT, int KP, int BN>
hipError_t launch_routed_gemm_panel_m(const GemmParams& p, hipStream_t stream) {
  // 256-row tiles keep 2 * (stores per tile) + DMA per tile within vmcnt
  constexpr int kWideStores = (sizeof(OutT) == 4 ? 4 : 2) * (BN / 16);
  if constexpr (2 * kWideStores + PanelCfg<KP, BN, 4>::D < 64) {
    if (p.n_experts > 0 && p.n_routes >= 256 * (int64_t)p.n_experts)
      return launch_routed_gemm_panel_t<OpT, OutT, KP, BN, 4>(p, stream);
  }
  return launch_routed_gemm_panel_t<OpT, OutT, KP, BN, 2>(p, stream);
}

template <typename OpT, typename OutT>
hipError_t launch_routed_gemm_panel_out(const GemmParams& p, hipStream_t stream) {
  if (p.K <= 64) {
    if (p.N % 128 == 0) return launch_routed_gemm_panel_m<OpT, OutT, 64, 128>(p, stream);
    return launch_routed_gemm_panel_m<OpT, OutT, 64, 64>(p, stream);
  }
  return launch_routed_gemm_panel_m<OpT, OutT, 128, 64>(p, stream);
}


}  // namespace cvmm
