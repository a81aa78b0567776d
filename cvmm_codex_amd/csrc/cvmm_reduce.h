// Reduce GEMM: the top-k sum of routed products, out[t] = sum over the routes
// r of token t of w_r * rnd(A_r . B_e(r)), computed without the route-ordered
// [R][N] buffer that the routed GEMM + combine pair writes and reads back
// (2.1 GB per step for the SwitchHead projections, top-64).
//
// A workgroup owns a group of TG tokens and a slice of 64 output columns and
// keeps their fp32 sums in LDS.  It walks the experts in order; the routes of
// expert e whose token lies in the group are contiguous in the sorted order
// (the stable sort keeps route order within an expert), and their A rows
// were gathered into that order beforehand, so every stage -- up to MAXR
// routes of one expert, listed beforehand per group -- is three contiguous
// DMA copies: the A rows, the expert's 64 x K weight slice and the routes'
// (token, weight) info.  Stages stream through a ring of STAGES LDS slots
// (one barrier per stage, exact vmcnt waits as in the other DMA rings; rows
// past the stage's routes are copied from the zero page).  Each stage's LDS
// reads are issued together and waited for once.
//
// The waves form RP x CQ: wave (rw, cw) computes the products of the route
// blocks rb with rb % RP == rw and the columns of part cw (a lane ends with
// one column of 4 routes) and adds the rounded products into its tokens'
// sums (LDS reads, then writes).  The sums are stored column-major with a
// row stride of TG + 1 floats: the 16 lanes that update one route's 16
// columns hit 16 consecutive banks.  A token meets an expert once, so the
// routes of a stage have distinct tokens and the waves' updates never meet
// (two waves that share columns hold different routes); the stages run in
// expert order, so a token's routes are summed in expert order: deterministic
// without atomics or extra barriers.  A token that picked one expert more
// than once has adjacent routes in one stage; such a stage adds its routes
// one at a time, in order.
//
// Traffic: every workgroup reads its group's A rows and its slice of every
// expert's weights.  Workgroups are ordered so that the ones resident on an
// XCD at a time share 4 token groups and 8 column slices: they walk the
// experts at about the same pace, so each A row and weight slice comes from
// HBM about once per XCD and from the XCD's L2 after that.
//
// Cost: every product value costs an LDS read and write of its sum, on top of
// the operand and DMA traffic; at the SwitchHead size (524288 routes x 2048
// columns) the kernel measured ~1.45 ms against ~0.74-0.97 ms for the
// route-buffer GEMM + combine, so the library takes it only when asked
// (CVMM_TUNE_REDUCE_MIN_TOPK), for its ~30x smaller workspace.
#pragma once

#include "cvmm_gemm_ring.h"

namespace cvmm {

template <int K, int MAXR, int STAGES, int TG, int RP, int CQ>
struct ReduceCfg {
  static constexpr int NW = RP * CQ;               // waves
  static constexpr int THREADS = 64 * NW;
  static constexpr int NC = kReduceCols;           // output columns per workgroup
  static constexpr int ROWB = K * 2;               // bytes per A / weight row
  static constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROWB;          // rows per 1 KB DMA instruction
  static constexpr int A_BYTES = MAXR * ROWB;
  static constexpr int W_BYTES = NC * ROWB;
  static constexpr int I_BYTES = 1024;             // 128 RouteInfo (MAXR used)
  static constexpr int SLOT = A_BYTES + W_BYTES + I_BYTES;
  static constexpr int A_INSTS = A_BYTES / 1024, W_INSTS = W_BYTES / 1024;
  static constexpr int INSTS = SLOT / 1024;        // DMA instructions per stage
  static constexpr int D_LO = INSTS / NW;          // per wave: waves < INSTS % NW issue one more
  static constexpr int D_HI = D_LO + (INSTS % NW != 0 ? 1 : 0);
  static constexpr int KS = K / 32;                // MFMA k steps
  static constexpr int RB = MAXR / 16;             // 16-route blocks per stage
  static constexpr int RBW = RB / RP;              // route blocks per wave
  static constexpr int NBW = 4 / CQ;               // 16-column blocks per wave
  static constexpr int ST = kReduceMaxStages;
  static constexpr int ACC_LD = TG + 1;            // sums: [NC][TG + 1] floats
  static constexpr int LDS = STAGES * SLOT + NC * ACC_LD * 4 + ST * 8;
  static_assert(MAXR % 16 == 0 && MAXR <= 128 && RB % RP == 0, "route blocks per wave, info in one DMA");
  static_assert(K == 64 || K == 128, "64 or 128 k");
  static_assert(NC == 64 && (CQ == 1 || CQ == 2 || CQ == 4), "16-column blocks; sum rows of 16 chunks");
  static_assert(A_BYTES % 1024 == 0 && W_BYTES % 1024 == 0, "whole DMA instructions");
  static_assert(D_LO >= 1 && (STAGES - 2) * D_HI < 64, "vmcnt range");
  static_assert(LDS <= 160 * 1024, "LDS");
};

// Group and slice of workgroup `id`: blocks of kBG groups x all slices, slice
// outer and group inner within a block, so that consecutive ids (one XCD's
// share, see xcd_remap) cover few groups and few slices at a time.
__device__ __forceinline__ void reduce_tile_of(int64_t id, int64_t n_groups, int64_t n_slices, int64_t* g,
                                               int64_t* sl) {
  constexpr int64_t kBG = 4;
  const int64_t gb = id / (n_slices * kBG);
  const int64_t r = id - gb * n_slices * kBG;
  const int64_t bg = n_groups - gb * kBG < kBG ? n_groups - gb * kBG : kBG;
  *sl = r / bg;
  *g = gb * kBG + r % bg;
}

#define CVMM_TIE(x) asm volatile("" : "+v"(x))

// RV: each route's product is rounded to OpT (else kept in fp32).
template <typename OpT, typename OutT, int K, int MAXR, int STAGES, int TG, int RP, int CQ, bool RV>
__global__ __launch_bounds__(64 * RP * CQ, 1) void routed_reduce_kernel(const ReduceParams p) {
  using Cfg = ReduceCfg<K, MAXR, STAGES, TG, RP, CQ>;
  constexpr int NC = Cfg::NC, NW = Cfg::NW, RBW = Cfg::RBW, NBW = Cfg::NBW, KS = Cfg::KS;
  __shared__ __attribute__((aligned(1024))) char ring[STAGES * Cfg::SLOT];
  __shared__ __attribute__((aligned(16))) float acc_lds[NC * Cfg::ACC_LD];
  __shared__ __attribute__((aligned(8))) ReduceStage s_st[Cfg::ST];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = wave % RP, cw = wave / RP;  // route-block class, column part
  const int64_t n_slices = p.N / NC;
  int64_t g, sl;
  reduce_tile_of(xcd_remap(blockIdx.x, gridDim.x), p.n_groups, n_slices, &g, &sl);
  const int64_t n0 = sl * NC;
  const int64_t t0 = g * TG;

  // ---- prologue: the group's stage list, zeroed sums
  int32_t n_st = p.n_stages[g];
  n_st = n_st < Cfg::ST ? n_st : Cfg::ST;
  for (int i = tid; i < n_st; i += Cfg::THREADS) s_st[i] = p.stages[g * Cfg::ST + i];
  for (int i = tid; i < NC * Cfg::ACC_LD; i += Cfg::THREADS) acc_lds[i] = 0.f;
  __syncthreads();

  // ---- DMA geometry: instruction i of the stage fills slot bytes [i*1024, +1024)
  const int n_mine = wave < Cfg::INSTS % NW ? Cfg::D_HI : Cfg::D_LO;
  const int first = wave * Cfg::D_LO + (wave < Cfg::INSTS % NW ? wave : Cfg::INSTS % NW);
  const char* zero = reinterpret_cast<const char*>(g_cvmm_zero_page);
  const char* abase = reinterpret_cast<const char*>(p.a);
  const char* bbase = reinterpret_cast<const char*>(p.b);
  const char* ibase = reinterpret_cast<const char*>(p.info);
  // this wave's DMA instructions j: region (0 A rows, 1 weight rows, 2 info;
  // wave-uniform), the A row of this lane and its byte offset in the region
  int32_t d_reg[Cfg::D_HI], d_row[Cfg::D_HI];
  int64_t d_off[Cfg::D_HI];
#pragma unroll
  for (int j = 0; j < Cfg::D_HI; ++j) {
    const int i = first + j;
    const int ra = i * Cfg::RPI + lane / Cfg::CPR, rw_ = (i - Cfg::A_INSTS) * Cfg::RPI + lane / Cfg::CPR;
    d_reg[j] = i < Cfg::A_INSTS ? 0 : (i < Cfg::A_INSTS + Cfg::W_INSTS ? 1 : 2);
    d_row[j] = d_reg[j] == 0 ? ra : 0;
    d_off[j] = d_reg[j] == 0 ? (int64_t)ra * Cfg::ROWB + (((lane % Cfg::CPR) ^ ring_swz<Cfg::CPR>(ra)) << 4)
             : d_reg[j] == 1 ? (n0 + rw_) * p.b_sn * 2 + (((lane % Cfg::CPR) ^ ring_swz<Cfg::CPR>(rw_)) << 4)
                             : (int64_t)lane * 16;
  }
  // stage (first sorted position r, expert * 256 + routes), uniform
  auto issue = [&](int32_t r, int32_t er, int slot) {
    char* dst = ring + slot * Cfg::SLOT;
    const int rows = er & 255;
    const char* a_seg = abase + (int64_t)r * Cfg::ROWB;
    const char* b_seg = bbase + (int64_t)(er >> 8) * p.b_se * 2;
    const char* i_seg = ibase + (int64_t)r * sizeof(RouteInfo);  // info padded by kReducePad
#pragma unroll
    for (int j = 0; j < Cfg::D_HI; ++j) {
      if (j >= n_mine) break;
      const char* src = d_reg[j] == 0 ? (d_row[j] < rows ? a_seg + d_off[j] : zero)
                      : d_reg[j] == 1 ? b_seg + d_off[j] : i_seg + d_off[j];
      dma16(src, dst + (first + j) * 1024);
    }
  };
  auto wait_for = [&](int ahead) {  // ahead: stages issued after the one waited for
    if (n_mine == Cfg::D_HI) vm_wait_slices<Cfg::D_HI, STAGES - 2>(ahead);
    else vm_wait_slices<Cfg::D_LO, STAGES - 2>(ahead);
  };

  // ---- fragments: routes are the MFMA rows, weight rows n its columns
  const int fr = lane & 15, fq = lane >> 4;
  uint32_t w_off[NBW][KS], a_off[RBW][KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      const int row = (cw * NBW + nb) * 16 + fr;
      w_off[nb][ks] = Cfg::A_BYTES + row * Cfg::ROWB + (((ks * 4 + fq) ^ ring_swz<Cfg::CPR>(row)) << 4);
    }
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
      const int row = (j * RP + rw) * 16 + fr;
      a_off[j][ks] = row * Cfg::ROWB + (((ks * 4 + fq) ^ ring_swz<Cfg::CPR>(row)) << 4);
    }
  }
  const uint32_t ring_a = lds_addr(ring);
  const uint32_t acc_a = lds_addr(acc_lds);
  const uint32_t st_a = lds_addr(s_st);
  // sum of token tr, column c
  auto acc_addr = [&](int32_t tr, int c) { return acc_a + (uint32_t)((c * Cfg::ACC_LD + tr) * 4); };

  // ---- ring prologue: descriptors of the first stages (no DMA in flight yet)
  int32_t cur_r = 0, cur_er = 0, iss_r = 0, iss_er = 0, pro_r[STAGES - 1], pro_er[STAGES - 1];
  if (n_st > 0) { cur_r = s_st[0].r; cur_er = s_st[0].er; }
  if (STAGES - 1 < n_st) { iss_r = s_st[STAGES - 1].r; iss_er = s_st[STAGES - 1].er; }
#pragma unroll
  for (int s0 = 0; s0 < STAGES - 1; ++s0) {
    pro_r[s0] = s0 < n_st ? s_st[s0].r : 0;
    pro_er[s0] = s0 < n_st ? s_st[s0].er : 0;
  }
  issue_fence();
#pragma unroll
  for (int s0 = 0; s0 < STAGES - 1; ++s0) {
    if (s0 < n_st) {
      issue(pro_r[s0], pro_er[s0], s0);
      issue_fence();
    }
  }

  int cur = 0;
  for (int s = 0; s < n_st; ++s) {
    const int last = s + STAGES - 2 < n_st - 1 ? s + STAGES - 2 : n_st - 1;  // last stage issued so far
    wait_for(last - s);
    wg_barrier();
    if (s + STAGES - 1 < n_st) {
      issue(iss_r, iss_er, cur == 0 ? STAGES - 1 : cur - 1);
      issue_fence();
    }
    const int rows = cur_er & 255;  // uniform over the workgroup
    const uint32_t base = ring_a + cur * Cfg::SLOT;
    const uint32_t info_a = base + Cfg::A_BYTES + Cfg::W_BYTES;

    // ---- every LDS read of the stage, one wait
    lds_u32x4 wf[NBW][KS], af[RBW][KS];
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) wf[nb][ks] = lds_read128_at<0>(base + w_off[nb][ks]);
#pragma unroll
    for (int j = 0; j < RBW; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        af[j][ks] = (j * RP + rw) * 16 < rows ? lds_read128_at<0>(base + a_off[j][ks]) : lds_u32x4{0, 0, 0, 0};
    // info of this lane's routes 4 fq .. 4 fq + 3 of every block
    lds_u32x4 inf[RBW][2];
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
      const uint32_t ia = info_a + ((j * RP + rw) * 16 + 4 * fq) * (uint32_t)sizeof(RouteInfo);
      inf[j][0] = lds_read128_at<0>(ia);
      inf[j][1] = lds_read128_at<16>(ia);
    }
    lds_u32x2 nx0 = lds_read64(info_a + lane * (uint32_t)sizeof(RouteInfo));
    lds_u32x2 nx1 = lds_read64(info_a + (lane + 1) * (uint32_t)sizeof(RouteInfo));
    lds_u32x2 nx2 = lds_read64(info_a + (lane + 64) * (uint32_t)sizeof(RouteInfo));
    lds_u32x2 nx3 = lds_read64(info_a + (lane + 65) * (uint32_t)sizeof(RouteInfo));
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(nx0), "+v"(nx1), "+v"(nx2), "+v"(nx3));
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) CVMM_TIE(wf[nb][ks]);
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
      CVMM_TIE(inf[j][0]);
      CVMM_TIE(inf[j][1]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) CVMM_TIE(af[j][ks]);
    }

    // ---- products: RBW route blocks x NBW column blocks of this wave
    f32x4_t acc[RBW][NBW];
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) acc[j][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if ((j * RP + rw) * 16 < rows) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) MfmaOp<OpT>::step(acc[j][nb], as_uint4(af[j][ks]), as_uint4(wf[nb][ks]));
      }
    }

    // ---- whether two routes of the stage share a token (uniform over the
    // workgroup); this lane's values: column fr of block nb, routes 4 fq + q
    const bool same = (lane + 1 < rows && (int32_t)nx0.x >= 0 && nx0.x == nx1.x) ||
                      (lane + 65 < rows && (int32_t)nx2.x >= 0 && nx2.x == nx3.x);
    const bool shared_token = __builtin_amdgcn_ballot_w64(same) != 0;
    float v[RBW][NBW][4];
    int32_t trs[RBW][4];
    bool mine[RBW][4];
#pragma unroll
    for (int j = 0; j < RBW; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const lds_u32x4& h = inf[j][q >> 1];
        const int32_t o = (int32_t)((q & 1) ? h.z : h.x);
        const float wv = __uint_as_float((q & 1) ? h.w : h.y);
        trs[j][q] = o - (int32_t)t0;
        mine[j][q] = (j * RP + rw) * 16 + 4 * fq + q < rows && o >= 0 && trs[j][q] >= 0 && trs[j][q] < TG;
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          // (the weight is 1 when unweighted)
          const float x = acc[j][nb][q];
          v[j][nb][q] = wv * (RV ? (float)(OpT)x : x);
        }
      }
    }
    // sum addresses of column block 0 (block nb: + nb * NBOFF); a lane whose
    // route is absent updates the padding float of its column instead
    constexpr uint32_t NBOFF = 16 * Cfg::ACC_LD * 4;
    uint32_t ab[RBW][4];
#pragma unroll
    for (int j = 0; j < RBW; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ab[j][q] = acc_a + (uint32_t)(((cw * NBW * 16 + fr) * Cfg::ACC_LD + (mine[j][q] ? trs[j][q] : TG)) * 4);
    auto rd = [&](uint32_t a, int nb) {
      float x;
      if (nb == 0) asm volatile("ds_read_b32 %0, %1" : "=v"(x) : "v"(a));
      else if (nb == 1) asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(x) : "v"(a), "i"(NBOFF));
      else if (nb == 2) asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(x) : "v"(a), "i"(2 * NBOFF));
      else asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(x) : "v"(a), "i"(3 * NBOFF));
      return x;
    };
    auto wr = [&](uint32_t a, int nb, float x) {
      if (nb == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(x) : "memory");
      else if (nb == 1) asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(a), "v"(x), "i"(NBOFF) : "memory");
      else if (nb == 2) asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(a), "v"(x), "i"(2 * NBOFF) : "memory");
      else asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(a), "v"(x), "i"(3 * NBOFF) : "memory");
    };
    if (!shared_token) {
      // every route of the stage has its own token: the stage's updates touch
      // distinct sums -- all reads, one wait, all writes
      float old[RBW][4][NBW];
#pragma unroll
      for (int j = 0; j < RBW; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) old[j][q][nb] = rd(ab[j][q], nb);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < RBW; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) {
            CVMM_TIE(old[j][q][nb]);
            wr(ab[j][q], nb, old[j][q][nb] + v[j][nb][q]);
          }
    } else {
      // one route at a time, in stage order: block by block (the waves of a
      // column part own the blocks in turn), a block's routes one by one
#pragma unroll
      for (int rb = 0; rb < Cfg::RB; ++rb) {
        const int j = rb / RP;
        if (rb % RP == rw) {
#pragma unroll 1
          for (int i = 0; i < 16; ++i) {
            const int q = i & 3;
            if (fq == (i >> 2)) {
              const uint32_t a = q == 0 ? ab[j][0] : q == 1 ? ab[j][1] : q == 2 ? ab[j][2] : ab[j][3];
#pragma unroll
              for (int nb = 0; nb < NBW; ++nb) {
                const float add = q == 0 ? v[j][nb][0] : q == 1 ? v[j][nb][1] : q == 2 ? v[j][nb][2] : v[j][nb][3];
                float x = rd(a, nb);
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x));
                wr(a, nb, x + add);
              }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          }
        }
        wg_barrier();
      }
    }
    // ---- next descriptors; the wait also covers this stage's adds, so the
    // next barrier finds them done and the slot read
    const int s_cur = s + 1 < n_st ? s + 1 : s;
    const int s_iss = s + STAGES < n_st ? s + STAGES : s;
    lds_u32x2 dc = lds_read64(st_a + (uint32_t)s_cur * 8);
    lds_u32x2 di = lds_read64(st_a + (uint32_t)s_iss * 8);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(dc), "+v"(di));
    cur_r = __builtin_amdgcn_readfirstlane((int)dc.x);
    cur_er = __builtin_amdgcn_readfirstlane((int)dc.y);
    iss_r = __builtin_amdgcn_readfirstlane((int)di.x);
    iss_er = __builtin_amdgcn_readfirstlane((int)di.y);
    cur = cur + 1 == STAGES ? 0 : cur + 1;
  }
  vm_wait<0>();
  __syncthreads();

  // ---- sums -> output rows (rounded to mid, then the output type)
  for (int i = tid; i < TG * (NC / 8); i += Cfg::THREADS) {
    const int r = i % TG, c8 = (i / TG) * 8;  // token r, columns c8 .. c8 + 7
    const int64_t t = t0 + r;
    if (t >= p.n_tokens) continue;
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      v[q] = acc_lds[(c8 + q) * Cfg::ACC_LD + r];
      if (p.mid_dtype >= 0) v[q] = round_to(v[q], p.mid_dtype);
    }
    OutT* dst = reinterpret_cast<OutT*>(p.out) + t * p.out_ld + n0 + c8;
    if constexpr (sizeof(OutT) == 4) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      union { uint4 u; OutT h[8]; } pk;
#pragma unroll
      for (int q = 0; q < 8; ++q) pk.h[q] = (OutT)v[q];
      *reinterpret_cast<uint4*>(dst) = pk.u;
    }
  }
}

#undef CVMM_TIE

template <typename OpT, typename OutT, int K, int MAXR, int STAGES, int TG, int RP, int CQ>
hipError_t launch_routed_reduce_t(const ReduceParams& p, hipStream_t stream) {
  if (p.group != TG || p.K != K || p.maxr != MAXR) return hipErrorInvalidValue;
  const int64_t grid = (int64_t)p.n_groups * (p.N / kReduceCols);
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.val_dtype == DTypeOf<OpT>::value)
    hipLaunchKernelGGL((routed_reduce_kernel<OpT, OutT, K, MAXR, STAGES, TG, RP, CQ, true>), dim3((unsigned)grid),
                       dim3(64 * RP * CQ), 0, stream, p);
  else if (p.val_dtype == kF32)
    hipLaunchKernelGGL((routed_reduce_kernel<OpT, OutT, K, MAXR, STAGES, TG, RP, CQ, false>), dim3((unsigned)grid),
                       dim3(64 * RP * CQ), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// 8 waves (2 route classes x 4 column quarters): two waves per SIMD.
template <typename OpT, typename OutT>
hipError_t launch_routed_reduce_out(const ReduceParams& p, hipStream_t stream) {
  if (p.K == 64) {
    if (p.maxr == 32) return launch_routed_reduce_t<OpT, OutT, 64, 32, 4, 256, 2, 4>(p, stream);
    return launch_routed_reduce_t<OpT, OutT, 64, 96, 4, 256, 2, 4>(p, stream);
  }
  if (p.maxr == 32) return launch_routed_reduce_t<OpT, OutT, 128, 32, 3, 128, 2, 4>(p, stream);
  return launch_routed_reduce_t<OpT, OutT, 128, 64, 3, 128, 2, 4>(p, stream);
}

template <typename OpT>
hipError_t launch_routed_reduce_op(const ReduceParams& p, hipStream_t stream) {
  if (p.out_dtype == kF32) return launch_routed_reduce_out<OpT, float>(p, stream);
  return launch_routed_reduce_out<OpT, OpT>(p, stream);
}

}  // namespace cvmm
