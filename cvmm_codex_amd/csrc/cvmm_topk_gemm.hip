// Top-k sums as one dense GEMM whose expert-slotted operand is built on the fly.
//
// A top-k sum of routed products -- the token gradient of a token-input
// selection, dX[t] = sum_j dY[t,j] @ W[e_tj]^T (cvmm.py:1204-1223), or the
// weighted forward combine, out[t] = sum_j w_tj x[t,j] @ W[e_tj]
// (cvmm.py:1541-1545) -- is one plain GEMM over expert slots:
//     A[t][(e, k)] = rnd_op(s_te * src[row(t, e)][k])   (zero where t has no route on e)
//     out[t][n]    = sum_(e,k) A[t][(e, k)] * W_e[k][n]
// A has E/top_k times the product's useful flops, but no [R, N] route buffer
// is written and read back: at SwitchHead fan-out (64 of 256 experts, a 2.1
// GB buffer) the GEMM is the cheaper way.
//
// A is never stored.  A workgroup owns 256 tokens x 256 output columns and
// walks the experts in order, one 32-wide k slice at a time.  Each slice moves
// straight into LDS by buffer loads (16 bytes per lane, 4 lanes per 64-byte
// row piece, one request each): the rows of the slice's A half are the
// tokens' route rows for expert e -- their byte offsets come from a table of
// first routes per (expert, token) that a small launch builds beforehand --
// or zeros (an offset past the descriptor's range) when a token has no route
// there; the B half holds the weight rows of expert e for the tile's columns.
// A token that picks one expert several times gets its further routes as
// further passes over the experts (the table's next-route links), so each
// product term is one operand row, as in the reference's per-route products.
// The weighted forward's routing weights are applied to the route rows
// beforehand (a scaling launch writes them), so the GEMM has no per-element
// work besides the MFMAs.
//
// Pipeline.  The operand rows are gathered from L2 in 64-byte requests, so a
// CU needs many requests in flight: slices rotate through a ring of four
// 32 KB LDS buffers with three in flight while one is multiplied, and every
// wait is an exact vmcnt (each slice is the same nine DMA instructions per
// wave: four A pieces, four B pieces and the 256 table bytes of the slice
// three ahead, which its issue needs).  The descriptors stay fixed: the
// lane offsets come from the table (A) or are constant (B), and the slice's
// k and expert move a uniform soffset.  The fragments of slice s + 1 are read
// while the MFMAs of slice s run (two register sets), and the DMA of slice
// s + 4 is issued between those MFMAs.
//
// LDS rows are 64 bytes with 16-byte chunk c of row r at c ^ ((r >> 1) & 3),
// which keeps the fragment reads (lane l: row l % 16 of a 16-row block, one
// chunk) free of bank conflicts.  Waves: 2 x 2, each 128 x 128 of the tile
// (8 x 8 blocks of 16x16x32 MFMA, 256 accumulators in AGPRs); one workgroup
// per CU.  Operands are swapped (C^T = W x A^T) so that a lane ends with 4
// consecutive columns of one token row; two lane swaps make that 8, stored as
// one 16-byte write.  The sum over a token's routes runs in the fp32
// accumulators and is rounded once.  No atomics: repeated calls give the same
// bits.
#include "cvmm_gemm_panel.h"
#include "cvmm_topk_gemm.h"

namespace cvmm {

constexpr int kTkBM = 256, kTkBN = 256;  // GEMM tile: tokens x output columns
constexpr int kTkStages = 4;             // LDS slice ring
constexpr int kTkSlice = 32768;          // one slice: A 256 rows x 64 B, then B alike
constexpr int kTkB = 16384;              // offset of B within a slice
constexpr int kTkD = 9;                  // DMA instructions per wave per slice
constexpr int kTkTokens = 16;            // slot table launch: tokens per workgroup

// ---------------------------------------------------------------------------
// slot table
// ---------------------------------------------------------------------------
// A workgroup of 4 waves takes 16 tokens; wave w takes tokens w, w + 4, w + 8
// and w + 12 of them, lane j route j of each.  Lane j < top_k resolves the
// expert e_j of route r = t * top_k + j (sorted position q = inv[r], valid
// when q < *rows_end and rp[q] == r, with an expert id in [0, E)); the loads
// of all four tokens are issued together.  Over the token's routes:
//   slots[e][t] = 1 + the first j with e_j = e, else 0   (expert-major rows of
//                 t_pad = n_tokens rounded up to 256 bytes; 0 past n_tokens)
//   offs[e][t]  = the byte offset (t * top_k + j) * a_row_bytes of that
//                 route's operand row, or kTopkOob
//   nxt[r]      = 1 + the next j' > j with e_j' = e_j, else 0
//   mult[t]     = the most routes of t on one expert (0: none valid)
// The routes of a token that share an expert are found through a per-wave
// LDS word per expert: each lane ORs in its bit, then reads back the set of
// routes on its expert (first = lowest bit, next = lowest bit above its own,
// count = population).
__global__ __launch_bounds__(256) void topk_slot_table_kernel(
    const int32_t* __restrict__ sorted_sel, const int32_t* __restrict__ inv, const int64_t* __restrict__ rp,
    const int64_t* __restrict__ rows_end, int64_t n_tokens, int64_t t_pad, int32_t top_k, int32_t n_experts,
    int32_t e16, uint32_t a_row_bytes, uint32_t* __restrict__ offs, uint8_t* __restrict__ slots,
    uint8_t* __restrict__ nxt, uint8_t* __restrict__ mult) {
  constexpr int kPer = kTkTokens / 4;  // tokens per wave
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTopkMaxExperts][kTkTokens];
  __shared__ unsigned long long s_set[4][kTopkMaxExperts];  // per wave: routes of the token on expert e
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int64_t tok0 = (int64_t)blockIdx.x * kTkTokens;
  for (int i = tid * 16; i < e16 * kTkTokens; i += 256 * 16)
    *reinterpret_cast<uint4*>(&tile[0][0] + i) = make_uint4(0, 0, 0, 0);
  const int64_t valid_end = *rows_end;
  // ---- the experts of the wave's routes, loads issued together
  int64_t q[kPer];
  int32_t e[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = tok0 + wave + 4 * u;
    q[u] = (t < n_tokens && lane < top_k) ? (int64_t)inv[t * top_k + lane] : -1;
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = tok0 + wave + 4 * u;
    e[u] = -1;
    if (q[u] >= 0 && q[u] < valid_end && rp[q[u]] == t * top_k + lane) {
      const int32_t id = sorted_sel[q[u]];
      if (id >= 0 && id < n_experts) e[u] = id;
    }
  }
  __syncthreads();  // the tile is zero
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int tl = wave + 4 * u;
    const int64_t t = tok0 + tl;
    if (t >= n_tokens) break;  // wave-uniform; later tokens are further out
    const int32_t eu = e[u];
    unsigned long long* cell = &s_set[wave][eu >= 0 ? eu : 0];
    if (eu >= 0) *cell = 0ull;
    __builtin_amdgcn_wave_barrier();
    if (eu >= 0) atomicOr(cell, 1ull << lane);
    __builtin_amdgcn_wave_barrier();
    const unsigned long long set = eu >= 0 ? *cell : 0ull;
    __builtin_amdgcn_wave_barrier();
    const int cnt = __popcll(set);
    const unsigned long long above = lane == 63 ? 0ull : (set >> (lane + 1)) << (lane + 1);
    int m = cnt;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const int v = __shfl_xor(m, o, 64);
      m = v > m ? v : m;
    }
    if (eu >= 0 && __ffsll((long long)set) - 1 == lane) tile[eu][tl] = (uint8_t)(lane + 1);
    if (lane < top_k) nxt[t * top_k + lane] = (uint8_t)(above != 0ull ? __ffsll((long long)above) : 0);
    if (lane == 0) mult[t] = (uint8_t)m;
  }
  __syncthreads();
  // one thread per expert: the row piece of the 16 tokens in both tables
  for (int e = tid; e < e16; e += 256) {
    const uint4 b4 = *reinterpret_cast<const uint4*>(&tile[e][0]);
    *reinterpret_cast<uint4*>(slots + (int64_t)e * t_pad + tok0) = b4;
    const uint32_t bw[4] = {b4.x, b4.y, b4.z, b4.w};
    uint32_t o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t b = (bw[i >> 2] >> (8 * (i & 3))) & 0xffu;
      o[i] = b != 0 ? (uint32_t)(((tok0 + i) * top_k + (int64_t)b - 1) * a_row_bytes) : kTopkOob;
    }
    uint4* dst = reinterpret_cast<uint4*>(offs + (int64_t)e * t_pad + tok0);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
  }
}

// ---------------------------------------------------------------------------
// the weighted sum's operand rows, scaled by the rounded routing weight as the
// reference's weighted combine has it (cvmm.py:1545: rnd_out(w) applied to
// the route's product; here to its operand row):
//   xs[r][k] = rnd_op(rnd(w[r], w_round) * rnd_op(x[row][k])),
// row = r for route input, r / top_k for token input.  Every route is
// scaled: the GEMM reads only the rows of valid routes (the table's), so no
// route needs resolving here.  16-byte chunks, four loads in flight per
// thread; IDX32: chunk indices fit 32 bits (cheaper division).
// ---------------------------------------------------------------------------
template <typename OpT, typename IdxT>
__global__ __launch_bounds__(256) void scale_rows_kernel(const void* __restrict__ x, int32_t x_dtype, int64_t x_ld,
                                                         int32_t x_per_route, const void* __restrict__ w,
                                                         int32_t w_dtype, int32_t w_round, int64_t n_routes,
                                                         int64_t top_k, int64_t K, OpT* __restrict__ xs) {
  constexpr int32_t kOp = DTypeOf<OpT>::value;
  constexpr int kU = 4;
  const IdxT cpr = (IdxT)(K / 8);
  const IdxT total = (IdxT)n_routes * cpr;
  const bool vec = x_dtype == kOp && x_ld % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  for (IdxT base = (IdxT)blockIdx.x * (256 * kU); base < total; base += (IdxT)gridDim.x * (256 * kU)) {
    Chunk16 in[kU];
    float sc[kU];
    IdxT it[kU];
#pragma unroll
    for (int v = 0; v < kU; ++v) {
      it[v] = base + (IdxT)(v * 256) + (IdxT)threadIdx.x;
      if (it[v] >= total) continue;
      const IdxT r = it[v] / cpr, c = it[v] - r * cpr;
      const int64_t row = x_per_route ? (int64_t)r : (int64_t)r / top_k;
      const int64_t off = row * x_ld + (int64_t)c * 8;
      sc[v] = round_to(load_as_f32(w, w_dtype, (int64_t)r), w_round);
      if (vec) {
        in[v].u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + off);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          reinterpret_cast<OpT*>(&in[v])[i] = from_f32<OpT>(round_to(load_as_f32(x, x_dtype, off + i), kOp));
      }
    }
#pragma unroll
    for (int v = 0; v < kU; ++v) {
      if (it[v] >= total) continue;
      Chunk16 o;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        reinterpret_cast<OpT*>(&o)[i] = from_f32<OpT>(sc[v] * to_f32(reinterpret_cast<const OpT*>(&in[v])[i]));
      *reinterpret_cast<uint4*>(xs + (int64_t)it[v] * 8) = o.u;
    }
  }
}

// ---------------------------------------------------------------------------
// rows of any float storage / alignment -> contiguous op-dtype rows (the A
// source when the caller's rows cannot be copied 16 bytes at a time)
// ---------------------------------------------------------------------------
template <typename OpT>
__global__ __launch_bounds__(256) void copy_rows_op_kernel(const void* __restrict__ src, int32_t src_dtype,
                                                           int64_t src_ld, int64_t rows, int64_t K,
                                                           OpT* __restrict__ dst) {
  const int64_t total = rows * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / K, k = i - r * K;
    dst[i] = from_f32<OpT>(load_as_f32(src, src_dtype, r * src_ld + k));
  }
}

// ---------------------------------------------------------------------------
// the GEMM
// ---------------------------------------------------------------------------

// Word 3 of a raw buffer descriptor on gfx9 (no format conversion), and the
// descriptors' byte range: every offset the kernel issues is either below
// kTopkOob (the launcher checks it, soffset included) or at or past it, which
// reads zeros whether or not the hardware adds soffset before the range check.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr uint32_t kTkRange = kTopkOob;
// the descriptors' bases sit this far before the data, so that the lane
// offsets stay positive when instruction j's immediate 1024 j is taken off them
constexpr uint32_t kTkBaseBack = 4096;

template <int J>
using TkRow = std::integral_constant<int, J>;

// BYTES (4 or 16) per lane from the descriptor's memory at voff + soff + IMM
// into LDS at lds + IMM + BYTES x the lane index (the immediate moves both
// addresses; lds goes to M0): one instruction per wave, counted by vmcnt.
template <int BYTES, int IMM>
__device__ __forceinline__ void buf_dma(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
  static_assert(BYTES == 4 || BYTES == 16, "dword or dwordx4");
  static_assert(IMM >= 0 && IMM < 4096, "12-bit immediate");
  auto* l = (__attribute__((address_space(3))) void*)lds;
  if constexpr (BYTES == 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, voff, soff, IMM, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, voff, soff, IMM, 0);
}

// lgkmcnt(0) / lgkmcnt(8) tied to the table entries (read before the 8 LDS
// reads still allowed to be pending)
__device__ __forceinline__ void lgkm_wait_x4(lds_u32x4& x) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x)); }
__device__ __forceinline__ void lgkm_wait8_x4(lds_u32x4& x) { asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(x)); }

// The 8 fragments of a slice half: blocks i = 0..7 (rows base_row + 16 i + l
// % 16); `base` holds the lane's chunk address in block 0, blocks are 16 rows
// = 1024 bytes apart.
__device__ __forceinline__ void tk_read8(uint32_t base, lds_u32x4 (&f)[8]) {
  f[0] = lds_read128_at<0 * 1024>(base);
  f[1] = lds_read128_at<1 * 1024>(base);
  f[2] = lds_read128_at<2 * 1024>(base);
  f[3] = lds_read128_at<3 * 1024>(base);
  f[4] = lds_read128_at<4 * 1024>(base);
  f[5] = lds_read128_at<5 * 1024>(base);
  f[6] = lds_read128_at<6 * 1024>(base);
  f[7] = lds_read128_at<7 * 1024>(base);
}

__device__ __forceinline__ void tk_wait_frags(lds_u32x4 (&af)[8], lds_u32x4 (&bf)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[0]), "+v"(bf[0]));
#pragma unroll
  for (int i = 1; i < 8; ++i) asm volatile("" : "+v"(af[i]), "+v"(bf[i]));
}

template <typename OpT, typename OutT, bool KFULL>
__global__ __launch_bounds__(256, 1) void topk_gemm_kernel(const TopkGemmParams p) {
  __shared__ __attribute__((aligned(1024))) char stage[kTkStages * kTkSlice];
  // table entries of a slice, per wave: its 64 tokens' operand-row offsets
  __shared__ __attribute__((aligned(1024))) uint32_t sring[kTkStages][4][64];
  __shared__ int32_t s_layers[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n_ntiles = (p.N + kTkBN - 1) / kTkBN;
  const int64_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t t0 = (id / n_ntiles) * kTkBM, n0 = (id % n_ntiles) * kTkBN;

  // ---- layers: the most routes one token of the tile has on one expert
  {
    const int64_t t = t0 + tid;
    int m = t < p.n_tokens ? (int)p.mult[t] : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const int v = __shfl_xor(m, o, 64);
      m = v > m ? v : m;
    }
    if (lane == 0) s_layers[wave] = m;
  }
  __syncthreads();
  int32_t layers = s_layers[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) layers = s_layers[w] > layers ? s_layers[w] : layers;
  layers = __builtin_amdgcn_readfirstlane(layers);
  const int32_t KS = (int32_t)((p.K + 31) / 32);  // k slices per expert
  const int64_t S = (int64_t)layers * p.n_experts * KS;

  // ---- DMA roles.  Instruction j (0..3) of this wave fills LDS rows
  // (wave*4 + j)*16 + lane / 4 of the slice's A half (and of its B half), 16
  // bytes each: the row's physical chunk lane % 4, which holds its logical
  // chunk c = (lane % 4) ^ ((row >> 1) & 3) = (lane % 4) ^ ((lane / 8) % 4).
  // A's LDS row (wave*4 + j)*16 + q holds token t0 + wave*64 + 4 q + j (its
  // route row for the slice's expert, or zeros), so a lane's 4 tokens are
  // adjacent and their table entries are one 16-byte LDS read; B's LDS row r
  // holds output column n0 + r.  The moves are buffer loads into LDS with
  // fixed descriptors: the lane offsets are the table's row offsets (A) or
  // fixed (B), the slice's k and expert go in the uniform soffset, and an
  // offset at or past kTopkOob (a token with no route on the expert, a column
  // past N, a k chunk past K) reads zeros.
  const int rq = lane >> 2;
  const int c = (lane & 3) ^ ((lane >> 3) & 3);
  const uint32_t row_bytes = (uint32_t)(p.src_ld * 2);
  const int64_t t_lane = t0 + wave * 64 + rq * 4;  // token of instruction j: + j
  uint32_t a_add[4], b_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a_add[j] = (uint32_t)(c * 16) + kTkBaseBack - 1024u * j;
    const int64_t nl = wave * 64 + 16 * j + rq;  // weight row of column n0 + nl
    b_off[j] = n0 + nl < p.N ? (uint32_t)(nl * p.b_sn * 2 + c * 16) + kTkBaseBack - 1024u * j : kTopkOob;
  }
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const char*>(p.src) - kTkBaseBack), (short)0, (int)kTkRange, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const char*>(p.b) + n0 * p.b_sn * 2 - kTkBaseBack), (short)0, (int)kTkRange,
      kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc((void*)(p.offs + t0), (short)0,
                                                                      (int)kTkRange, kBufferRsrcWord3);
  const uint32_t t_voff = (uint32_t)(wave * 64 + lane) * 4;  // the wave's 64 tokens
  const uint32_t t_row = (uint32_t)(p.t_pad * 4);            // table bytes per expert
  const uint32_t b_e = (uint32_t)(p.b_se * 2);               // weight bytes per expert
  const uint32_t b_wrap = b_e - (uint32_t)(KS - 1) * 64;     // soffset step from an expert's last slice
  const uint32_t sring_rd = lds_addr(&sring[0][wave][0]) + rq * 16;  // + buf * 1024

  // The slice counters run ks fastest, then e, then l, and advance without
  // branches; sb = e * b_e + 64 ks is the weights' soffset.  Slices past the
  // last (S, S + 1, ...) are issued too: they read valid addresses (layer
  // `layers` and beyond walks the next-route links to their end, so their A
  // rows are zeros) into buffers that are never multiplied -- except slice
  // S, which pads an odd S to the loop's pairs and adds zeros -- so the loop
  // issues the same nine loads every slice and its waits are exact.
  struct Ctr {
    int32_t ks, e, l;
    uint32_t sb;
  };
  auto advance = [&](Ctr& q) {
    const int32_t ks1 = q.ks + 1;
    const bool wrap_k = ks1 == KS;
    q.ks = wrap_k ? 0 : ks1;
    q.sb += wrap_k ? b_wrap : 64u;
    const int32_t e1 = q.e + (wrap_k ? 1 : 0);
    const bool wrap_e = e1 == p.n_experts;
    q.e = wrap_e ? 0 : e1;
    q.sb = wrap_e ? 0u : q.sb;
    q.l += wrap_e ? 1 : 0;
  };
  struct TCtr {
    int32_t ks, e;
  };
  Ctr ci{0, 0, 0, 0u};  // the slice issued next
  TCtr cs{0, 0};        // the slice whose table entries load next
  // table entries of slice `cs` into ring entry `buf`
  auto load_slots = [&](int buf) {
    buf_dma<4, 0>(rt, t_voff, (uint32_t)cs.e * t_row, &sring[buf][wave][0]);
    const int32_t ks1 = cs.ks + 1;
    const bool wrap_k = ks1 == KS;
    cs.ks = wrap_k ? 0 : ks1;
    const int32_t e1 = cs.e + (wrap_k ? 1 : 0);
    cs.e = e1 == p.n_experts ? 0 : e1;
  };
  // the table entries of the lane's 4 tokens (the A offsets of layer 0)
  lds_u32x4 toff;
  auto read_slots = [&](int buf) { toff = lds_read128_at<0>(sring_rd + (uint32_t)buf * 1024); };
  auto walk_layers = [&]() {
    if (ci.l > 0) {
      // layer l: the token's l-th further route on e, from its first route
      // (byte table) along the next-route links
      const uint32_t first4 = *reinterpret_cast<const uint32_t*>(p.slots + (int64_t)ci.e * p.t_pad + t_lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int32_t r = (int32_t)((first4 >> (8 * j)) & 0xffu) - 1;
        for (int32_t i = 0; i < ci.l && r >= 0; ++i) r = (int32_t)p.nxt[(t_lane + j) * p.top_k + r] - 1;
        toff[j] = r >= 0 ? (uint32_t)(((t_lane + j) * p.top_k + r) * (int64_t)row_bytes) : kTopkOob;
      }
    }
  };
  // the slice being issued: its LDS buffer and soffsets
  char* i_dst = nullptr;
  uint32_t i_sa = 0, i_sb = 0;
  bool i_kok = true;
  auto issue_begin = [&](int buf) {
    i_dst = stage + buf * kTkSlice + wave * 4 * 1024;
    i_sa = (uint32_t)ci.ks * 64;
    i_sb = ci.sb;
    if constexpr (!KFULL) i_kok = ci.ks * 32 + c * 8 < p.K;
    advance(ci);
  };
  // row pieces J, J + 1 of the slice's A half (AB = 0) or B half (AB = 1):
  // the four A loads, then the four B loads, share one M0 each
  auto issue_pair = [&](auto abc, auto jc) {
    constexpr int AB = decltype(abc)::value, J = decltype(jc)::value;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t v = AB == 0 ? toff[J + h] + a_add[J + h] : b_off[J + h];
      if constexpr (!KFULL) v = i_kok ? v : kTopkOob;
      if (h == 0) buf_dma<16, J * 1024>(AB == 0 ? ra : rb, v, AB == 0 ? i_sa : i_sb, i_dst + AB * kTkB);
      else buf_dma<16, (J + 1) * 1024>(AB == 0 ? ra : rb, v, AB == 0 ? i_sa : i_sb, i_dst + AB * kTkB);
    }
  };
  // the 8 row loads of the slice, as 4 pairs
  auto issue_part = [&](int q) {
    if (q == 0) issue_pair(TkRow<0>{}, TkRow<0>{});
    else if (q == 1) issue_pair(TkRow<0>{}, TkRow<2>{});
    else if (q == 2) issue_pair(TkRow<1>{}, TkRow<0>{});
    else issue_pair(TkRow<1>{}, TkRow<2>{});
  };
  // slice `ci` into buffer buf, with the table entries of slice `cs` (three
  // later) into ring entry (buf + 3) % 4
  auto issue_slice = [&](int buf) {
    read_slots(buf);
    lgkm_wait_x4(toff);
    walk_layers();
    issue_begin(buf);
    issue_part(0);
    issue_part(1);
    issue_part(2);
    issue_part(3);
    load_slots((buf + 3) & 3);
  };

  // ---- fragments: lane reads row (l % 16) of each 16-row block, logical
  // chunk l / 16 at physical chunk ^ ((row >> 1) & 3) = ^ (((l % 16) >> 1) & 3)
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 15, fq = lane >> 4;
  const int pc = fq ^ ((fr >> 1) & 3);
  const uint32_t st0 = lds_addr(stage);
  const uint32_t a_f = st0 + (wm * 128 + fr) * 64 + (pc << 4);
  const uint32_t b_f = st0 + kTkB + (wn * 128 + fr) * 64 + (pc << 4);

  f32x4_t acc[8][8];  // acc[jb][i]: column block jb, row block i (C^T orientation)
#pragma unroll
  for (int jb = 0; jb < 8; ++jb)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[jb][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // the 8 MFMAs of column block jb
  auto mfma_group = [&](int jb, lds_u32x4 (&af)[8], lds_u32x4 (&bf)[8]) {
    const uint4 bq = as_uint4(bf[jb]);
#pragma unroll
    for (int i = 0; i < 8; ++i) MfmaOp<OpT>::step(acc[jb][i], bq, as_uint4(af[i]));
  };

  if (S > 0) {
    // prologue: table entries of slices 0..2, then slices 0..3 (each with the
    // table entries of the slice three later)
    load_slots(0);
    load_slots(1);
    load_slots(2);
    vm_wait<0>();
    issue_slice(0);
    issue_slice(1);
    issue_slice(2);
    vm_wait<0>();  // the table entries of slice 3
    issue_slice(3);
    vm_wait<3 * kTkD>();  // slice 0
    lds_barrier();
    lds_u32x4 a0[8], b0[8], a1[8], b1[8];
    tk_read8(a_f, a0);
    tk_read8(b_f, b0);
    tk_wait_frags(a0, b0);
    int buf = 0;  // buffer of slice s
    // One slice: multiply the fragments in (CA, CB) while the next slice's
    // are read into (NA, NB) and slice s + 4 is issued.  Slice s + 1 (and
    // the table entries of slice s + 4) have landed; every wave holds slice s
    // in registers, so its buffer takes slice s + 4.  The table entries are
    // read first, then slice s + 1's A fragments; the first 8 MFMAs cover
    // their latency, and the entries are in once at most those 8 reads are
    // pending.  The loop runs the slices in pairs (two register sets, no
    // copies); an odd S gets slice S, whose operand rows are zeros.
#define CVMM_TK_STEP(CA, CB, NA, NB)                      \
  {                                                      \
    const int nbuf = (buf + 1) & 3;                      \
    vm_wait<2 * kTkD>();                                 \
    lds_barrier();                                       \
    read_slots(buf);                                     \
    tk_read8(a_f + nbuf * kTkSlice, NA);                 \
    mfma_group(0, CA, CB);                               \
    __builtin_amdgcn_sched_barrier(0);                   \
    lgkm_wait8_x4(toff);                                 \
    tk_read8(b_f + nbuf * kTkSlice, NB);                 \
    walk_layers();                                       \
    issue_begin(buf);                                    \
    _Pragma("unroll") for (int jb = 1; jb < 8; ++jb) {   \
      mfma_group(jb, CA, CB);                            \
      if (jb <= 4) issue_part(jb - 1);                   \
      if (jb == 5) load_slots((buf + 3) & 3);            \
      __builtin_amdgcn_sched_barrier(0);                 \
    }                                                    \
    tk_wait_frags(NA, NB);                               \
    buf = nbuf;                                          \
  }
    for (int64_t s = 0; s < S; s += 2) {
      CVMM_TK_STEP(a0, b0, a1, b1)
      CVMM_TK_STEP(a1, b1, a0, b0)
    }
#undef CVMM_TK_STEP
    vm_wait<0>();
  }

  // ---- epilogue from registers: lane holds C[LDS row wm*128 + 16 i + fr]
  // [n = n0 + wn*128 + 16 jb + 4 fq + {0..3}], rounded once to the output type
  const int64_t nw = n0 + wn * 128;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // LDS row wm*128 + 16 i + fr holds token t0 + (wm*2 + i/4)*64 + 4 fr + i%4
    const int64_t tt = t0 + (wm * 2 + (i >> 2)) * 64 + fr * 4 + (i & 3);
    char* rowp = tt < p.n_tokens ? reinterpret_cast<char*>(p.out) + tt * p.out_ld * (int64_t)sizeof(OutT) : nullptr;
    if constexpr (sizeof(OutT) == 4) {
#pragma unroll
      for (int jb = 0; jb < 8; ++jb) {
        const int64_t nn = nw + jb * 16 + 4 * fq;
        if (rowp == nullptr || nn >= p.N) continue;
        if (p.out_vec) {
          *reinterpret_cast<float4*>(rowp + nn * 4) =
              make_float4(acc[jb][i][0], acc[jb][i][1], acc[jb][i][2], acc[jb][i][3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) reinterpret_cast<float*>(rowp)[nn + q] = acc[jb][i][q];
        }
      }
    } else {
      // blocks 2 pr, 2 pr + 1 -> columns 32 pr + 8 fq + [0, 8) per lane (two lane swaps)
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        uint32_t a[2], b[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          union { uint32_t u; OutT e[2]; } pa, pb;
          pa.e[0] = (OutT)acc[2 * pr][i][2 * h];
          pa.e[1] = (OutT)acc[2 * pr][i][2 * h + 1];
          pb.e[0] = (OutT)acc[2 * pr + 1][i][2 * h];
          pb.e[1] = (OutT)acc[2 * pr + 1][i][2 * h + 1];
          a[h] = pa.u;
          b[h] = pb.u;
        }
        const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
        const auto u0 = __builtin_amdgcn_permlane16_swap(s0[0], s0[1], false, false);
        const auto u1 = __builtin_amdgcn_permlane16_swap(s1[0], s1[1], false, false);
        const int64_t nn = nw + pr * 32 + 8 * fq;
        if (rowp == nullptr || nn >= p.N) continue;
        const uint4 v = make_uint4(u0[0], u1[0], u0[1], u1[1]);
        if (p.out_vec) {
          *reinterpret_cast<uint4*>(rowp + nn * 2) = v;
        } else {
          const uint16_t* hv = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
          for (int q = 0; q < 8; ++q) reinterpret_cast<uint16_t*>(rowp)[nn + q] = hv[q];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
int64_t topk_slot_rows(int64_t n_tokens) { return (n_tokens + kTkBM - 1) / kTkBM * kTkBM; }

// The buffer loads address the operand rows, the weights and the table with
// 32-bit offsets below kTopkOob: their largest soffset + lane offset +
// immediate, with the descriptors' bases kTkBaseBack before the data.
namespace {
int64_t tk_slack(int64_t K) { return kTkBaseBack + (K + 31) / 32 * 64 + 64; }
}  // namespace
bool topk_gemm_a_fits(int64_t rows, int64_t a_ld, int64_t K) {
  return rows * a_ld * 2 + tk_slack(K) < (int64_t)kTopkOob;
}
bool topk_gemm_b_fits(int32_t n_experts, int64_t b_se, int64_t b_sn, int64_t K) {
  return (int64_t)n_experts * b_se * 2 + kTkBN * b_sn * 2 + tk_slack(K) < (int64_t)kTopkOob;
}
bool topk_gemm_table_fits(int32_t n_experts, int64_t n_tokens) {
  return (int64_t)topk_e16(n_experts) * topk_slot_rows(n_tokens) * 4 < (int64_t)kTopkOob;
}

hipError_t launch_topk_slot_table(const int32_t* sorted_sel, const int32_t* inv, const int64_t* rp,
                                  const int64_t* rows_end, int64_t n_tokens, int64_t top_k, int32_t n_experts,
                                  int64_t a_ld, int64_t K, uint32_t* offs, uint8_t* slots, uint8_t* nxt, uint8_t* mult,
                                  hipStream_t stream) {
  if (n_tokens <= 0) return hipSuccess;
  if (top_k > 64 || n_experts > kTopkMaxExperts || !topk_gemm_a_fits(n_tokens * top_k, a_ld, K) ||
      !topk_gemm_table_fits(n_experts, n_tokens))
    return hipErrorInvalidValue;
  const int32_t e16 = topk_e16(n_experts);
  const int64_t t_pad = topk_slot_rows(n_tokens);
  const unsigned grid = (unsigned)(t_pad / kTkTokens);
  hipLaunchKernelGGL(topk_slot_table_kernel, dim3(grid), dim3(256), 0, stream, sorted_sel, inv, rp, rows_end,
                     n_tokens, t_pad, (int32_t)top_k, n_experts, e16, (uint32_t)(a_ld * 2), offs, slots, nxt, mult);
  return hipGetLastError();
}

hipError_t launch_scale_rows(const void* x, int32_t x_dtype, int64_t x_ld, bool x_per_route, const void* w,
                             int32_t w_dtype, int32_t w_round, int64_t n_routes, int64_t top_k, int64_t K,
                             int32_t op_dtype, void* xs, hipStream_t stream) {
  const int64_t total = n_routes * (K / 8);
  if (total <= 0) return hipSuccess;
  if (K % 8 != 0 || top_k <= 0) return hipErrorInvalidValue;
  int64_t blocks = (total + 1023) / 1024;
  if (blocks > 8192) blocks = 8192;
  const bool i32 = total + 8192 * 1024 < (1ll << 32);
#define CVMM_SCALE(OP, IDX)                                                                                 \
  hipLaunchKernelGGL((scale_rows_kernel<OP, IDX>), dim3((unsigned)blocks), dim3(256), 0, stream, x, x_dtype, \
                     x_ld, x_per_route ? 1 : 0, w, w_dtype, w_round, n_routes, top_k, K, (OP*)xs)
  if (op_dtype == kBF16) {
    if (i32) CVMM_SCALE(bf16_t, uint32_t);
    else CVMM_SCALE(bf16_t, int64_t);
  } else if (op_dtype == kF16) {
    if (i32) CVMM_SCALE(f16_t, uint32_t);
    else CVMM_SCALE(f16_t, int64_t);
  } else {
    return hipErrorInvalidValue;
  }
#undef CVMM_SCALE
  return hipGetLastError();
}

hipError_t launch_copy_rows_op(const void* src, int32_t src_dtype, int64_t src_ld, int64_t rows, int64_t K,
                               int32_t op_dtype, void* dst, hipStream_t stream) {
  const int64_t total = rows * K;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (op_dtype == kBF16)
    hipLaunchKernelGGL(copy_rows_op_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, src, src_dtype,
                       src_ld, rows, K, (bf16_t*)dst);
  else
    hipLaunchKernelGGL(copy_rows_op_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, src, src_dtype,
                       src_ld, rows, K, (f16_t*)dst);
  return hipGetLastError();
}

template <typename OpT, bool KFULL>
void launch_topk_gemm_k(const TopkGemmParams& p, int32_t out_dtype, int64_t grid, hipStream_t stream) {
  const dim3 g((unsigned)grid), b(256);
  if (out_dtype == kF32) hipLaunchKernelGGL((topk_gemm_kernel<OpT, float, KFULL>), g, b, 0, stream, p);
  else if (out_dtype == kBF16) hipLaunchKernelGGL((topk_gemm_kernel<OpT, bf16_t, KFULL>), g, b, 0, stream, p);
  else hipLaunchKernelGGL((topk_gemm_kernel<OpT, f16_t, KFULL>), g, b, 0, stream, p);
}

// K a multiple of the 32-wide slice: no partial k slice to mask
template <typename OpT>
void launch_topk_gemm_op(const TopkGemmParams& p, int32_t out_dtype, int64_t grid, hipStream_t stream) {
  if (p.K % 32 == 0) launch_topk_gemm_k<OpT, true>(p, out_dtype, grid, stream);
  else launch_topk_gemm_k<OpT, false>(p, out_dtype, grid, stream);
}

hipError_t launch_topk_gemm(const TopkGemmParams& p, int32_t op_dtype, int32_t out_dtype, hipStream_t stream) {
  const int64_t grid = ((p.n_tokens + kTkBM - 1) / kTkBM) * ((p.N + kTkBN - 1) / kTkBN);
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffll || p.K % 8 != 0 || p.N % 8 != 0 || p.top_k > 64 || p.n_experts > kTopkMaxExperts ||
      p.t_pad != topk_slot_rows(p.n_tokens) || !topk_gemm_a_fits(p.n_tokens * p.top_k, p.src_ld, p.K) ||
      !topk_gemm_b_fits(p.n_experts, p.b_se, p.b_sn, p.K) || !topk_gemm_table_fits(p.n_experts, p.n_tokens))
    return hipErrorInvalidValue;
  if (op_dtype == kBF16) launch_topk_gemm_op<bf16_t>(p, out_dtype, grid, stream);
  else if (op_dtype == kF16) launch_topk_gemm_op<f16_t>(p, out_dtype, grid, stream);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace cvmm
