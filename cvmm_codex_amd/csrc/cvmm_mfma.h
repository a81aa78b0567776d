// MFMA tile core for gfx950: a 256-thread workgroup (4 waves) computes a
// BM x BN fp32 tile; each wave owns a 64 x 64 sub-tile = 4 x 4 blocks of the
// 16x16 MFMA output.  Operands come from LDS in "k-contiguous" layout:
//   As[m][k], Bs[n][k]  (row stride LDS_ROW elements, +16 B padding)
// so every MFMA operand fragment is one 16-byte ds_read per lane.
//
// Lane layouts (CDNA3/CDNA4 ISA, 16x16 MFMA family):
//   A (16 x KSTEP): lane l holds row l%16, k-chunk l/16
//   B (KSTEP x 16): lane l holds col l%16, k-chunk l/16
//   D (16 x 16)   : lane l holds col l%16, rows 4*(l/16) + {0,1,2,3}
// bf16/f16: v_mfma_f32_16x16x32_{bf16,f16}: one chunk = 8 k, KSTEP = 32.
// fp32:     v_mfma_f32_16x16x4_f32 x4: a chunk of 4 k is consumed one k per
//           MFMA (the k order inside a 16-k step is permuted identically for
//           A and B, which leaves the dot product unchanged), KSTEP = 16.
#pragma once

#include "cvmm_common.h"

namespace cvmm {

template <typename OpT> struct MfmaOp;

template <> struct MfmaOp<bf16_t> {
  static constexpr int EPC = 8;     // elements per 16-byte chunk
  static constexpr int KSTEP = 32;  // k per MFMA step (4 lane groups x 8)
  __device__ __forceinline__ static void step(f32x4_t& c, const uint4& a, const uint4& b) {
    bf16x8_t va = __builtin_bit_cast(bf16x8_t, a);
    bf16x8_t vb = __builtin_bit_cast(bf16x8_t, b);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, vb, c, 0, 0, 0);
  }
};

template <> struct MfmaOp<f16_t> {
  static constexpr int EPC = 8;
  static constexpr int KSTEP = 32;
  __device__ __forceinline__ static void step(f32x4_t& c, const uint4& a, const uint4& b) {
    f16x8_t va = __builtin_bit_cast(f16x8_t, a);
    f16x8_t vb = __builtin_bit_cast(f16x8_t, b);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, vb, c, 0, 0, 0);
  }
};

template <> struct MfmaOp<float> {
  static constexpr int EPC = 4;
  static constexpr int KSTEP = 16;
  __device__ __forceinline__ static void step(f32x4_t& c, const uint4& a, const uint4& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
  }
};

// Tile geometry shared by the GEMM kernels.
template <typename OpT, int BM_, int BN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int EPC = MfmaOp<OpT>::EPC;
  static constexpr int KSTEP = MfmaOp<OpT>::KSTEP;
  static constexpr int BK = 128 / sizeof(OpT);        // 128-byte LDS rows: 64 bf16 / 32 fp32
  static constexpr int KCH = BK / EPC;                // 16-byte chunks per row (8)
  static constexpr int LDS_ROW = BK + EPC;            // +16 B padding per row
  static constexpr int WN = BN / 64, WM = BM / 64;    // wave grid
  static_assert(WM * WN == 4, "4 waves of 64x64");
  static constexpr int A_ELEMS = BM * LDS_ROW;
  static constexpr int B_ELEMS = BN * LDS_ROW;
  static constexpr int STAGE_ELEMS = A_ELEMS + B_ELEMS;
  static constexpr int STAGE_BYTES = STAGE_ELEMS * (int)sizeof(OpT);
  static constexpr int C_LD = BN + 4;                  // fp32 epilogue tile row
  static constexpr int C_BYTES = BM * C_LD * 4;
  static constexpr int SMEM = (2 * STAGE_BYTES > C_BYTES) ? 2 * STAGE_BYTES : C_BYTES;
};

// One LDS stage: 4x4 blocks of 16x16 per wave, BK/KSTEP MFMA steps.
template <typename OpT, typename Cfg>
__device__ __forceinline__ void mfma_stage(f32x4_t (&acc)[4][4], const OpT* __restrict__ As,
                                           const OpT* __restrict__ Bs, int wm, int wn, int lane) {
  const int r = lane & 15;
  const int q = lane >> 4;
#pragma unroll
  for (int st = 0; st < Cfg::BK / Cfg::KSTEP; ++st) {
    uint4 a[4], b[4];
    const int koff = st * Cfg::KSTEP + q * Cfg::EPC;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = *reinterpret_cast<const uint4*>(As + (wm * 64 + i * 16 + r) * Cfg::LDS_ROW + koff);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[j] = *reinterpret_cast<const uint4*>(Bs + (wn * 64 + j * 16 + r) * Cfg::LDS_ROW + koff);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) MfmaOp<OpT>::step(acc[i][j], a[i], b[j]);
  }
}

// Spill the accumulators of a wave into the fp32 LDS tile Cs[BM][C_LD].
template <typename Cfg>
__device__ __forceinline__ void acc_to_lds(const f32x4_t (&acc)[4][4], float* Cs, int wm, int wn, int lane) {
  const int col = lane & 15;
  const int rq = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        Cs[(wm * 64 + i * 16 + rq + v) * Cfg::C_LD + wn * 64 + j * 16 + col] = acc[i][j][v];
}

// 8 values (of any storage type) -> one 16-byte chunk of OpT.
template <typename OpT> __device__ __forceinline__ uint4 pack_chunk(const float (&v)[16 / sizeof(OpT)]);
template <> __device__ __forceinline__ uint4 pack_chunk<bf16_t>(const float (&v)[8]) {
  Chunk16 c;
#pragma unroll
  for (int j = 0; j < 8; ++j) c.b[j] = (bf16_t)v[j];
  return c.u;
}
template <> __device__ __forceinline__ uint4 pack_chunk<f16_t>(const float (&v)[8]) {
  Chunk16 c;
#pragma unroll
  for (int j = 0; j < 8; ++j) c.h[j] = (f16_t)v[j];
  return c.u;
}
template <> __device__ __forceinline__ uint4 pack_chunk<float>(const float (&v)[4]) {
  Chunk16 c;
#pragma unroll
  for (int j = 0; j < 4; ++j) c.f[j] = v[j];
  return c.u;
}

// Load EPC consecutive elements p[0..EPC) of storage type T and convert to
// OpT packed in a chunk.  `vec` = 16-byte (or 8-byte) aligned and in range.
template <typename OpT, typename T>
__device__ __forceinline__ uint4 load_chunk(const T* __restrict__ p, int64_t k, int64_t K, bool vec) {
  constexpr int EPC = 16 / sizeof(OpT);
  if (vec && k + EPC <= K) {
    if constexpr (sizeof(T) == sizeof(OpT) && DTypeOf<T>::value == DTypeOf<OpT>::value) {
      return *reinterpret_cast<const uint4*>(p + k);
    } else if constexpr (sizeof(T) == 4) {  // fp32 storage -> 16-bit op type (8 values)
      const float4 lo = *reinterpret_cast<const float4*>(p + k);
      const float4 hi = *reinterpret_cast<const float4*>(p + k + 4);
      float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      return pack_chunk<OpT>(v);
    } else if constexpr (sizeof(OpT) == 4) {  // 16-bit storage -> fp32 op type (4 values)
      Chunk16 c;
      const uint2 raw = *reinterpret_cast<const uint2*>(p + k);
      const T* e = reinterpret_cast<const T*>(&raw);
      float v[4] = {to_f32(e[0]), to_f32(e[1]), to_f32(e[2]), to_f32(e[3])};
      (void)c;
      return pack_chunk<OpT>(v);
    } else {  // 16-bit storage of the other 16-bit type
      const uint4 raw = *reinterpret_cast<const uint4*>(p + k);
      const T* e = reinterpret_cast<const T*>(&raw);
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = to_f32(e[j]);
      return pack_chunk<OpT>(v);
    }
  } else {
    float v[EPC];
#pragma unroll
    for (int j = 0; j < EPC; ++j) v[j] = (k + j < K) ? to_f32(p[k + j]) : 0.f;
    return pack_chunk<OpT>(v);
  }
}

}  // namespace cvmm
