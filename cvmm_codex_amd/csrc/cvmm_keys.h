// The vectorised per-step weight cast, shared by the cast kernel and the
// launch that casts beside the selector scatter.
#pragma once

#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

template <typename OutT>
struct CastArgs {
  const float* keys;
  int64_t se, si;  // element strides of expert and d_in (d_out is unit-stride)
  int64_t d_in, d_out;
  OutT* kt;        // rows of d_in values, one per (expert, d_out column), or nullptr
  OutT* kn;        // rows of d_out values, one per (expert, d_in row), or nullptr
  int64_t t_se, t_sr;  // kt element strides of expert and row (d_in is unit-stride)
  int64_t n_se, n_sr;  // kn element strides of expert and row (d_out is unit-stride)
};

// The output strides of a cast layout (CVMM_CAST_*_INTERLEAVED bits):
// kt [E][d_out][d_in] or, interleaved, [d_out][E][d_in]; kn [E][d_in][d_out]
// or, interleaved, [d_in][E][d_out].  The interleaved copies are the
// [N][E*K] row-major B^T of a dense top-k GEMM with both operands
// k-contiguous.
template <typename OutT>
inline CastArgs<OutT> make_cast_args(const void* keys, int64_t se, int64_t si, int64_t n_experts, int64_t d_in,
                                     int64_t d_out, void* kt, void* kn, int32_t layout) {
  CastArgs<OutT> a{static_cast<const float*>(keys), se, si, d_in, d_out, static_cast<OutT*>(kt),
                   static_cast<OutT*>(kn), 0, 0, 0, 0};
  const bool ti = (layout & kCastTInterleaved) != 0, ni = (layout & kCastNInterleaved) != 0;
  a.t_se = ti ? d_in : d_out * d_in;
  a.t_sr = ti ? n_experts * d_in : d_in;
  a.n_se = ni ? d_out : d_in * d_out;
  a.n_sr = ni ? n_experts * d_out : d_out;
  return a;
}

// One 64 x 64 tile (expert e, d_in tile ti, d_out tile tj) of fp32 keys with
// unit column stride, 16-byte aligned rows, d_in and d_out multiples of 64:
// read as float4 rows (16 threads per 256-byte row), written to kn as 8-byte
// pieces of the same rows and, through a padded fp32 LDS tile, to kt as
// 16-byte pieces of its rows (8 consecutive d_in values per thread); a tile
// with kn alone goes 8 values per thread, one 16-byte store each (the
// 8-byte stores cost the SwitchHead value projection's cast ~9 us).  RNE,
// the rounding of the reference's in-register cast (cvmm.py:198-204).
// LDS of one cast block: the fp32 tile, 64 rows of up to 128 columns plus
// one padding column (the launches that cast provide it).
constexpr int kCastTileFloats = 64 * 129;

template <typename OutT>
__device__ __forceinline__ void cast_tile_vec(const CastArgs<OutT>& a, int64_t e, int64_t ti, int64_t tj,
                                              float* lds) {
  float(*tile)[65] = reinterpret_cast<float(*)[65]>(lds);
  const int64_t i0 = ti * 64, j0 = tj * 64;
  const int t = threadIdx.x;
  if (a.kt == nullptr) {
    // kn only: 8 consecutive values of a row per thread, one 16-byte store
    const int c8 = (t & 7) * 8;
    float4 v[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float* src = a.keys + e * a.se + (i0 + (t >> 3) + 32 * q) * a.si + j0 + c8;
      v[q][0] = *reinterpret_cast<const float4*>(src);
      v[q][1] = *reinterpret_cast<const float4*>(src + 4);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      union { uint4 u; OutT h[8]; } pk;
      const float f[8] = {v[q][0].x, v[q][0].y, v[q][0].z, v[q][0].w, v[q][1].x, v[q][1].y, v[q][1].z, v[q][1].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(f[k]);
      *reinterpret_cast<uint4*>(a.kn + e * a.n_se + (i0 + (t >> 3) + 32 * q) * a.n_sr + j0 + c8) = pk.u;
    }
    return;
  }
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    const float4 v = *reinterpret_cast<const float4*>(a.keys + e * a.se + (i0 + r) * a.si + j0 + c4);
    if (a.kt != nullptr) {  // the tile only feeds the transposed copy
      tile[r][c4] = v.x;
      tile[r][c4 + 1] = v.y;
      tile[r][c4 + 2] = v.z;
      tile[r][c4 + 3] = v.w;
    }
    if (a.kn != nullptr) {
      union { uint2 u; OutT h[4]; } pk;
      pk.h[0] = from_f32<OutT>(v.x);
      pk.h[1] = from_f32<OutT>(v.y);
      pk.h[2] = from_f32<OutT>(v.z);
      pk.h[3] = from_f32<OutT>(v.w);
      *reinterpret_cast<uint2*>(a.kn + e * a.n_se + (i0 + r) * a.n_sr + j0 + c4) = pk.u;
    }
  }
  if (a.kt == nullptr) return;
  lds_barrier();  // the tile is complete; the kn stores need not have landed
  const int i8 = (t & 7) * 8;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = (t >> 3) + 32 * q;
    union { uint4 u; OutT h[8]; } pk;
#pragma unroll
    for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(tile[i8 + k][j]);
    *reinterpret_cast<uint4*>(a.kt + e * a.t_se + (j0 + j) * a.t_sr + i0 + i8) = pk.u;
  }
}

// One 64 x 128 block (expert e, d_in rows i0.., d_out columns j0..) where
// d_out is a multiple of 128: each thread loads 8 consecutive d_out values
// of 4 rows (two float4 each, all 8 loads in flight), stores them to kn as
// one 16-byte piece per row, and through a padded fp32 LDS tile to kt as
// 16-byte pieces of 8 consecutive d_in values.  LDS banks: the transposed
// reads (lane l: d_in 8 * (l % 8) + k, d_out l / 8) hit 64 distinct banks
// with the 129-float row pitch; the row writes conflict two ways.
template <typename OutT>
__device__ __forceinline__ void cast_tile_vec128(const CastArgs<OutT>& a, int64_t e, int64_t ti, int64_t tj,
                                                 float* lds) {
  float(*tile)[129] = reinterpret_cast<float(*)[129]>(lds);
  const int64_t i0 = ti * 64, j0 = tj * 128;
  const int t = threadIdx.x;
  const int c8 = (t & 15) * 8;
  float4 v[4][2];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = q * 16 + (t >> 4);
    const float* src = a.keys + e * a.se + (i0 + r) * a.si + j0 + c8;
    v[q][0] = *reinterpret_cast<const float4*>(src);
    v[q][1] = *reinterpret_cast<const float4*>(src + 4);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = q * 16 + (t >> 4);
    const float f[8] = {v[q][0].x, v[q][0].y, v[q][0].z, v[q][0].w, v[q][1].x, v[q][1].y, v[q][1].z, v[q][1].w};
    if (a.kn != nullptr) {
      union { uint4 u; OutT h[8]; } pk;
#pragma unroll
      for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(f[k]);
      *reinterpret_cast<uint4*>(a.kn + e * a.n_se + (i0 + r) * a.n_sr + j0 + c8) = pk.u;
    }
    if (a.kt != nullptr) {  // the tile only feeds the transposed copy
#pragma unroll
      for (int k = 0; k < 8; ++k) tile[r][c8 + k] = f[k];
    }
  }
  if (a.kt == nullptr) return;
  lds_barrier();  // the tile is complete; the kn stores need not have landed
  const int i8 = (t & 7) * 8;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = q * 32 + (t >> 3);
    union { uint4 u; OutT h[8]; } pk;
#pragma unroll
    for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(tile[i8 + k][j]);
    *reinterpret_cast<uint4*>(a.kt + e * a.t_se + (j0 + j) * a.t_sr + i0 + i8) = pk.u;
  }
}

// Blocks of the vectorised cast: 64 x 128 where d_out % 128 == 0, else
// 64 x 64; block t = (expert, d_in block, d_out block), d_out fastest.
__host__ __device__ inline int64_t cast_block_cols(int64_t d_out) { return d_out % 128 == 0 ? 128 : 64; }
__host__ __device__ inline int64_t cast_blocks(int64_t n_experts, int64_t d_in, int64_t d_out) {
  return n_experts * (d_in / 64) * (d_out / cast_block_cols(d_out));
}
template <typename OutT>
__device__ __forceinline__ void cast_block(const CastArgs<OutT>& a, int64_t t, float* lds) {
  const int64_t ti = a.d_in / 64;
  if (a.d_out % 128 == 0) {
    const int64_t tj = a.d_out / 128;
    cast_tile_vec128(a, t / (ti * tj), (t / tj) % ti, t % tj, lds);
  } else {
    const int64_t tj = a.d_out / 64;
    cast_tile_vec(a, t / (ti * tj), (t / tj) % ti, t % tj, lds);
  }
}

}  // namespace cvmm
