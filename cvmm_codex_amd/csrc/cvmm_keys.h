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
  OutT* kt;        // [E][d_out][d_in] or nullptr
  OutT* kn;        // [E][d_in][d_out] or nullptr
};

// One 64 x 64 tile (expert e, d_in tile ti, d_out tile tj) of fp32 keys with
// unit column stride, 16-byte aligned rows, d_in and d_out multiples of 64:
// read as float4 rows (16 threads per 256-byte row), written to kn as 8-byte
// pieces of the same rows and, through a padded fp32 LDS tile, to kt as
// 16-byte pieces of its rows (8 consecutive d_in values per thread).  RNE,
// the rounding of the reference's in-register cast (cvmm.py:198-204).
template <typename OutT>
__device__ __forceinline__ void cast_tile_vec(const CastArgs<OutT>& a, int64_t e, int64_t ti, int64_t tj) {
  __shared__ float tile[64][65];
  const int64_t i0 = ti * 64, j0 = tj * 64;
  const int t = threadIdx.x;
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    const float4 v = *reinterpret_cast<const float4*>(a.keys + e * a.se + (i0 + r) * a.si + j0 + c4);
    tile[r][c4] = v.x;
    tile[r][c4 + 1] = v.y;
    tile[r][c4 + 2] = v.z;
    tile[r][c4 + 3] = v.w;
    if (a.kn != nullptr) {
      union { uint2 u; OutT h[4]; } pk;
      pk.h[0] = from_f32<OutT>(v.x);
      pk.h[1] = from_f32<OutT>(v.y);
      pk.h[2] = from_f32<OutT>(v.z);
      pk.h[3] = from_f32<OutT>(v.w);
      *reinterpret_cast<uint2*>(a.kn + (e * a.d_in + i0 + r) * a.d_out + j0 + c4) = pk.u;
    }
  }
  if (a.kt == nullptr) return;
  __syncthreads();
  const int i8 = (t & 7) * 8;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = (t >> 3) + 32 * q;
    union { uint4 u; OutT h[8]; } pk;
#pragma unroll
    for (int k = 0; k < 8; ++k) pk.h[k] = from_f32<OutT>(tile[i8 + k][j]);
    *reinterpret_cast<uint4*>(a.kt + (e * a.d_out + j0 + j) * a.d_in + i0 + i8) = pk.u;
  }
}

}  // namespace cvmm
