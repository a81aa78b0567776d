// Shared device/host helpers for the CVMM HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace cvmm {

// dtype ids follow the reference's dtype_to_type_id (cvmm.py:36-44).
enum DType : int32_t { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

template <typename T> struct DTypeOf;
template <> struct DTypeOf<float> { static constexpr int32_t value = kF32; };
template <> struct DTypeOf<f16_t> { static constexpr int32_t value = kF16; };
template <> struct DTypeOf<bf16_t> { static constexpr int32_t value = kBF16; };

__host__ __device__ inline size_t dtype_size(int32_t dt) { return dt == kF32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// conversions (RNE; gfx950 lowers float->bf16 to v_cvt_pk_bf16_f32)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return (float)v; }
__device__ __forceinline__ float to_f32(f16_t v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return (bf16_t)v; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float v) { return (f16_t)v; }

// Round a float to the storage precision of dtype `dt` (value stays a float).
__device__ __forceinline__ float round_to(float v, int32_t dt) {
  if (dt == kBF16) return (float)(bf16_t)v;
  if (dt == kF16) return (float)(f16_t)v;
  return v;
}

// GELU, erf form: 0.5 x (1 + erf(x / sqrt 2)) (torch's F.gelu default).
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
// d gelu / dx = 0.5 (1 + erf(x / sqrt 2)) + x exp(-x^2 / 2) / sqrt(2 pi)
__device__ __forceinline__ float gelu_erf_grad(float x) {
  const float cdf = 0.5f * (1.f + erff(x * 0.70710678118654752f));
  const float pdf = expf(-0.5f * x * x) * 0.39894228040143268f;
  return cdf + x * pdf;
}

// Load element i of a tensor of runtime dtype `dt` as float.
__device__ __forceinline__ float load_as_f32(const void* p, int32_t dt, int64_t i) {
  if (dt == kBF16) return (float)((const bf16_t*)p)[i];
  if (dt == kF16) return (float)((const f16_t*)p)[i];
  return ((const float*)p)[i];
}

// Store float v (rounded RNE) into element i of a tensor of runtime dtype `dt`.
__device__ __forceinline__ void store_from_f32(void* p, int32_t dt, int64_t i, float v) {
  if (dt == kBF16) ((bf16_t*)p)[i] = (bf16_t)v;
  else if (dt == kF16) ((f16_t*)p)[i] = (f16_t)v;
  else ((float*)p)[i] = v;
}

// ---------------------------------------------------------------------------
// 16-byte chunk <-> 8 (or 4) lanes of op-type values
// ---------------------------------------------------------------------------
union Chunk16 {
  uint4 u;
  float f[4];
  bf16_t b[8];
  f16_t h[8];
  uint16_t s[8];
};

// Exact division of 0 <= n < 2^31 by a fixed 1 <= d < 2^31 as a multiply and
// shift (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994): l = ceil(log2 d), m = ceil(2^(31+l) / d),
// n / d = (n * m) >> (31 + l); n * m < 2^63.
struct FastDiv {
  uint64_t m;
  int32_t shift;
  __host__ __device__ __forceinline__ int64_t div(int64_t n) const { return (int64_t)(((uint64_t)n * m) >> shift); }
};

inline FastDiv make_fast_div(int64_t d) {
  int l = 0;
  while ((1ll << l) < d) ++l;
  const unsigned __int128 num = (unsigned __int128)1 << (31 + l);
  const uint64_t m = (uint64_t)((num + (unsigned __int128)(d - 1)) / (unsigned __int128)d);
  return FastDiv{m, 31 + l};
}

// The same constants computed on the device, for 1 <= d < 2^31: then
// 2^(31+l) < 2^63 and 64-bit arithmetic suffices.
__device__ __forceinline__ FastDiv make_fast_div_dev(int64_t d) {
  int l = 0;
  while ((1ll << l) < d) ++l;
  const uint64_t num = 1ull << (31 + l);
  return FastDiv{(num + (uint64_t)d - 1) / (uint64_t)d, 31 + l};
}

// Wave helpers (64-wide wavefronts).
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ int64_t wave_incl_scan(int64_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int64_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Workgroup barrier for a hand-over through LDS only: this wave's LDS
// operations complete (lgkmcnt(0)), then s_barrier.  __syncthreads() would
// also wait for the wave's outstanding global stores (its release fence),
// which a hand-over of LDS data does not need when no thread of the launch
// reads those stores.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Split-K hand-over of fp32 partial tiles between the workgroups of one
// output tile, which may run on different XCDs (each with its own L2): each
// writes its partials, counts itself in at the tile's counter, and the last to
// arrive adds every chunk's partials.  The partials are stored and loaded as
// agent-scope relaxed atomics and the counter is a relaxed agent-scope
// fetch_add.
//
// gfx942 / gfx950: agent-scope atomic stores and loads are issued with sc1
// (LLVM AMDGPUUsage, "Memory Model GFX942": stores write through the XCD's L2
// to the agent's coherent level, loads do not hit stale L2 lines), and a
// store leaves vmcnt only once that level has acknowledged it.  So a vmcnt(0)
// wait after the partial stores, before the workgroup barrier and the count,
// orders every partial before the count, and the last arriver's loads see
// them -- without the whole-L2 writeback and invalidate that release/acquire
// fences would cost.  Other targets use device-scope fences around the count
// (release before it, acquire after it), the memory model's own protocol.
#if defined(__gfx942__) || defined(__gfx950__)
#define CVMM_SPLITK_SC1_PROTOCOL 1
#else
#define CVMM_SPLITK_SC1_PROTOCOL 0
#endif

// after this thread's partial stores, before the workgroup barrier
__device__ __forceinline__ void splitk_published() {
#if CVMM_SPLITK_SC1_PROTOCOL
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0) (gfx9 encoding)
#else
  __threadfence();
#endif
}

// one thread per workgroup, after the barrier: count in; true for the last
// of n arrivals (the counter is reset for the next launch)
__device__ __forceinline__ bool splitk_arrive(int32_t* ctr, int32_t n) {
#if CVMM_SPLITK_SC1_PROTOCOL
  const int32_t prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#else
  const int32_t prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
#endif
  const bool last = prev == n - 1;
  if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// the last arriver, before reading the other chunks' partials (after the
// workgroup barrier that shares the arrival's outcome)
__device__ __forceinline__ void splitk_acquired() {
#if !CVMM_SPLITK_SC1_PROTOCOL
  __threadfence();
#endif
}

// Map a linear workgroup id so that consecutive logical ids are dispatched to
// the same XCD (the hardware places workgroup i on XCD i % 8).  Bijective for
// any grid size.
__device__ __forceinline__ int64_t xcd_remap(int64_t i, int64_t n) {
  constexpr int kXcd = 8;
  if (n < kXcd) return i;
  const int64_t xcd = i % kXcd, local = i / kXcd;
  const int64_t per = n / kXcd, rem = n % kXcd;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

}  // namespace cvmm
