// Top-k sums as one dense GEMM over expert-slotted rows.
//
// A top-k sum of routed products -- the token gradient of a token-input
// selection, dX[t] = sum_j dY[t,j] @ W[e_tj]^T (cvmm.py:1204-1223), or the
// weighted forward combine, out[t] = sum_j w_tj x[t,j] @ W[e_tj]
// (cvmm.py:1541-1545) -- equals one plain GEMM when each token's operand rows
// are placed in expert slots:
//     A[t][e*K + k] = sum over the routes j of token t with expert e of
//                     rnd_op(s_tj * src[row(t,j)][k])         (zero elsewhere)
//     out[t] = A[t] @ Wk,   Wk[(e, k)][n] = W[e][k][n] of the product
// where Wk is an op-dtype weight copy, either as Wk^T [N][E*K] rows (the
// cast's expert-interleaved copy of the phase's own orientation: both GEMM
// operands k-contiguous, the faster form) or as [E*K][N] rows (the routed
// copy of the other orientation).  A has E/top_k times
// the product's useful flops, but no [R, N] route-ordered buffer is written
// and read back: at high fan-out (SwitchHead, 64 of 256 experts, a 2.1 GB
// buffer) the GEMM is the cheaper way.  The sum over a token's routes runs in
// the GEMM's fp32 accumulators and is rounded once (the route-buffer path
// rounds every route's product first, as the reference does); the GEMM is
// rocBLAS with atomics off, so results are deterministic.
#include <mutex>
#include <rocblas/rocblas.h>

#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

constexpr int kSlotWaves = 4;

// One wave per token row of A; only the token's own slots are written (the
// caller provides A zero elsewhere).  Lane j < top_k finds the expert of
// route (t, j) through the inverse permutation (its sorted position q =
// inv[r], valid when q < *rows_end and rp[q] == r); a per-wave LDS table maps
// each expert to its first route (bit 30 marks an expert the token picked
// twice: that slot gets the sum of both rows).  The wave then writes the
// slots, K/8 16-byte pieces per route: the rows' values, or zeros when
// `clear` (restoring an all-zero A after the GEMM).
constexpr int32_t kSlotNone = 0xffff;
template <typename OpT>
__global__ __launch_bounds__(64 * kSlotWaves) void slot_rows_kernel(const void* __restrict__ src, int32_t src_dtype,
                                                                   int64_t src_ld, int32_t src_per_route,
                                                                   const int32_t* __restrict__ sorted_sel,
                                                                   const int32_t* __restrict__ inv,
                                                                   const int64_t* __restrict__ rp,
                                                                   const int64_t* __restrict__ rows_end,
                                                                   int64_t n_tokens, int32_t top_k, int32_t n_experts,
                                                                   int64_t K, const void* __restrict__ w,
                                                                   int32_t w_dtype, int32_t w_round, int32_t clear,
                                                                   OpT* __restrict__ A) {
  constexpr int32_t kOp = DTypeOf<OpT>::value;
  extern __shared__ int32_t lds[];  // per wave: n_experts slots, 64 ids, 64 scales
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int32_t* slot = lds + wave * (n_experts + 128);
  int32_t* ids = slot + n_experts;
  float* scale = reinterpret_cast<float*>(ids + 64);
  const int64_t t = (int64_t)blockIdx.x * kSlotWaves + wave;
  const bool active = t < n_tokens;
  const int64_t valid_end = *rows_end;

  int32_t e = -1;
  float sc = 1.f;
  if (active && lane < top_k) {
    const int64_t r = t * top_k + lane;
    const int64_t q = inv[r];
    if (q >= 0 && q < valid_end && rp[q] == r) {
      const int32_t id = sorted_sel[q];
      if (id >= 0 && id < n_experts) e = id;
    }
    if (w != nullptr && !clear) sc = round_to(load_as_f32(w, w_dtype, r), w_round);
  }
  for (int32_t i = lane; i < n_experts; i += 64) slot[i] = kSlotNone;
  ids[lane] = e;
  scale[lane] = sc;
  __syncthreads();
  if (e >= 0) atomicMin(&slot[e], lane);
  __syncthreads();
  if (e >= 0 && slot[e] != lane) atomicOr(&slot[e], 1 << 30);
  __syncthreads();
  if (!active) return;

  const int32_t cpr = (int32_t)(K / 8);  // 16-byte pieces per slot
  OpT* out_row = A + t * (int64_t)n_experts * K;
  const bool vec_src = src_dtype == kOp && (src_ld % 8) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
  for (int32_t it = lane; it < top_k * cpr; it += 64) {
    const int32_t j0 = it / cpr, c = it - j0 * cpr;
    const int32_t ex = ids[j0];
    if (ex < 0) continue;
    const int32_t sl = slot[ex];
    if ((sl & 0xffff) != j0) continue;  // a later route of a repeated expert: summed by the first
    Chunk16 ch;
    if (clear) {
      ch.u = make_uint4(0, 0, 0, 0);
    } else {
      const bool dup = (sl >> 30) & 1;
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      for (int32_t j = j0; j < top_k; ++j) {
        if (j != j0 && ids[j] != ex) continue;
        const int64_t row = src_per_route ? t * top_k + j : t;
        const float sj = scale[j];
        const int64_t off = row * src_ld + (int64_t)c * 8;
        float v[8];
        if (vec_src) {
          Chunk16 in;
          in.u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(src) + off);
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = to_f32(reinterpret_cast<const OpT*>(&in)[i]);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = round_to(load_as_f32(src, src_dtype, off + i), kOp);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += w != nullptr ? round_to(sj * v[i], kOp) : v[i];
        if (!dup) break;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) reinterpret_cast<OpT*>(&ch)[i] = from_f32<OpT>(acc[i]);
    }
    *reinterpret_cast<uint4*>(out_row + (int64_t)ex * K + (int64_t)c * 8) = ch.u;
  }
}

hipError_t launch_slot_rows(const void* src, int32_t src_dtype, int64_t src_ld, bool src_per_route,
                            const int32_t* sorted_sel, const int32_t* inv, const int64_t* rp, const int64_t* rows_end,
                            int64_t n_tokens, int64_t top_k, int32_t n_experts, int64_t K, const void* w,
                            int32_t w_dtype, int32_t w_round, bool clear, int32_t op_dtype, void* A,
                            hipStream_t stream) {
  const size_t lds = (size_t)kSlotWaves * (n_experts + 128) * sizeof(int32_t);
  const unsigned grid = (unsigned)((n_tokens + kSlotWaves - 1) / kSlotWaves);
  if (lds > 65536) {  // above 3968 experts: ask for the larger dynamic LDS
    const void* f = op_dtype == kBF16 ? reinterpret_cast<const void*>(slot_rows_kernel<bf16_t>)
                                      : reinterpret_cast<const void*>(slot_rows_kernel<f16_t>);
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  if (op_dtype == kBF16)
    hipLaunchKernelGGL(slot_rows_kernel<bf16_t>, dim3(grid), dim3(64 * kSlotWaves), lds, stream, src, src_dtype, src_ld,
                       src_per_route ? 1 : 0, sorted_sel, inv, rp, rows_end, n_tokens, (int32_t)top_k, n_experts, K, w,
                       w_dtype, w_round, clear ? 1 : 0, (bf16_t*)A);
  else
    hipLaunchKernelGGL(slot_rows_kernel<f16_t>, dim3(grid), dim3(64 * kSlotWaves), lds, stream, src, src_dtype, src_ld,
                       src_per_route ? 1 : 0, sorted_sel, inv, rp, rows_end, n_tokens, (int32_t)top_k, n_experts, K, w,
                       w_dtype, w_round, clear ? 1 : 0, (f16_t*)A);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// rocBLAS: one handle per device (atomics off: deterministic results), its
// stream set per call under a lock.
// ---------------------------------------------------------------------------
namespace {
constexpr int kMaxBlasDevices = 64;
std::mutex g_blas_mu;
rocblas_handle g_blas[kMaxBlasDevices] = {};

rocblas_datatype blas_type(int32_t dt) {
  return dt == kF32 ? rocblas_datatype_f32_r : dt == kF16 ? rocblas_datatype_f16_r : rocblas_datatype_bf16_r;
}
}  // namespace

// out[t][n] (row stride out_ld, out_dtype) = sum_c A[t][c] * B[c][n], with A
// [T][C] row-major and B as [C][N] rows or (b_by_col) as B^T [N][C] rows, op
// dtype, fp32 accumulation.  Returns a HIP-style error: hipErrorUnknown with
// `status` set on a rocBLAS failure.
hipError_t dense_rows_gemm(const void* A, const void* B, bool b_by_col, int64_t T, int64_t C, int64_t N,
                           int32_t op_dtype, void* out, int32_t out_dtype, int64_t out_ld, hipStream_t stream,
                           int* status) {
  *status = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxBlasDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_blas_mu);
  if (g_blas[dev] == nullptr) {
    rocblas_handle h = nullptr;
    rocblas_status st = rocblas_create_handle(&h);
    if (st == rocblas_status_success) st = rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
    if (st != rocblas_status_success) {
      *status = (int)st;
      return hipErrorUnknown;
    }
    g_blas[dev] = h;
  }
  rocblas_handle h = g_blas[dev];
  rocblas_status st = rocblas_set_stream(h, stream);
  // column-major view: out^T [N x T] = B^T [N x C] * A^T [C x T]; the
  // row-major arrays are those column-major matrices, B^T transposed when B
  // comes as [N][C] rows (both operands k-contiguous: ~15 % faster at
  // SwitchHead size on MI355X)
  const float alpha = 1.f, beta = 0.f;
  if (st == rocblas_status_success)
    st = rocblas_gemm_ex(h, b_by_col ? rocblas_operation_transpose : rocblas_operation_none, rocblas_operation_none,
                         (rocblas_int)N, (rocblas_int)T, (rocblas_int)C, &alpha, B, blas_type(op_dtype),
                         (rocblas_int)(b_by_col ? C : N), A, blas_type(op_dtype),
                         (rocblas_int)C, &beta, out, blas_type(out_dtype), (rocblas_int)out_ld, out,
                         blas_type(out_dtype), (rocblas_int)out_ld, rocblas_datatype_f32_r, rocblas_gemm_algo_standard,
                         0, rocblas_gemm_flags_none);
  if (st != rocblas_status_success) {
    *status = (int)st;
    return hipErrorUnknown;
  }
  return hipSuccess;
}

}  // namespace cvmm
