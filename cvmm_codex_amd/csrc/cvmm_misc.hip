// Small bandwidth kernels around the routed GEMMs: zero fill (used instead of
// hipMemsetAsync so a captured graph holds only kernel nodes), the top-k row
// combine of a route-ordered buffer, fp32 -> storage casts and the ordered
// sum of per-tile routing-weight gradient partials.  Row kernels move 8
// columns (16 bytes of 16-bit data) per thread.
#include "cvmm_common.h"
#include "cvmm_internal.h"

namespace cvmm {

// head: bytes before the first 16-byte boundary; body: 16-byte stores; tail.
__global__ void fill_zero_kernel(uint8_t* __restrict__ head, int64_t n_head, uint4* __restrict__ body, int64_t n16,
                                 uint8_t* __restrict__ tail, int64_t n_tail) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) body[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < n_head) head[threadIdx.x] = 0;
  if (blockIdx.x == 0 && threadIdx.x < n_tail) tail[threadIdx.x] = 0;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  uint8_t* b = static_cast<uint8_t*>(p);
  int64_t n_head = (int64_t)((16 - (reinterpret_cast<uintptr_t>(b) & 15)) & 15);
  if ((size_t)n_head > bytes) n_head = (int64_t)bytes;
  const int64_t rest = (int64_t)bytes - n_head;
  const int64_t n16 = rest / 16;
  const int64_t n_tail = rest % 16;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, b, n_head,
                     reinterpret_cast<uint4*>(b + n_head), n16, b + n_head + n16 * 16, n_tail);
  return hipGetLastError();
}

// The int32 copy of a selection (int32 or int64 ids, int64 read as its low
// 32 bits): 4 ids per thread, vector loads and stores when aligned.
template <typename IdxT>
__global__ __launch_bounds__(256) void copy_ids_kernel(const IdxT* __restrict__ sel, int64_t n,
                                                       int32_t* __restrict__ out, int32_t vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t n4 = vec ? n / 4 : 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    int4 o;
    if constexpr (sizeof(IdxT) == 8) {
      const longlong2 a = reinterpret_cast<const longlong2*>(sel)[2 * i];
      const longlong2 b = reinterpret_cast<const longlong2*>(sel)[2 * i + 1];
      o = make_int4((int32_t)a.x, (int32_t)a.y, (int32_t)b.x, (int32_t)b.y);
    } else {
      o = reinterpret_cast<const int4*>(sel)[i];
    }
    reinterpret_cast<int4*>(out)[i] = o;
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = (int32_t)sel[i];
}

hipError_t launch_copy_ids(const void* sel, bool sel_is_int64, int64_t n, int32_t* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const size_t align = sel_is_int64 ? 16 : 16;
  const int32_t vec = (reinterpret_cast<uintptr_t>(sel) % align) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  int64_t blocks = (n / 4 + 255) / 256 + 1;
  if (blocks > 1024) blocks = 1024;
  if (sel_is_int64)
    hipLaunchKernelGGL(copy_ids_kernel<int64_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(sel), n, out, vec);
  else
    hipLaunchKernelGGL(copy_ids_kernel<int32_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(sel), n, out, vec);
  return hipGetLastError();
}

// 8 consecutive columns of any storage type as floats (vector when aligned).
__device__ __forceinline__ void load8_any(const void* p, int32_t dt, int64_t off, bool vec, int64_t nvalid,
                                          float (&v)[8]) {
  if (vec && nvalid >= 8) {
    if (dt == kF32) {
      const float4 a = *reinterpret_cast<const float4*>((const float*)p + off);
      const float4 b = *reinterpret_cast<const float4*>((const float*)p + off + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      Chunk16 c;
      c.u = *reinterpret_cast<const uint4*>((const uint16_t*)p + off);
      if (dt == kBF16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)c.b[j];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)c.h[j];
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = j < nvalid ? load_as_f32(p, dt, off + j) : 0.f;
  }
}

__device__ __forceinline__ void store8_any(void* p, int32_t dt, int64_t off, bool vec, int64_t nvalid,
                                           const float (&v)[8]) {
  if (vec && nvalid >= 8) {
    if (dt == kF32) {
      *reinterpret_cast<float4*>((float*)p + off) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>((float*)p + off + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      Chunk16 c;
      if (dt == kBF16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c.b[j] = (bf16_t)v[j];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) c.h[j] = (f16_t)v[j];
      }
      *reinterpret_cast<uint4*>((uint16_t*)p + off) = c.u;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < nvalid) store_from_f32(p, dt, off + j, v[j]);
  }
}

__host__ __device__ inline bool vec_ok(const void* p, int32_t dt, int64_t ld) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (ld * (int64_t)dtype_size(dt)) % 16 == 0;
}

// out[t][n] = rnd(rnd(sum_j w_j * buf[row(t*k + j)][n], mid), out), j in route
// order (the top-k sum of cvmm.py:1223 and the weighted combine of
// cvmm.py:1545).  row(r) = r, or, with a route-ordered buffer (row q holds
// route rp[q]), row(r) = inv[r] checked against rp: a route no row holds adds
// nothing.
__global__ __launch_bounds__(256) void combine_rows_kernel(
    const void* __restrict__ buf, int32_t buf_dtype, int64_t buf_ld, const int32_t* __restrict__ inv,
    const int64_t* __restrict__ rp, int64_t n_routes, const int64_t* __restrict__ rows_end, const void* __restrict__ w,
    int32_t w_dtype, int32_t w_round, int64_t k, int64_t n, int32_t mid_dtype, void* __restrict__ out,
    int32_t out_dtype, int64_t out_ld, bool in_vec, bool out_vec) {
  // the token's routes are resolved once per workgroup (64 at a time) into
  // LDS: row of the route in `buf` (-1: none) and its rounded weight
  __shared__ int64_t s_row[64];
  __shared__ float s_w[64];
  const int64_t t = blockIdx.x;
  const int64_t c = ((int64_t)blockIdx.y * blockDim.x + threadIdx.x) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t j0 = 0; j0 < k; j0 += 64) {
    const int64_t kj = k - j0 < 64 ? k - j0 : 64;
    if (threadIdx.x < kj) {
      const int64_t r = t * k + j0 + threadIdx.x;
      int64_t row = r;
      if (inv != nullptr) {
        row = inv[r];
        const int64_t lim = rows_end != nullptr && *rows_end < n_routes ? *rows_end : n_routes;
        if (row < 0 || row >= lim || rp[row] != r) row = -1;
      }
      s_row[threadIdx.x] = row;
      s_w[threadIdx.x] = w != nullptr ? round_to(load_as_f32(w, w_dtype, r), w_round) : 1.f;
    }
    __syncthreads();
    if (c < n) {
      int64_t j = 0;
      // four rows in flight, summed in route order
      for (; j + 4 <= kj; j += 4) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t row = s_row[j + u];
          if (row >= 0) load8_any(buf, buf_dtype, row * buf_ld + c, in_vec, n - c, v[u]);
          else {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[u][q] = 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float wv = s_w[j + u];
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[q] += wv * v[u][q];
        }
      }
      for (; j < kj; ++j) {
        const int64_t row = s_row[j];
        if (row < 0) continue;
        float v[8];
        load8_any(buf, buf_dtype, row * buf_ld + c, in_vec, n - c, v);
        const float wv = s_w[j];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] += wv * v[q];
      }
    }
    __syncthreads();
  }
  if (c >= n) return;
  if (mid_dtype >= 0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = round_to(acc[q], mid_dtype);
  }
  store8_any(out, out_dtype, t * out_ld + c, out_vec, n - c, acc);
}

// The same sum with one wave per token, for 16-bit row buffers with aligned
// rows, n % 8 == 0 and k <= 64: lane j resolves route t*k + j, and every lane
// then holds 16 bytes of each of NP 512-column pieces of 16 / NP rows in
// flight before summing them in route order -- no LDS, no barriers, four
// tokens per workgroup.  NP = 4 reads whole 4 KB rows of 2048 columns per
// batch (one DRAM page run per row instead of two 1 KB halves at different
// times).
template <typename BufT, int NP>
__global__ __launch_bounds__(256) void combine_rows_wave_kernel(
    const BufT* __restrict__ buf, int64_t buf_ld, const int32_t* __restrict__ inv, const int64_t* __restrict__ rp,
    int64_t n_routes, const int64_t* __restrict__ rows_end, const void* __restrict__ w, int32_t w_dtype,
    int32_t w_round, int64_t k, int64_t n, int32_t mid_dtype, void* __restrict__ out, int32_t out_dtype,
    int64_t out_ld, int64_t n_tokens, int32_t accumulate) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tokens) return;
  int64_t my_row = -1;
  float my_w = 0.f;
  if (lane < k) {
    const int64_t r = t * k + lane;
    int64_t row = r;
    if (inv != nullptr) {
      row = inv[r];
      const int64_t lim = rows_end != nullptr && *rows_end < n_routes ? *rows_end : n_routes;
      if (row < 0 || row >= lim || rp[row] != r) row = -1;
    }
    my_row = row;
    my_w = w != nullptr ? round_to(load_as_f32(w, w_dtype, r), w_round) : 1.f;
  }
  constexpr int RB = 16 / NP;  // rows per batch
  // the column loop is uniform over the wave (the row shuffles need every
  // lane active); columns past n only mask the loads and stores
  for (int64_t cb = 0; cb < n; cb += 512 * NP) {
    bool in[NP];
    float acc[NP][8];
#pragma unroll
    for (int pc = 0; pc < NP; ++pc) {
      in[pc] = cb + pc * 512 + lane * 8 < n;
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[pc][q] = 0.f;
      if (accumulate && in[pc]) {  // out: the fp32 running sum
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(out) + t * out_ld + cb +
                                                            pc * 512 + lane * 8);
        const float4 a = src[0], b = src[1];
        acc[pc][0] = a.x; acc[pc][1] = a.y; acc[pc][2] = a.z; acc[pc][3] = a.w;
        acc[pc][4] = b.x; acc[pc][5] = b.y; acc[pc][6] = b.z; acc[pc][7] = b.w;
      }
    }
    for (int64_t j0 = 0; j0 < k; j0 += RB) {
      uint4 v[RB][NP];
      float wv[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int src = (int)((j0 + u) & 63);
        const int64_t row = __shfl(my_row, src, 64);
        wv[u] = __shfl(my_w, src, 64);
        const bool ok = j0 + u < k && row >= 0;
        const BufT* rowp = buf + (ok ? row : 0) * buf_ld + cb + lane * 8;
#pragma unroll
        for (int pc = 0; pc < NP; ++pc)
          v[u][pc] = ok && in[pc] ? *reinterpret_cast<const uint4*>(rowp + pc * 512) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        if (j0 + u >= k) break;
#pragma unroll
        for (int pc = 0; pc < NP; ++pc) {
          Chunk16 a;
          a.u = v[u][pc];
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[pc][q] += wv[u] * to_f32(reinterpret_cast<const BufT*>(&a)[q]);
        }
      }
    }
#pragma unroll
    for (int pc = 0; pc < NP; ++pc) {
      if (mid_dtype >= 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[pc][q] = round_to(acc[pc][q], mid_dtype);
      }
      const int64_t c = cb + pc * 512 + lane * 8;
      if (in[pc]) store8_any(out, out_dtype, t * out_ld + c, true, n - c, acc[pc]);
    }
  }
}

// inv[rp[q]] = q for every q with rp[q] in [0, R): the sorted position of
// each route.
__global__ void invert_rows_kernel(const int64_t* __restrict__ rp, int64_t n_routes, int32_t* __restrict__ inv) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n_routes) return;
  const int64_t r = rp[q];
  if (r >= 0 && r < n_routes) inv[r] = (int32_t)q;
}

hipError_t launch_invert_rows(const int64_t* rp, int64_t n_routes, int32_t* inv, hipStream_t stream) {
  if (n_routes <= 0) return hipSuccess;
  if (n_routes > 0x7fffffffll) return hipErrorInvalidValue;
  const int64_t blocks = (n_routes + 255) / 256;
  hipLaunchKernelGGL(invert_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, rp, n_routes, inv);
  return hipGetLastError();
}

static void rows_grid(int64_t rows, int64_t n, dim3* grid, dim3* block) {
  int64_t chunks = (n + 7) / 8;
  int threads = (int)((chunks + 63) / 64 * 64);
  if (threads > 256) threads = 256;
  *block = dim3(threads);
  *grid = dim3((unsigned)rows, (unsigned)((chunks + threads - 1) / threads));
}

hipError_t launch_combine_rows(const void* buf, int32_t buf_dtype, int64_t buf_ld, const int32_t* inv,
                               const int64_t* rp, const int64_t* rows_end, const void* w, int32_t w_dtype,
                               int32_t w_round, int64_t n_tokens,
                               int64_t k, int64_t n, int32_t mid_dtype, void* out, int32_t out_dtype, int64_t out_ld,
                               hipStream_t stream, bool accumulate) {
  if (n_tokens <= 0 || n <= 0) return hipSuccess;
  if (n_tokens > 0x7fffffffll || (n + 2047) / 2048 > 65535) return hipErrorInvalidValue;
  if ((inv == nullptr) != (rp == nullptr)) return hipErrorInvalidValue;
  const bool wave_ok = (buf_dtype == kBF16 || buf_dtype == kF16) && k <= 64 && n % 8 == 0 &&
                       vec_ok(buf, buf_dtype, buf_ld) && vec_ok(out, out_dtype, out_ld);
  // a running sum: fp32 rows, added to unrounded, by the wave kernel only
  if (accumulate && !(wave_ok && out_dtype == kF32 && mid_dtype < 0)) return hipErrorInvalidValue;
  if (wave_ok) {
    const dim3 grid((unsigned)((n_tokens + 3) / 4));
    // whole 2048-column rows per batch where rows are that wide; 1024 columns
    // (two pieces) otherwise
    const bool wide = n >= 2048;
#define CVMM_COMBINE(T, NP)                                                                                      \
  hipLaunchKernelGGL((combine_rows_wave_kernel<T, NP>), grid, dim3(256), 0, stream, (const T*)buf, buf_ld, inv, \
                     rp, n_tokens * k, rows_end, w, w_dtype, w_round, k, n, mid_dtype, out, out_dtype, out_ld, n_tokens, \
                     accumulate ? 1 : 0)
    if (buf_dtype == kBF16) {
      if (wide) CVMM_COMBINE(bf16_t, 4);
      else CVMM_COMBINE(bf16_t, 2);
    } else {
      if (wide) CVMM_COMBINE(f16_t, 4);
      else CVMM_COMBINE(f16_t, 2);
    }
#undef CVMM_COMBINE
    return hipGetLastError();
  }
  dim3 grid, block;
  rows_grid(n_tokens, n, &grid, &block);
  hipLaunchKernelGGL(combine_rows_kernel, grid, block, 0, stream, buf, buf_dtype, buf_ld, inv, rp, n_tokens * k,
                     rows_end, w, w_dtype, w_round, k, n, mid_dtype, out, out_dtype, out_ld, vec_ok(buf, buf_dtype, buf_ld),
                     vec_ok(out, out_dtype, out_ld));
  return hipGetLastError();
}

__global__ void cast_rows_kernel(const float* __restrict__ acc, int64_t acc_ld, int64_t n, int32_t mid_dtype,
                                 void* __restrict__ out, int32_t out_dtype, int64_t out_ld, bool in_vec,
                                 bool out_vec) {
  const int64_t t = blockIdx.x;
  const int64_t c = ((int64_t)blockIdx.y * blockDim.x + threadIdx.x) * 8;
  if (c >= n) return;
  float v[8];
  load8_any(acc, kF32, t * acc_ld + c, in_vec, n - c, v);
  if (mid_dtype >= 0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = round_to(v[q], mid_dtype);
  }
  store8_any(out, out_dtype, t * out_ld + c, out_vec, n - c, v);
}

hipError_t launch_cast_rows(const float* acc, int64_t acc_ld, int64_t rows, int64_t n, int32_t mid_dtype,
                            void* out, int32_t out_dtype, int64_t out_ld, hipStream_t stream) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  if (rows > 0x7fffffffll || (n + 2047) / 2048 > 65535) return hipErrorInvalidValue;
  dim3 grid, block;
  rows_grid(rows, n, &grid, &block);
  hipLaunchKernelGGL(cast_rows_kernel, grid, block, 0, stream, acc, acc_ld, n, mid_dtype, out, out_dtype, out_ld,
                     vec_ok(acc, kF32, acc_ld), vec_ok(out, out_dtype, out_ld));
  return hipGetLastError();
}

__global__ void sum_partials_kernel(const float* __restrict__ part, int64_t rows, int32_t ntiles,
                                    void* __restrict__ out, int32_t out_dtype) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = 0.f;
  for (int32_t t = 0; t < ntiles; ++t) s += part[r * ntiles + t];
  store_from_f32(out, out_dtype, r, s);
}

hipError_t launch_sum_partials(const float* part, int64_t rows, int32_t ntiles, void* out, int32_t out_dtype,
                               hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int64_t blocks = (rows + 255) / 256;
  hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, part, rows, ntiles, out,
                     out_dtype);
  return hipGetLastError();
}

}  // namespace cvmm

namespace cvmm {

// The GELU passes walk a [rows][cols] block as a flat range of 8-element
// pieces (cols % 8 == 0; row strides may differ from cols), 256 threads per
// workgroup, so that narrow rows still make full workgroups.
// (rows are split with 32-bit arithmetic; flat blocks need none)
__device__ __forceinline__ void gelu_piece(int64_t i, int64_t cols8, bool flat, int64_t* r, int64_t* c) {
  if (flat) {
    *r = 0;
    *c = i * 8;
  } else {
    const uint32_t q = (uint32_t)i / (uint32_t)cols8;
    *r = q;
    *c = ((int64_t)((uint32_t)i - q * (uint32_t)cols8)) * 8;
  }
}

// y = rnd(gelu(h)) per element (F.gelu, erf form).
__global__ __launch_bounds__(256) void gelu_rows_kernel(const void* __restrict__ h, int32_t h_dtype, int64_t h_ld,
                                                        int64_t rows, int64_t cols, void* __restrict__ y,
                                                        int32_t y_dtype, int64_t y_ld, bool in_vec, bool out_vec,
                                                        bool flat) {
  const int64_t cols8 = (cols + 7) / 8;
  const int64_t n = rows * cols8;
  const int64_t lim = flat ? rows * cols : cols;  // valid elements from the piece's row start
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r, c;
    gelu_piece(i, cols8, flat, &r, &c);
    float v[8];
    load8_any(h, h_dtype, r * h_ld + c, in_vec, lim - c, v);
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = gelu_erf(v[q]);
    store8_any(y, y_dtype, r * y_ld + c, out_vec, lim - c, v);
  }
}

// dh = rnd(dy * gelu'(h)) per element (the gelu backward formula).
__global__ __launch_bounds__(256) void gelu_backward_kernel(
    const void* __restrict__ dy, int32_t dy_dtype, int64_t dy_ld, const void* __restrict__ h, int32_t h_dtype,
    int64_t h_ld, int64_t rows, int64_t cols, void* __restrict__ dh, int32_t dh_dtype, int64_t dh_ld, bool dy_vec,
    bool h_vec, bool out_vec, bool flat) {
  const int64_t cols8 = (cols + 7) / 8;
  const int64_t n = rows * cols8;
  const int64_t lim = flat ? rows * cols : cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r, c;
    gelu_piece(i, cols8, flat, &r, &c);
    float g[8], x[8];
    load8_any(dy, dy_dtype, r * dy_ld + c, dy_vec, lim - c, g);
    load8_any(h, h_dtype, r * h_ld + c, h_vec, lim - c, x);
#pragma unroll
    for (int q = 0; q < 8; ++q) g[q] = g[q] * gelu_erf_grad(x[q]);
    store8_any(dh, dh_dtype, r * dh_ld + c, out_vec, lim - c, g);
  }
}

// The common case of the derivative pass: dY, h and dH of one 16-bit type,
// back-to-back rows, 16-byte aligned: one 8-element piece per thread per
// step, no runtime type dispatch.  The Gaussian density uses the hardware
// exp2 (v_exp_f32) on x^2 * (-log2(e) / 2), a few ulp from expf; erff is the
// library's, as in the forward.
template <typename T>
__global__ __launch_bounds__(256) void gelu_backward_vec_kernel(const uint4* __restrict__ dy,
                                                                const uint4* __restrict__ h, uint4* __restrict__ dh,
                                                                int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    Chunk16 g, x, o;
    g.u = dy[i];
    x.u = h[i];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float xv = to_f32(reinterpret_cast<const T*>(&x)[q]);
      const float gv = to_f32(reinterpret_cast<const T*>(&g)[q]);
      const float cdf = 0.5f * (1.f + erff(xv * 0.70710678118654752f));
      const float pdf = __builtin_amdgcn_exp2f(xv * xv * -0.72134752044448170f) * 0.39894228040143268f;
      reinterpret_cast<T*>(&o)[q] = (T)(gv * (cdf + xv * pdf));
    }
    dh[i] = o.u;
  }
}

// A block whose rows are back to back (every row stride = cols, cols % 8 == 0)
// is walked as one flat row.
static bool gelu_flat(int64_t cols, int64_t a, int64_t b, int64_t c) {
  return cols % 8 == 0 && a == cols && b == cols && c == cols;
}

static unsigned gelu_grid(int64_t rows, int64_t cols) {
  const int64_t pieces = rows * ((cols + 7) / 8);
  int64_t blocks = (pieces + 255) / 256;
  if (blocks > 65536) blocks = 65536;  // grid-stride beyond
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

hipError_t launch_gelu_rows(const void* h, int32_t h_dtype, int64_t h_ld, int64_t rows, int64_t cols, void* y,
                            int32_t y_dtype, int64_t y_ld, hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (rows * ((cols + 7) / 8) > 0xffffffffll) return hipErrorInvalidValue;  // 32-bit row split
  hipLaunchKernelGGL(gelu_rows_kernel, dim3(gelu_grid(rows, cols)), dim3(256), 0, stream, h, h_dtype, h_ld, rows,
                     cols, y, y_dtype, y_ld, vec_ok(h, h_dtype, h_ld), vec_ok(y, y_dtype, y_ld),
                     gelu_flat(cols, h_ld, y_ld, cols));
  return hipGetLastError();
}

hipError_t launch_gelu_backward(const void* dy, int32_t dy_dtype, int64_t dy_ld, const void* h, int32_t h_dtype,
                                int64_t h_ld, int64_t rows, int64_t cols, void* dh, int32_t dh_dtype, int64_t dh_ld,
                                hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (rows * ((cols + 7) / 8) > 0xffffffffll) return hipErrorInvalidValue;  // 32-bit row split
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  if (dy_dtype == h_dtype && dh_dtype == h_dtype && (h_dtype == kBF16 || h_dtype == kF16) &&
      gelu_flat(cols, dy_ld, h_ld, dh_ld) && a16(dy) && a16(h) && a16(dh)) {
    const int64_t n8 = rows * cols / 8;
    const dim3 grid(gelu_grid(rows, cols));
    if (h_dtype == kBF16)
      hipLaunchKernelGGL(gelu_backward_vec_kernel<bf16_t>, grid, dim3(256), 0, stream, (const uint4*)dy,
                         (const uint4*)h, (uint4*)dh, n8);
    else
      hipLaunchKernelGGL(gelu_backward_vec_kernel<f16_t>, grid, dim3(256), 0, stream, (const uint4*)dy,
                         (const uint4*)h, (uint4*)dh, n8);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(gelu_backward_kernel, dim3(gelu_grid(rows, cols)), dim3(256), 0, stream, dy, dy_dtype, dy_ld, h,
                     h_dtype, h_ld, rows, cols, dh, dh_dtype, dh_ld, vec_ok(dy, dy_dtype, dy_ld),
                     vec_ok(h, h_dtype, h_ld), vec_ok(dh, dh_dtype, dh_ld), gelu_flat(cols, dy_ld, h_ld, dh_ld));
  return hipGetLastError();
}

}  // namespace cvmm
