// Internal launch interfaces between the C-ABI layer and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "cvmm_common.h"
#include "cvmm_topk_gemm.h"

namespace cvmm {

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// routed GEMM:  for every expert-sorted route p,
//   acc[p][n] = sum_k rnd_op(A[arow(p)][k]) * rnd_op(B_e[k][n]),   e = expert of p
// with arow(p) = a_idx[p] / a_div.  B_e[k][n] = b[e*b_se + k*b_sk + n*b_sn] with
// either b_sn == 1 (kBNContig) or b_sk == 1 (kBKContig).
// ---------------------------------------------------------------------------
enum Epilogue : int32_t {
  kEpiStore = 0,   // out[orow][n] = v            (out dtype out_dtype)
  kEpiAtomic = 1,  // ((float*)out)[orow][n] += v (fp32 accumulation buffer)
};

struct GemmParams {
  // A operand (gathered rows, unit column stride)
  const void* a;
  int32_t a_dtype;
  int64_t a_ld, a_rows;
  int32_t a_vec;
  const int64_t* a_idx;
  int64_t a_div;
  // B operand (per-expert matrix)
  const void* b;
  int32_t b_dtype;
  int64_t b_se, b_sk, b_sn;
  int32_t b_vec;
  int64_t K, N;
  // route grouping
  const int64_t* offsets;  // inclusive per-expert offsets, int64[E]
  int32_t n_experts;
  int64_t n_routes;
  int64_t grid_tiles;      // m-tile slots launched (>= actual number of tiles)
  // epilogue:  v = rnd(acc, val_dtype);  if w: v = rnd(v * rnd(w[w_idx[p]], w_round), prod_dtype)
  int32_t epi;
  void* out;
  int32_t out_dtype;
  int64_t out_ld, out_rows;
  const int64_t* o_idx;    // orow(p) = o_idx[p] / o_div, or p when NULL
  int64_t o_div;
  int32_t val_dtype;
  const void* w;           // optional per-route scale
  int32_t w_dtype;
  const int64_t* w_idx;
  int32_t w_round;
  int32_t prod_dtype;      // -1: no rounding of the product
  // optional routing-weight gradient: dg[w_idx[p] * dg_ntiles + n_tile] =
  //   sum_{n in tile} rnd(acc, dg_val_dtype) * dg_x[dg_x_idx[p]][n]
  float* dg;
  int32_t dg_ntiles;
  const void* dg_x;
  int32_t dg_x_dtype;
  int64_t dg_x_ld, dg_x_rows;
  const int64_t* dg_x_idx;
  int32_t dg_val_dtype;
  // 0 = forward, 1 = grad-input: selects separately named kernel
  // instantiations so that profiles tell the two products apart
  int32_t role;
  // n-tiles per workgroup of the small-K kernel (0: built-in choice)
  int32_t panel_tpw;
  // m-tile order: 0 = expert-major (an expert's tiles are consecutive),
  // 1 = token-major (tile j of every expert, then tile j + 1, ...), -1 = the
  // launcher's choice; token major needs n_experts <= kTokenMajorMaxExperts
  int32_t token_major;
  // activation of the forward's stored values (ring kernel only): 1 = GELU
  // (erf form): out = gelu(h), and h (the product in the output type) to aux
  int32_t act;
  void* aux;
  // m-tile height of the long-K kernel with 128-column tiles: 0 = the
  // launcher's choice, 1 = 128 rows, 2 = 160 rows
  int32_t ring_tile;
  // zero the output rows (and aux rows) of the routes no tile covers: those
  // whose expert id is outside [0, E), sorted past offsets[E - 1]; done by the
  // workgroups past the last m-tile (direct per-route stores only)
  int32_t zero_unrouted;
  // small-K kernel only (routed_gemm_is_panel): also write every tile row's
  // activation row scaled by its routing weight, xs_out[arow][k] =
  // rnd_op(rnd_op(xs_w[widx]) * a[arow][k]) ([a_rows][K], op dtype); NULL: no
  int32_t xs_w_dtype;
  void* xs_out;
  const void* xs_w;
};
constexpr int32_t kTokenMajorMaxExperts = 256;

// op_dtype selects the MFMA type; returns hipErrorInvalidValue on unsupported combos.
hipError_t launch_routed_gemm(const GemmParams& p, int32_t op_dtype, hipStream_t stream);
int routed_gemm_bm(int64_t N);

// ---------------------------------------------------------------------------
// per-expert weight gradient:
//   dW[e][m][n] = sum_{p in e} rnd_op(X[x_idx[p]][m]) * G(p)[n]
//   G(p)[n] = rnd_op(g[g_idx[p] / g_div][n])           (unweighted)
//           = rnd_op(rnd_op(g[..][n]) * rnd_op(w[w_idx[p]]))  (weighted)
// deterministic split over routes (chunks of `split` routes, fixed-order sum).
// ---------------------------------------------------------------------------
struct WgradParams {
  const void* x;
  int32_t x_dtype;
  int64_t x_ld, x_rows;
  int32_t x_vec;
  const int64_t* x_idx;
  const void* g;
  int32_t g_dtype;
  int64_t g_ld, g_rows;
  int32_t g_vec;
  const int64_t* g_idx;
  int64_t g_div;
  FastDiv g_fdiv;          // g_div as multiply-shift (route indices < 2^31)
  const void* w;
  int32_t w_dtype;
  const int64_t* w_idx;
  int64_t M, N;
  const int64_t* offsets;
  int32_t n_experts;
  int64_t n_routes;
  int64_t split;
  int64_t grid_chunks;
  void* dw;
  int32_t dw_dtype;
  int64_t dw_se, dw_sm, dw_sn;
  float* partial;          // [max_slots][M][N] fp32
  int64_t max_slots;
  int32_t* counters;       // [E][tiles_m*tiles_n], zero on entry
  int32_t order;           // workgroup order, one of kWgOrder*
  int32_t tile_choice;     // 16-bit fast path tile: kWgTile*
};

// Small fp32 problems (cvmm_small.hip): 16 x 64 routed-product tiles and
// 64 x 64 weight-gradient blocks, plain FMAs.
bool small_gemm_eligible(const GemmParams& p, int32_t op);
hipError_t launch_routed_small(const GemmParams& p, hipStream_t stream);
bool small_wgrad_eligible(const WgradParams& p, int32_t op);
hipError_t launch_wgrad_small(const WgradParams& p, hipStream_t stream);

// Weight-gradient workgroup orders.  The hardware places workgroup i on XCD
// i % 8; each XCD has its own L2.
//   chunk-major:  the tiles of one route chunk adjacent, contiguous ranges of
//                 chunks per XCD (experts in order);
//   tile-major:   one dW tile of every chunk adjacent (an XCD shares the
//                 column slice of its tiles across experts);
//   chunk-xcd:    chunk c on XCD c % 8 with all its tiles adjacent there: the
//                 tiles running together on one XCD read the same routes'
//                 rows, and every XCD gets every eighth chunk (hot and cold
//                 experts spread evenly).
constexpr int32_t kWgOrderChunk = 0, kWgOrderTile = 1, kWgOrderChunkXcd = 2;

hipError_t launch_wgrad(const WgradParams& p, int32_t op_dtype, hipStream_t stream);

// dW tile shape [BM x BN] for a dW of M x N: 64 wide on a narrow side.
__host__ __device__ inline void wgrad_tile(int64_t M, int64_t N, int* bm, int* bn) {
  if (N <= 64 && M > 64) { *bm = 256; *bn = 64; }
  else if (M <= 64 && N > 64) { *bm = 64; *bn = 256; }
  else { *bm = 128; *bn = 128; }
}
// The 16-bit fast path may take a coarser tile where the base tile is
// 128 x 128: 256 x 128, 128 x 256 or 256 x 256 (fewer bytes gathered per
// flop; four waves of up to 128 x 128, or 256 x 256 as eight waves of 128 x
// 64; one workgroup per CU).
constexpr int32_t kWgTileBase = 0, kWgTile256x128 = 1, kWgTile128x256 = 2, kWgTile256x256 = 3;
constexpr int32_t kWgTile256x256W8 = 4;  // 256 x 256 of eight waves
__host__ __device__ inline void wgrad_fast_tile(int64_t M, int64_t N, int32_t choice, int* bm, int* bn) {
  wgrad_tile(M, N, bm, bn);
  if (*bm != 128 || *bn != 128) return;
  if (choice == kWgTile256x128) *bm = 256;
  else if (choice == kWgTile128x256) *bn = 256;
  else if (choice == kWgTile256x256 || choice == kWgTile256x256W8) { *bm = 256; *bn = 256; }
}
// tiles_mn counts base tiles (the finest: one counter each, enough for any
// coarser tile); partials are sized for the largest rounding of M x N.
void wgrad_geometry(int64_t M, int64_t N, int64_t n_routes, int32_t n_experts, int32_t op_dtype,
                    int64_t* split, int64_t* grid_chunks, int64_t* max_slots, int64_t* tiles_mn);
int64_t wgrad_partial_elems(int64_t M, int64_t N);
// built-in tile choice (no knob): 256 x 256 of eight waves where M, N >= 256
// and the grid holds >= 4 tiles per CU, else the base tile
int32_t wgrad_auto_tile(int64_t M, int64_t N, int64_t grid_chunks);

// ---------------------------------------------------------------------------
// selector preparation
// ---------------------------------------------------------------------------
size_t sort_workspace_bytes(int64_t n_routes, int32_t n_experts);
int64_t sort_chunk_size(int64_t n_routes, int32_t n_experts);
// routes per chunk of the sort (0: the built-in choice)
void set_sort_chunk(int64_t routes);
// whether the selector scatter and the weight cast fit one launch
bool sort_cast_fusable(int32_t n_experts);
// bytes of a chunks x (E + 1) int32 count matrix, rounded up to 256
size_t sort_counts_bytes(int64_t n_chunks, int32_t n_experts);
// Layout bits of the cast's outputs (the C ABI's CVMM_CAST_T_INTERLEAVED /
// CVMM_CAST_N_INTERLEAVED): kt as [d_out][E][d_in], kn as [d_in][E][d_out].
constexpr int32_t kCastTInterleaved = 1;
constexpr int32_t kCastNInterleaved = 2;

// A weight cast to run in the sort's scatter launch (vectorised cast only).
struct CastRequest {
  const void* keys;
  int64_t se, si;
  int32_t n_experts;
  int64_t d_in, d_out;
  int32_t out_dtype;
  void* kt;
  void* kn;
  int32_t layout;
};
// The vectorised cast applies: fp32 keys with unit column stride, 16-byte
// aligned rows, d_in and d_out multiples of 64, 16-bit output.
inline bool cast_vec_ok(const void* keys, int32_t keys_dtype, int64_t se, int64_t si, int64_t sj, int64_t d_in,
                        int64_t d_out, int32_t out_dtype, const void* kt, const void* kn) {
  return keys_dtype == kF32 && sj == 1 && d_in % 64 == 0 && d_out % 64 == 0 && si % 4 == 0 && se % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(keys) & 15) == 0 && (reinterpret_cast<uintptr_t>(kt) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(kn) & 15) == 0 && (out_dtype == kBF16 || out_dtype == kF16);
}
hipError_t launch_sort_routes(const void* sel, bool sel_is_int64, int64_t n_routes, int32_t n_experts,
                              int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                              int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* ws,
                              hipStream_t stream, const CastRequest* cast = nullptr, bool counts_ready = false);
// The int32 copy of the ids plus the sort's count matrix for n_experts
// (written into the sort workspace `ws`, as the histogram launch would).
hipError_t launch_copy_ids_count(const void* sel, bool sel_is_int64, int64_t n_routes, int32_t n_experts,
                                 int32_t* out, void* ws, hipStream_t stream);
hipError_t launch_expert_offsets(const int32_t* sorted_sel, int64_t n_routes, int32_t n_experts,
                                 int64_t* offsets, hipStream_t stream);

// keys (any float storage / strides) -> op dtype copies kt [E][d_out][d_in]
// and/or kn [E][d_in][d_out] (either may be null; `layout` bits interleave
// the experts between the rows instead)
hipError_t launch_cast_keys(const void* keys, int32_t keys_dtype, int64_t se, int64_t si, int64_t sj,
                            int32_t n_experts, int64_t d_in, int64_t d_out, int32_t out_dtype, void* kt,
                            void* kn, int32_t layout, hipStream_t stream);

// ---------------------------------------------------------------------------
// small kernels
// ---------------------------------------------------------------------------
// The stable scatter of cvmm_sort_routes over int64 ids whose per-chunk
// histogram (counts[chunk][E + 1], chunks of `chunk` routes) is already built.
// A large histogram is turned in place into per-chunk bucket prefixes, with
// the bucket totals at sort_counts_bytes(chunks, E) bytes past `counts`: the
// workspace holds both.
hipError_t launch_sort_scatter(const int64_t* sel, int64_t n_routes, int32_t n_experts, int64_t chunk, int64_t top_k,
                               int32_t* counts, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid_out, hipStream_t stream);

// ---------------------------------------------------------------------------
// router: softmax -> top-k -> renormalise -> stable sort by expert
// ---------------------------------------------------------------------------
constexpr int32_t kRouteMaxExperts = 1024;  // logits of a token held in registers (16 per lane)
constexpr int64_t kRouteMaxK = 64;          // lane j holds the token's j-th choice
// Tokens per router workgroup (= per sort chunk): whole tokens, at least the
// sort's chunk size in routes.
int64_t route_chunk_tokens(int64_t n_tokens, int32_t n_experts, int64_t top_k);
size_t route_workspace_bytes(int64_t n_tokens, int32_t n_experts, int64_t top_k);
hipError_t launch_route_topk(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                             int32_t n_experts, int64_t top_k, int32_t renormalize, float* weights, int64_t* sel,
                             int32_t* sorted_sel, int64_t* perm, int64_t* token_index, int64_t* offsets,
                             int32_t* route_pos, void* workspace, hipStream_t stream);
hipError_t launch_route_topk_backward(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                                      int32_t n_experts, int64_t top_k, int32_t renormalize, const int64_t* sel,
                                      const float* grad_weights, void* grad_logits, int64_t grad_ld,
                                      hipStream_t stream);

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);
// out[i] = (int32) sel[i] (int64 ids: their low 32 bits)
hipError_t launch_copy_ids(const void* sel, bool sel_is_int64, int64_t n, int32_t* out, hipStream_t stream);
// GELU (erf form) over rows: y = rnd(gelu(h)); its backward
// dh = rnd(dy * gelu'(h)) (the formula of torch's gelu backward).
hipError_t launch_gelu_rows(const void* h, int32_t h_dtype, int64_t h_ld, int64_t rows, int64_t cols, void* y,
                            int32_t y_dtype, int64_t y_ld, hipStream_t stream);
hipError_t launch_gelu_backward(const void* dy, int32_t dy_dtype, int64_t dy_ld, const void* h, int32_t h_dtype,
                                int64_t h_ld, int64_t rows, int64_t cols, void* dh, int32_t dh_dtype, int64_t dh_ld,
                                hipStream_t stream);
// out[t][n] = rnd(rnd(sum_j rnd(w[t*k+j], w_round) * buf[row(t*k+j)][n], mid_dtype), out_dtype)
// row(r) = inv[r] (checked against rp; rows at or past *rows_end, a device
// pointer to the number of routes with a valid expert id -- the rows the
// GEMMs wrote -- count as absent), or r when inv == NULL.
hipError_t launch_combine_rows(const void* buf, int32_t buf_dtype, int64_t buf_ld, const int32_t* inv,
                               const int64_t* rp, const int64_t* rows_end, const void* w, int32_t w_dtype,
                               int32_t w_round, int64_t n_tokens,
                               int64_t k, int64_t n, int32_t mid_dtype, void* out, int32_t out_dtype, int64_t out_ld,
                               hipStream_t stream, bool accumulate = false);
hipError_t launch_invert_rows(const int64_t* rp, int64_t n_routes, int32_t* inv, hipStream_t stream);
// out[t][n] = rnd(rnd(acc[t][n], mid_dtype), out_dtype)
hipError_t launch_cast_rows(const float* acc, int64_t acc_ld, int64_t rows, int64_t n, int32_t mid_dtype,
                            void* out, int32_t out_dtype, int64_t out_ld, hipStream_t stream);
// out[r] = rnd(sum_t part[r*ntiles + t], out_dtype)
hipError_t launch_sum_partials(const float* part, int64_t rows, int32_t ntiles, void* out, int32_t out_dtype,
                               hipStream_t stream);

}  // namespace cvmm
