// Launch interface of the dense top-k GEMM (cvmm_topk_gemm.hip): a top-k sum
// over routed products taken as one GEMM over expert slots whose operand rows
// are gathered on the fly (no slotted buffer, no route buffer).
#pragma once

#include "cvmm_common.h"

namespace cvmm {

// Experts a token row of the slot table covers (LDS of the table launch).
constexpr int32_t kTopkMaxExperts = 1024;
// Operand-row offset that reads zeros (2^31; every real offset is below it).
constexpr uint32_t kTopkOob = 0x80000000u;

// Slot-table rows: the expert count rounded up to 16; row length: the token
// count rounded up to the GEMM's 256-token tile.
inline int32_t topk_e16(int32_t n_experts) { return (n_experts + 15) / 16 * 16; }
int64_t topk_slot_rows(int64_t n_tokens);

struct TopkGemmParams {
  // operand rows (op dtype, 16-byte aligned rows, unit column stride): row
  // t * top_k + j of route j of token t
  const void* src;
  int64_t src_ld;
  // slot table (launch_topk_slot_table)
  const uint32_t* offs;   // [e16][t_pad]: byte offset in src of the token's first route row on e, or kTopkOob
  const uint8_t* slots;   // [e16][t_pad]: 1 + the token's first route on e, or 0
  int64_t t_pad;          // topk_slot_rows(n_tokens)
  const uint8_t* nxt;     // [n_tokens * top_k]: 1 + the token's next route on the same expert, or 0
  const uint8_t* mult;    // [n_tokens]: the most routes of the token on one expert
  // B: B_e[k][n] = b[e * b_se + n * b_sn + k] (op dtype, 16-byte aligned rows)
  const void* b;
  int64_t b_se, b_sn;
  int64_t n_tokens, top_k, K, N;
  int32_t n_experts, e16;
  // out[t][n] = rnd(sum), row stride out_ld; out_vec: 16-byte aligned rows
  void* out;
  int64_t out_ld;
  int32_t out_vec;
};

// Slot table of a selection (see TopkGemmParams; slots holds e16 x
// topk_slot_rows(n_tokens) bytes, offs as many 32-bit offsets, those of
// operand rows a_ld elements apart): the expert of route r is
// sorted_sel[inv[r]] when inv[r] < *rows_end and rp[inv[r]] == r, with an id in
// [0, E).  top_k <= 64, n_experts <= kTopkMaxExperts.
hipError_t launch_topk_slot_table(const int32_t* sorted_sel, const int32_t* inv, const int64_t* rp,
                                  const int64_t* rows_end, int64_t n_tokens, int64_t top_k, int32_t n_experts,
                                  int64_t a_ld, int64_t K, uint32_t* offs, uint8_t* slots, uint8_t* nxt, uint8_t* mult,
                                  hipStream_t stream);
// The operand rows of a weighted sum: xs[r][k] = rnd_op(rnd(w[r], w_round) *
// rnd_op(x[row][k])), row = r (x_per_route) or r / top_k, xs contiguous
// [n_routes][K]; 16-bit op dtype, K % 8 == 0.
hipError_t launch_scale_rows(const void* x, int32_t x_dtype, int64_t x_ld, bool x_per_route, const void* w,
                             int32_t w_dtype, int32_t w_round, int64_t n_routes, int64_t top_k, int64_t K,
                             int32_t op_dtype, void* xs, hipStream_t stream);
// dst[r][k] = rnd_op(src[r * src_ld + k]), contiguous rows of K values
hipError_t launch_copy_rows_op(const void* src, int32_t src_dtype, int64_t src_ld, int64_t rows, int64_t K,
                               int32_t op_dtype, void* dst, hipStream_t stream);
// Layouts the GEMM addresses with 32-bit offsets (below kTopkOob): `rows`
// operand rows a_ld elements apart; the weights of n_experts experts; the
// slot table of n_tokens tokens.
bool topk_gemm_a_fits(int64_t rows, int64_t a_ld, int64_t K);
bool topk_gemm_b_fits(int32_t n_experts, int64_t b_se, int64_t b_sn, int64_t K);
bool topk_gemm_table_fits(int32_t n_experts, int64_t n_tokens);
// out = the top-k sum (16-bit op dtype; out dtype bf16, f16 or f32; K % 8 == 0, N % 8 == 0)
hipError_t launch_topk_gemm(const TopkGemmParams& p, int32_t op_dtype, int32_t out_dtype, hipStream_t stream);

}  // namespace cvmm
