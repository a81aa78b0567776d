/*
 * cvmm_hip.h -- C ABI of libcvmm_hip.so, the MI355X (gfx950) CVMM kernels.
 *
 * CVMM ("conditional vector-matrix multiply") is the routed grouped GEMM of
 * MoE projections.  Every entry point takes raw device pointers, sizes,
 * element strides, dtype ids and a hipStream_t (passed as void*), launches
 * asynchronously on that stream and never synchronises the host.  Scratch
 * memory is passed in by the caller; query its size with the matching
 * *_workspace_bytes function (a NULL/short workspace is an error).
 *
 * Terminology (reference: RobertCsordas/cvmm_codex cvmm.py):
 *   route            one (token, top-k slot) pair; R = tokens * top_k
 *   sorted_sel       int32[R]  expert ids sorted ascending       (CVMMSel.sel)
 *   sel_index        int64[R]  x row read by sorted route i      (CVMMSel.sel_index)
 *   out_index        int64[R]  route position of sorted route i, or NULL for
 *                              route-major input                   (CVMMSel.out_index)
 *   route position   rp(i) = out_index ? out_index[i] : sel_index[i]
 *   offsets          int64[E]  inclusive per-expert route counts (cumsum)
 *   reduction_weight per-route weights indexed by route position (CVMMSel.reduction_weight)
 *
 * Return value: CVMM_OK (0) or an error code; cvmm_last_error() describes the
 * last failure of the calling thread.
 */
#ifndef CVMM_HIP_H
#define CVMM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids: the reference's dtype_to_type_id (cvmm.py:36-44) */
#define CVMM_DTYPE_F32 0
#define CVMM_DTYPE_F16 1
#define CVMM_DTYPE_BF16 2

#define CVMM_OK 0
#define CVMM_ERR_INVALID 1     /* bad argument (shape, dtype, alignment, NULL) */
#define CVMM_ERR_UNSUPPORTED 2 /* valid but not implemented (e.g. > 32767 experts) */
#define CVMM_ERR_WORKSPACE 3   /* workspace missing or too small */
#define CVMM_ERR_LAUNCH 4      /* HIP launch error */

/* flags */
#define CVMM_FLAG_ATOMIC_REDUCE 1 /* top-k sums (weighted combine, token grad) by fp32 atomics
                                     instead of a route-ordered buffer + ordered row sum */
#define CVMM_FLAG_COUNTERS_ZEROED 2 /* cvmm_bwd_w: the counter region at the start of the
                                       workspace is already zero (see cvmm_bwd_w) */
#define CVMM_FLAG_COUNTS_READY 16 /* cvmm_sort_routes_cast_keys_ex: the workspace already holds the
                                     count matrix of these ids for n_experts, written by
                                     cvmm_copy_ids_count (see there) */
#define CVMM_FLAG_ACCUMULATE 32 /* cvmm_bwd_x, token-input unweighted top-k sum: grad_x is an fp32
                                   running sum; this call's sums (each route's row rounded to
                                   x_dtype, as it would be stored) are added to it in route order,
                                   unrounded.  Calls over consecutive slices of a selection's
                                   top-k columns, then one rounding to x_dtype, give the bits of
                                   one call over all of them (the low-memory grad-input). */
#define CVMM_FLAG_ROWS_SCALED 64 /* cvmm_bwd_w, weighted selection with route input: x holds the
                                    route rows already scaled, x'_r = rnd_op(rnd_op(w_r) *
                                    rnd_op(x_r)), as cvmm_fwd_keep_scaled keeps them (op dtype,
                                    one row per route); reduction_weight is still passed (the
                                    gradient rows stay one per token) but not applied again */

/* kernel classes for the timing hooks */
#define CVMM_KC_SORT 1        /* histogram + scan + scatter of cvmm_sort_routes */
#define CVMM_KC_OFFSETS 2
#define CVMM_KC_CAST_KEYS 4
#define CVMM_KC_GEMM_FWD 8    /* routed GEMM of cvmm_fwd */
#define CVMM_KC_GEMM_BWDX 16  /* routed GEMM of cvmm_bwd_x */
#define CVMM_KC_WGRAD 32      /* weight-gradient kernel of cvmm_bwd_w */
#define CVMM_KC_COMBINE 64    /* row work: top-k row combine / fp32 cast / gate-grad sum / dense
                                 top-k slot table and row scaling / weighted rows of the weight
                                 gradient */
#define CVMM_KC_FILL 128      /* zero fills */
#define CVMM_KC_ROUTE 512     /* router (softmax, top-k, histogram) + its scatter; router backward */

/* Thread-local description of the last error. */
const char* cvmm_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int cvmm_abi_version(void);

/* Measurement hooks (no counterpart in the reference; for benchmarks): while
 * a kernel class is enabled, every launch of it is bracketed by HIP events
 * recorded on the launch stream.  cvmm_timing_result synchronises on those
 * events and returns the summed elapsed milliseconds and the launch count of
 * one class, then forgets them.  Process-wide; not for concurrent use. */
int cvmm_timing_enable(uint32_t class_mask);
int cvmm_timing_result(uint32_t kernel_class, double* total_ms, int64_t* launches);

/* Tuning knobs (no counterpart in the reference; for tests and tuning
 * sweeps).  Process-wide; value 0 restores the built-in choice.
 *   CVMM_TUNE_PANEL_TILES_PER_WG: n-tiles per workgroup of the small-K
 *     routed GEMM (1..4096).
 *   CVMM_TUNE_WGRAD_ORDER: workgroup order of the weight-gradient kernel,
 *     1 = the tiles of one expert chunk on one XCD, 2 = one dW tile of every
 *     expert on one XCD, 3 = expert chunk c on XCD c % 8 with all its tiles.
 *     Built in: 3 for the 16-bit kernel's 128 x 128 dW tile, else 2.
 *   CVMM_TUNE_WGRAD_TILE: dW tile of the 16-bit weight-gradient kernel where
 *     its base tile is 128 x 128 and dW is contiguous aligned fp32: 1 = 128 x
 *     128, 2 = 256 x 128, 3 = 128 x 256, 4 = 256 x 256 of four waves, 5 =
 *     256 x 256 of eight waves.  Built in: 256 x 256 of eight waves when
 *     d_in, d_out >= 256 and the grid holds >= 4 tiles per CU.
 *   CVMM_TUNE_GEMM_ORDER: m-tile order of the routed GEMMs (forward, grad
 *     input), 1 = expert-major, 2 = token-major (tile j of every expert next
 *     to each other; up to 256 experts).  Built in: token-major for the
 *     long-K kernel when every gathered row feeds >= 32 routes.
 *   CVMM_TUNE_DENSE_TOPK: how top-k sums are taken (the weighted forward
 *     combine, the token gradient of a token-input selection): 1 = always
 *     the routed GEMM + route-ordered buffer, 2 = the dense GEMM over
 *     expert-slotted rows wherever its shapes fit (see cvmm_topk_dense).
 *     Built in: the cost model of cvmm_topk_dense.
 *   CVMM_TUNE_SORT_CHUNK: routes per chunk of the selector sort (a multiple
 *     of 256; larger chunks, fewer scatter workgroups).  Built in: >= 1024,
 *     and the count matrix (chunks x (E + 1)) at most 64K entries; a sort of
 *     fewer than 8192 routes takes 8 chunks of at least 256.  A chunk that
 *     makes the sort's workspace exceed 1 MiB fails
 *     cvmm_sort_routes_noalloc.
 *   CVMM_TUNE_WGRAD_CHUNK: routes per chunk of the weight gradient's split
 *     reduction (rounded up to the kernel's 32- or 64-route slices; an
 *     expert with more routes is split into chunks whose fp32 partials are
 *     summed in chunk order).  Built in: max(1024, 6 x the mean routes per
 *     expert).  Workspace queries depend on it: query after setting it.
 *   CVMM_TUNE_RING_TILE: tile of the long-K routed GEMM (K > 128, N > 64):
 *     1 = 128 x 128, 2 = 160 x 128, 3 = 256 x 256 of eight waves where N is
 *     a multiple of 256 (elsewhere the built-in height).  Built in: 256 x
 *     256 where it applies and the grid fills two rounds of 256 CUs (the
 *     FFN stack); else 160 rows
 *     unless the estimated dispatch rounds times the tile height come out
 *     more than 5 % higher (the ff_up forward: one round of ~442 tiles
 *     instead of 544 tiles on 512 slots).  All give the same bits. */
#define CVMM_TUNE_PANEL_TILES_PER_WG 1
#define CVMM_TUNE_WGRAD_ORDER 2
#define CVMM_TUNE_GEMM_ORDER 3
#define CVMM_TUNE_WGRAD_TILE 5
#define CVMM_TUNE_DENSE_TOPK 6
#define CVMM_TUNE_SORT_CHUNK 7
#define CVMM_TUNE_RING_TILE 8
#define CVMM_TUNE_WGRAD_CHUNK 9
int cvmm_tuning_set(int32_t knob, int64_t value);

/* Whether a top-k sum -- out[t] = sum over the top_k routes (t, j) of
 * [K]-row x [K, N] expert products, for n_tokens tokens over n_experts
 * experts -- is taken as one dense GEMM (no counterpart in the reference,
 * which writes every route's product and sums them afterwards,
 * cvmm.py:1204-1223, :1541-1545).  The dense form is the GEMM of A [T, E*K]
 * (each token's K-wide operand rows in the slots of its experts, zero
 * elsewhere) and the weights as [E*K, N] rows, with A's tiles gathered into
 * LDS on the fly from a per-(token, expert) table of first routes (a token's
 * further routes on one expert run as extra passes): fp32 accumulation, one
 * rounding, deterministic; E / top_k times the useful flops, but no [R, N]
 * route-ordered buffer (2.1 GB at SwitchHead size).  It is taken when the
 * shapes fit (16-bit op, K % 8 == 0, N % 8 == 0, 2 <= top_k <= 64, <= 1024
 * experts) and, unless CVMM_TUNE_DENSE_TOPK says otherwise, a cost model of
 * the two ways (measured rates) favours it: at high fan-out (top_k / E >=
 * ~1/4).
 *   cvmm_fwd, weighted:          K = d_in,  N = d_out; the weights are read
 *     as they stand when an op-dtype copy with unit stride on d_in (the
 *     [E][d_out][d_in] copy, or its expert-interleaved [d_out][E][d_in] form);
 *   cvmm_bwd_x, unweighted token input, top_k > 1: K = d_out, N = d_in; the
 *     weights with unit stride on d_out ([E][d_in][d_out] or [d_in][E][d_out]).
 * Other keys are cast into the workspace.  Returns 1 or 0. */
int cvmm_topk_dense(int64_t n_tokens, int32_t n_experts, int64_t K, int64_t N, int64_t top_k, int32_t op_dtype);

/* ------------------------------------------------------------------------ */
/* Selector preparation                                                      */
/* ------------------------------------------------------------------------ */

size_t cvmm_sort_workspace_bytes(int64_t n_routes, int32_t n_experts);

/* Stable counting sort of the flattened expert ids `sel` (int32, or int64
 * read as its low 32 bits, the value the reference's int32 conversion gives).
 * Replaces the sort in cvmm_prepare_sel (cvmm.py:24-27) and
 * cvmm_prepare_sel2 (cvmm.py:1796-1803) plus the offsets kernel
 * (cvmm.py:315-335).  Writes sorted_sel[R] (int32), perm[R] (int64, the
 * stable sorting permutation), token_index[R] = perm / top_k when
 * token_index != NULL, offsets[E] (int64 inclusive cumsum), when
 * route_pos != NULL the inverse permutation route_pos[perm[i]] = i (int32;
 * no counterpart in the reference: it lets cvmm_fwd / cvmm_bwd_x gather each
 * token's routes from route-ordered rows) and, when n_invalid != NULL, the
 * number of ids outside [0, E) (those sort last and are ignored by the
 * GEMMs). */
int cvmm_sort_routes(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                     int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                     int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                     size_t workspace_bytes, void* stream);

/* cvmm_sort_routes without a workspace argument (no counterpart in the
 * reference: for callers that cannot allocate device memory -- code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and outputs as cvmm_sort_routes minus the workspace; calls no
 * hipMalloc/hipFree.  The scratch is a static device array of 1 MiB per GPU
 * (held until the process ends), enough for every size cvmm_sort_routes
 * accepts (<= 32767 experts need at most 512 KiB); a larger need would be
 * refused with CVMM_ERR_WORKSPACE.  Call it with the stream's device
 * current.  Calls that overlap on one GPU (different streams) share the
 * scratch and race: serialise them. */
int cvmm_sort_routes_noalloc(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                             int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                             int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* stream);

/* cvmm_sort_routes and cvmm_cast_keys in one call (no counterpart in the
 * reference, whose sort and in-kernel weight cast are separate steps): the
 * cast of the same step's weights runs in the launch that scatters the
 * routes, so the latency-bound scatter hides behind it.  Arguments and
 * outputs as in the two calls; the two keys/output arguments follow the
 * cast's.  Falls back to the two separate launches where the vectorised cast
 * does not apply. */
int cvmm_sort_routes_cast_keys(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                               int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                               size_t workspace_bytes, const void* keys, int32_t keys_dtype, int64_t d_in,
                               int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype,
                               void* keys_t, void* keys_n, int32_t layout, void* stream);

/* cvmm_sort_routes_cast_keys with flags: CVMM_FLAG_COUNTS_READY skips the
 * sort's histogram launch, whose count matrix the workspace already holds
 * (cvmm_copy_ids_count of the same ids for the same n_experts).  The library
 * keeps a record of each such count (workspace, ids, experts, sort chunk)
 * and honours the flag only when the record matches this call and the
 * sort-chunk tuning knob still gives the same chunk; the record is used up.
 * Otherwise the sort counts again.  keys == NULL (or both outputs NULL): the
 * sort alone, as cvmm_sort_routes.  No counterpart in the reference. */
int cvmm_sort_routes_cast_keys_ex(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                                  int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                                  int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                                  size_t workspace_bytes, const void* keys, int32_t keys_dtype, int64_t d_in,
                                  int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype,
                                  void* keys_t, void* keys_n, int32_t layout, int32_t flags, void* stream);

/* Router (no counterpart in cvmm.py; replaces its callers' router lines,
 * benchmark_ffn_moe.py:91-97 and benchmark_framework_moe.py:129-135:
 *   probs = softmax(logits.float()); weights, sel = probs.topk(top_k)
 *   weights = weights / weights.sum(-1).clamp_min(1e-20)   (renormalize != 0)
 *   cvmm_prepare_sel2(sel)                                  (cvmm.py:1786-1803)).
 * logits: [n_tokens][n_experts] rows (row stride logits_ld), fp32 / bf16 /
 * fp16.  Writes weights[n_tokens * top_k] (fp32) and sel[n_tokens * top_k]
 * (int64) in probability order (descending, ties to the lower expert id, NaN
 * lowest), then the outputs of cvmm_sort_routes for sel (token_index and
 * route_pos may be NULL).  Two launches: the router (one wave per token,
 * leaving the sort's per-chunk histogram) and the sort's stable scatter.
 * Limits: n_experts <= 1024, top_k <= min(64, n_experts). */
size_t cvmm_route_topk_workspace_bytes(int64_t n_tokens, int32_t n_experts, int64_t top_k);
int cvmm_route_topk(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                    int32_t n_experts, int64_t top_k, int32_t renormalize, float* weights, int64_t* sel,
                    int32_t* sorted_sel, int64_t* perm, int64_t* token_index, int64_t* offsets,
                    int32_t* route_pos, void* workspace, size_t workspace_bytes, void* stream);
/* Gradient of the router's weights with respect to the logits (the softmax,
 * top-k and renormalisation backward of the lines above):
 * grad_logits[t][e] = p_e (g_e - sum_i g_i p_i), g = d loss / d probs, in the
 * logits dtype (row stride grad_ld).  sel and grad_weights as written and
 * received for cvmm_route_topk's outputs. */
int cvmm_route_topk_backward(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                             int32_t n_experts, int64_t top_k, int32_t renormalize, const int64_t* sel,
                             const float* grad_weights, void* grad_logits, int64_t grad_ld, void* stream);

/* out[i] = the int32 value of id i (int64 ids: their low 32 bits), n ids:
 * the `fsel = sel.flatten().to(torch.int32)` copy cvmm_prepare_sel2 takes
 * (cvmm.py:1796), which fixes the routing when the selector is prepared. */
int cvmm_copy_ids(const void* sel, int32_t sel_is_int64, int64_t n, int32_t* out, void* stream);

/* cvmm_copy_ids that also writes, into a sort workspace (size
 * cvmm_sort_workspace_bytes(n, n_experts)), the per-chunk expert histogram
 * the sort of the copy would compute first for n_experts; a later
 * cvmm_sort_routes_cast_keys_ex with CVMM_FLAG_COUNTS_READY and that
 * workspace skips its histogram launch.  The copy is what cvmm_copy_ids
 * writes (cvmm.py:1796); the histogram has no counterpart in the reference:
 * cvmm_prepare_sel2 does not know the expert count, so the caller passes the
 * count it expects and sorts without the flag when the call uses another. */
int cvmm_copy_ids_count(const void* sel, int32_t sel_is_int64, int64_t n, int32_t n_experts, int32_t* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* offsets[e] = #{i : sorted_sel[i] <= e}; replaces cvmm_expert_offsets
 * (cvmm.py:1108-1120, kernel cvmm.py:315-335). */
int cvmm_expert_offsets(const int32_t* sorted_sel, int64_t n_routes, int32_t n_experts, int64_t* offsets,
                        void* stream);

/* Cast the expert weights once per step to the MFMA operand type (bf16/f16)
 * in the two k-contiguous layouts the routed GEMMs read:
 *   keys_t [E][d_out][d_in]  (forward)   keys_n [E][d_in][d_out]  (grad-input)
 * Either output may be NULL.  `layout` bits interleave the experts between
 * the rows instead: CVMM_CAST_T_INTERLEAVED writes keys_t as
 * [d_out][E][d_in], CVMM_CAST_N_INTERLEAVED keys_n as [d_in][E][d_out] -- the
 * B^T rows of a dense top-k sum (cvmm_topk_dense), passed to cvmm_fwd /
 * cvmm_bwd_x as the logical [E, d_in, d_out] view (strides (d_in, 1, E*d_in)
 * and (d_out, E*d_out, 1)).  Replaces the per-tile in-register weight cast
 * of cvmm_kernel (cvmm.py:198-204) with one pass per step; RNE rounding. */
#define CVMM_CAST_T_INTERLEAVED 1
#define CVMM_CAST_N_INTERLEAVED 2
int cvmm_cast_keys(const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
                   int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype, void* keys_t, void* keys_n,
                   int32_t layout, void* stream);

/* ------------------------------------------------------------------------ */
/* Forward: CVMM.forward (cvmm.py:1524-1550) = cvmm_triton (cvmm.py:814-867)  */
/* + the weighted top-k combine (cvmm.py:1543-1545)                            */
/* ------------------------------------------------------------------------ */

/* y_i = rnd_out(x[sel_index[i]] @ keys[sorted_sel[i]]) for each sorted route i.
 *  reduction_weight == NULL: out[rp(i)] = y_i            (out: [R, d_out])
 *  otherwise:                out[t] = rnd_out(sum_j rnd_out(w[t*k+j]) * y_(t*k+j))
 *                                                       (out: [R/reduce_k, d_out])
 * keys element (e, i, j) is at keys[e*k_se + i*k_si + j*k_sj]; x rows are
 * contiguous with row stride x_ld.  op_dtype is the MFMA operand type
 * (autocast dtype or F32); x/keys are converted to it in-kernel.  Op-dtype
 * keys with either inner stride 1 take the DMA-staged kernels where the
 * product's k dimension (d_in here, d_out in cvmm_bwd_x) exceeds 128; so one
 * cast copy (cvmm_cast_keys) can serve both products of a step.
 * route_pos (optional): the inverse of rp = out_index or sel_index, as
 * cvmm_sort_routes writes it; computed in the workspace when NULL.
 * Top-k sums (weighted here, token-input in cvmm_bwd_x) are taken in one of
 * three ways: fp32 atomics (CVMM_FLAG_ATOMIC_REDUCE, not deterministic in the
 * last bits); the dense GEMM over expert-slotted rows where cvmm_topk_dense
 * says so (the per-token sum in the GEMM's fp32 accumulators, one rounding);
 * else a route-ordered buffer and a per-token sum in route order (each
 * route's product rounded first, as the reference does).  The last two are
 * deterministic.
 * Routes whose expert id is outside [0, E) (no counterpart: the reference
 * indexes keys with them) are left out: the top-k sums skip them, and their
 * own rows of out (unweighted) or grad_x (per-route gradient) are zero. */
size_t cvmm_fwd_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t out_rows,
                                int32_t out_dtype, int32_t op_dtype, int32_t has_offsets, int32_t weighted,
                                int32_t flags);
int cvmm_fwd(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld,
             const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
             int64_t k_se, int64_t k_si, int64_t k_sj,
             const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
             const int64_t* offsets, const int32_t* route_pos, const void* reduction_weight, int32_t rw_dtype,
             int64_t reduce_k, int32_t op_dtype, void* out, int32_t out_dtype, int64_t out_rows, int64_t out_ld,
             int32_t flags, void* workspace, size_t workspace_bytes, void* stream);

/* cvmm_fwd that keeps the scaled route rows of a weighted top-k sum for the
 * backward.  For route input (out_index NULL, x_rows == n_routes) with a
 * 16-bit op and out_dtype == op_dtype, where the call makes them anyway --
 * the dense GEMM's operand rows (cvmm_topk_dense), or the activation
 * fragments of the small-K routed product (d_in <= 128, 16-byte aligned
 * op-dtype rows and keys) -- the rows x'_r = rnd_op(rnd_op(w_r) * rnd_op(x_r)),
 * bit for bit the rows cvmm_bwd_w would scale, are written to scaled_rows
 * ([n_routes][d_in], op dtype, row stride d_in) and *scaled_written is set to
 * 1; otherwise nothing is written there and *scaled_written is 0.  Rows of
 * routes whose expert id is outside [0, E) may be left unwritten (no product
 * reads them).  cvmm_bwd_w with CVMM_FLAG_ROWS_SCALED then takes them as x,
 * without its own scaling pass.  Same workspace as cvmm_fwd.  No counterpart
 * in the reference (which scales inside its kernels): it saves the weight
 * gradient a read and a write of the route rows. */
int cvmm_fwd_keep_scaled(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld,
                         const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
                         int64_t k_se, int64_t k_si, int64_t k_sj,
                         const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index,
                         int64_t n_routes, const int64_t* offsets, const int32_t* route_pos,
                         const void* reduction_weight, int32_t rw_dtype, int64_t reduce_k, int32_t op_dtype,
                         void* out, int32_t out_dtype, int64_t out_rows, int64_t out_ld, void* scaled_rows,
                         int32_t* scaled_written, int32_t flags, void* workspace, size_t workspace_bytes,
                         void* stream);

/* cvmm_fwd followed by the GELU (erf form), for the up projection of the
 * reference's MoE callers (no counterpart in cvmm.py: its callers write
 * F.gelu(cvmm(...)), benchmark_ffn_moe.py:96).  Unweighted selections:
 * pre_act = h = what cvmm_fwd writes to out, out = rnd_out(gelu(h)); pre_act
 * has out's shape, dtype and row stride (kept for cvmm_gelu_backward).  When
 * the long-K GEMM (d_in > 128, 16-bit op) runs, the GELU is in its epilogue
 * and both outputs are written once; otherwise a GELU pass follows the GEMM.
 * Workspace: cvmm_fwd_workspace_bytes of the unweighted call. */
int cvmm_fwd_gelu(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld,
                  const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
                  int64_t k_se, int64_t k_si, int64_t k_sj,
                  const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
                  const int64_t* offsets, const int32_t* route_pos, int32_t op_dtype, void* out, int32_t out_dtype,
                  int64_t out_rows, int64_t out_ld, void* pre_act, int32_t flags, void* workspace,
                  size_t workspace_bytes, void* stream);
/* grad_pre = rnd(grad * gelu'(pre_act)) per element of a [rows][cols] block
 * (the GELU backward; gelu'(x) = 0.5 (1 + erf(x / sqrt 2)) + x exp(-x^2/2) /
 * sqrt(2 pi)). */
int cvmm_gelu_backward(const void* grad, int32_t grad_dtype, int64_t grad_ld, const void* pre_act,
                       int32_t pre_dtype, int64_t pre_ld, int64_t rows, int64_t cols, void* grad_pre,
                       int32_t grad_pre_dtype, int64_t grad_pre_ld, void* stream);

/* ------------------------------------------------------------------------ */
/* Backward, input side: grad_x and the reduction-weight gradient.          */
/* Replaces cvmm_grouped_bwd_x_kernel (+ top-k .sum, cvmm.py:1204-1223),     */
/* cvmm_weighted_route_bwd_x (cvmm.py:1386-1433) and the generic fallback    */
/* (cvmm.py:1687-1753).                                                       */
/* ------------------------------------------------------------------------ */

/* g_i = grad[rp(i) / (weighted ? top_k : 1)] @ keys[e_i]^T, then
 *  unweighted, route-major x or top_k == 1 : grad_x[rp(i)] = rnd_x(g_i)
 *  unweighted, token x, top_k > 1          : grad_x[t] = rnd_x(sum_j rnd_x(g_(t,j)))
 *  weighted, route-major x                 : grad_x[rp] = rnd_x(rnd_op(rnd_op(g) * rnd_op(w[rp])))
 *  weighted, token x                       : grad_x[t] = rnd_x(rnd_op(sum_j rnd_op(w) * rnd_op(g)))
 *  weighted (both)                          : grad_rw[rp] = <rnd_op(g_i), x[sel_index[i]]>
 * grad_x and/or grad_rw may be NULL when not needed; route_pos and the
 * top-k sum's flags as for cvmm_fwd (here K = d_out, N = d_in; the reduce
 * GEMM is not taken for a weighted call that asks for grad_rw).  With
 * grad_rw and d_out > 128, 16-bit x with 8-byte aligned rows (x pointer and
 * x_ld) keeps the DMA-staged kernel; other x takes the slower tiled one.
 * CVMM_FLAG_ACCUMULATE (the low-memory grad-input over slices of the top-k
 * columns, cvmm.py:1228-1338): grad_x fp32 holds a running sum that the
 * call adds to; x may be NULL but x_dtype names the rows' dtype; the
 * workspace query takes that dtype as grad_x_dtype. */
size_t cvmm_bwd_x_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                  int64_t grad_x_rows, int32_t has_offsets, int32_t weighted, int32_t token_input,
                                  int64_t top_k, int32_t grad_x_dtype, int32_t op_dtype, int32_t need_grad_rw,
                                  int32_t flags);
int cvmm_bwd_x(const void* grad, int32_t grad_dtype, int64_t grad_rows, int64_t grad_ld,
               const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
               int64_t k_se, int64_t k_si, int64_t k_sj,
               const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
               const int64_t* offsets, const int32_t* route_pos, const void* reduction_weight, int32_t rw_dtype,
               int64_t top_k, const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, int32_t op_dtype,
               void* grad_x, int32_t grad_x_dtype, int64_t grad_x_rows, int64_t grad_x_ld,
               void* grad_rw, int32_t grad_rw_dtype,
               int32_t flags, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Backward, weight side: grad_keys[e] = sum_{i in e} x_i^T G_i              */
/* Replaces cvmm_grouped_bwd_w_gather_x_kernel (cvmm.py:481-538),            */
/* cvmm_grouped_bwd_w_weighted_kernel (cvmm.py:541-604) and                  */
/* cvmm_triton_backward / kernel3 (cvmm.py:1470-1518, :607-805).             */
/* Deterministic: fixed route chunks, partials summed in chunk order.        */
/* ------------------------------------------------------------------------ */

/* x_i = rnd_op(x[sel_index[i]]), G_i = rnd_op(grad[rp(i)]) (unweighted) or
 * rnd_op(rnd_op(grad[rp(i)/top_k]) * rnd_op(w[rp(i)])) (weighted).  Every
 * expert's gradient is written, zeros for experts without routes.
 * The workspace starts with cvmm_bwd_w_counter_bytes() bytes of tile
 * counters.  They must be zero on entry: the call zeroes them itself unless
 * flags has CVMM_FLAG_COUNTERS_ZEROED, and it leaves them zero when it ends,
 * so a caller that keeps one workspace per stream zeroes it once. */
size_t cvmm_bwd_w_counter_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                int32_t op_dtype);
size_t cvmm_bwd_w_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                  int32_t op_dtype, int32_t has_offsets);
/* The workspace of a weighted selection with route input (x row = route,
 * out_index NULL) given room for its scaled rows: with at least this many
 * bytes, cvmm_bwd_w scales each route row once, x'_r = rnd_op(rnd_op(w_r) *
 * rnd_op(x_r)) (16-bit op, d_in % 8 == 0), and runs the unweighted product
 * sum_i x'_i^T rnd_op(grad[rp(i)/top_k]) -- the weight applied to the route
 * row instead of the gradient row (the rounding point moves; the product is
 * the same).  With cvmm_bwd_w_workspace_bytes' size the weight is applied to
 * the gradient rows inside the kernel.  weighted_route_input = 0: the same as
 * cvmm_bwd_w_workspace_bytes.  No counterpart in the reference. */
size_t cvmm_bwd_w_workspace_bytes_ex(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                     int32_t op_dtype, int32_t has_offsets, int32_t weighted_route_input);
int cvmm_bwd_w(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld,
               const void* grad, int32_t grad_dtype, int64_t grad_rows, int64_t grad_ld,
               int32_t n_experts, int64_t d_in, int64_t d_out,
               const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
               const int64_t* offsets, const void* reduction_weight, int32_t rw_dtype, int64_t top_k,
               int32_t op_dtype, void* grad_keys, int32_t grad_keys_dtype, int64_t gk_se, int64_t gk_si,
               int64_t gk_sj, int32_t flags, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CVMM_HIP_H */
