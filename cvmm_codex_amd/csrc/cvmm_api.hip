// C ABI of libcvmm_hip.so: argument checking, workspace carving and the
// per-case choice of kernels (the reference's CVMM.backward dispatcher,
// cvmm.py:1552-1755, reduced to what the selector layout decides).
#include <string>
#include <cstdio>
#include <cstdarg>
#include <atomic>
#include <mutex>
#include <vector>

#include "cvmm_common.h"
#include "cvmm_internal.h"
#include "../../include/cvmm_hip.h"

namespace cvmm {
hipError_t launch_routed_gemm_bf16(const GemmParams& p, hipStream_t stream);
hipError_t launch_routed_gemm_f16(const GemmParams& p, hipStream_t stream);
hipError_t launch_routed_gemm_f32(const GemmParams& p, hipStream_t stream);
hipError_t launch_wgrad_bf16(const WgradParams& p, hipStream_t stream);
hipError_t launch_wgrad_f16(const WgradParams& p, hipStream_t stream);
hipError_t launch_wgrad_f32(const WgradParams& p, hipStream_t stream);

hipError_t launch_routed_gemm_nt_bf16(const GemmParams& p, hipStream_t stream);
hipError_t launch_routed_gemm_nt_f16(const GemmParams& p, hipStream_t stream);
bool routed_gemm_ring_applies(const GemmParams& p, int32_t op);
bool routed_gemm_panel_applies(const GemmParams& p, int32_t op);

// Fast path (DMA-staged, 16-bit k-contiguous operands) when eligible, else the
// general kernel (any storage type / stride / width).
// Weights k-contiguous, or n-contiguous ([k][n] rows of the other
// orientation's copy) where the long-K ring kernel takes them.
static bool nt_eligible(const GemmParams& p, int32_t op) {
  auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool common = (op == kBF16 || op == kF16) && p.a_dtype == op && p.b_dtype == op && p.K % 8 == 0 &&
                      p.epi == kEpiStore && al(p.a) && al(p.b) && p.a_ld % 8 == 0 && p.b_se % 8 == 0;
  if (!common) return false;
  if (p.b_sk == 1) return p.b_sn % 8 == 0;
  return p.b_sn == 1 && p.b_sk % 8 == 0 && p.N % 8 == 0 && routed_gemm_ring_applies(p, op);
}

// Whether launch_routed_gemm runs the small-K (panel) kernel for p: the only
// kernel that writes xs_out.
static bool routed_gemm_is_panel(const GemmParams& p, int32_t op) {
  return !small_gemm_eligible(p, op) && nt_eligible(p, op) && routed_gemm_panel_applies(p, op);
}

hipError_t launch_routed_gemm(const GemmParams& p, int32_t op, hipStream_t s) {
  if (small_gemm_eligible(p, op)) return launch_routed_small(p, s);
  if (nt_eligible(p, op)) return op == kBF16 ? launch_routed_gemm_nt_bf16(p, s) : launch_routed_gemm_nt_f16(p, s);
  if (p.act != 0) return hipErrorInvalidValue;  // the activation epilogue exists in the ring kernel only
  if (op == kBF16) return launch_routed_gemm_bf16(p, s);
  if (op == kF16) return launch_routed_gemm_f16(p, s);
  if (op == kF32) return launch_routed_gemm_f32(p, s);
  return hipErrorInvalidValue;
}

hipError_t launch_wgrad_v3_bf16(const WgradParams& p, hipStream_t stream);
hipError_t launch_wgrad_v3_f16(const WgradParams& p, hipStream_t stream);

// Fast path: 16-bit x and dY in the op dtype, 16-byte aligned rows, widths % 8.
static bool wgrad_fast_eligible(const WgradParams& p, int32_t op) {
  auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  return (op == kBF16 || op == kF16) && p.x_dtype == op && p.g_dtype == op && p.M % 8 == 0 && p.N % 8 == 0 &&
         al(p.x) && al(p.g) && p.x_ld % 8 == 0 && p.g_ld % 8 == 0;
}

hipError_t launch_wgrad(const WgradParams& p, int32_t op, hipStream_t s) {
  if (small_wgrad_eligible(p, op)) return launch_wgrad_small(p, s);
  if (wgrad_fast_eligible(p, op)) return op == kBF16 ? launch_wgrad_v3_bf16(p, s) : launch_wgrad_v3_f16(p, s);
  if (op == kBF16) return launch_wgrad_bf16(p, s);
  if (op == kF16) return launch_wgrad_f16(p, s);
  if (op == kF32) return launch_wgrad_f32(p, s);
  return hipErrorInvalidValue;
}

// m-tile height the routed GEMM uses for output width N (kept in sync with
// launch_routed_gemm_op: 256x64 tiles for N <= 64, else 128x128).
int routed_gemm_bm(int64_t N) { return N <= 64 ? 256 : 128; }

// routes per weight-gradient chunk (CVMM_TUNE_WGRAD_CHUNK; 0: built in)
static std::atomic<int64_t> g_wgrad_chunk{0};

void wgrad_geometry(int64_t M, int64_t N, int64_t n_routes, int32_t n_experts, int32_t op_dtype, int64_t* split,
                    int64_t* grid_chunks, int64_t* max_slots, int64_t* tiles_mn) {
  const int64_t bk = op_dtype == kF32 ? 32 : 64;
  // chunk = max(1024, 6 * mean routes per expert): an expert is split only
  // when it holds over six times the mean.  Every split adds an fp32 partial
  // of the expert's dW per chunk, written and read back; measured on the FFN
  // stack (Zipf-skewed, up to 16x the mean on one expert) the weight gradient
  // takes 670 / 570 / 516 / 534 / 644 / 710 us per launch at 2 / 4 / 6 / 8 /
  // 12 / 16 x the mean (unsplit experts beyond that become the last
  // workgroups to finish); balanced configs do not split at any of them.
  const int64_t knob = g_wgrad_chunk.load();
  int64_t s = knob;
  if (s <= 0) {
    s = n_experts > 0 ? (6 * n_routes + n_experts - 1) / n_experts : n_routes;
    if (s < 1024) s = 1024;
  }
  s = (s + bk - 1) / bk * bk;
  *split = s;
  *grid_chunks = (n_routes + s - 1) / s + n_experts;
  // a multi-chunk expert has > s routes and < 2*count/s chunks
  *max_slots = (2 * n_routes) / s + 1;
  int bm, bn;
  wgrad_tile(M, N, &bm, &bn);
  *tiles_mn = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

int32_t wgrad_auto_tile(int64_t M, int64_t N, int64_t grid_chunks) {
  if (M < 256 || N < 256) return kWgTileBase;
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  return grid_chunks * tiles >= 4 * 256 ? kWgTile256x256W8 : kWgTileBase;
}

// fp32 partial elements of one slot: the M x N rounding of the tile the
// launch may take, at most (base or any coarser fast-path tile)
int64_t wgrad_partial_elems(int64_t M, int64_t N) {
  int64_t best = 0;
  for (int32_t c = kWgTileBase; c <= kWgTile256x256W8; ++c) {
    int bm, bn;
    wgrad_fast_tile(M, N, c, &bm, &bn);
    const int64_t e = ((M + bm - 1) / bm * bm) * ((N + bn - 1) / bn * bn);
    best = e > best ? e : best;
  }
  return best;
}

}  // namespace cvmm

using namespace cvmm;

namespace {

// ---- timing hooks -----------------------------------------------------------
struct TimedLaunch {
  uint32_t cls;
  hipEvent_t start, stop;
};
std::atomic<int32_t> g_panel_tpw{0};
std::atomic<int32_t> g_wgrad_order{0};
std::atomic<int32_t> g_wgrad_tile{0};
std::atomic<int32_t> g_gemm_order{0};
std::atomic<int32_t> g_dense_topk{0};
std::atomic<int32_t> g_ring_tile{0};

// m-tile order of the routed GEMMs (see GemmParams::token_major): the knob's
// choice, or -1 to let the kernel launcher decide
int32_t gemm_token_major(int32_t n_experts) {
  if (n_experts > kTokenMajorMaxExperts) return 0;
  const int32_t o = g_gemm_order.load();
  return o == 2 ? 1 : (o == 1 ? 0 : -1);
}
std::mutex g_timing_mu;
uint32_t g_timing_mask = 0;
std::vector<TimedLaunch> g_timed;

// Runs `launch()` (which enqueues on `stream`), bracketed by events when the
// class is being timed.
template <typename F>
hipError_t timed(uint32_t cls, hipStream_t stream, F&& launch);
template <typename F>
hipError_t timed_combine(hipStream_t stream, F&& launch) { return timed(CVMM_KC_COMBINE, stream, launch); }
template <typename F>
hipError_t timed_fill(hipStream_t stream, F&& launch) { return timed(CVMM_KC_FILL, stream, launch); }

template <typename F>
hipError_t timed(uint32_t cls, hipStream_t stream, F&& launch) {
  uint32_t mask;
  {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    mask = g_timing_mask;
  }
  if (!(mask & cls)) return launch();
  TimedLaunch t{cls, nullptr, nullptr};
  if (hipEventCreate(&t.start) != hipSuccess || hipEventCreate(&t.stop) != hipSuccess) return launch();
  hipEventRecord(t.start, stream);
  const hipError_t e = launch();
  hipEventRecord(t.stop, stream);
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timed.push_back(t);
  return e;
}

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(CVMM_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return CVMM_OK;
}

bool valid_dtype(int32_t d) { return d == kF32 || d == kF16 || d == kBF16; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Workspace carving: fixed-order list of 256-byte aligned regions.
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  void* take(size_t bytes) {
    void* p = base ? base + used : nullptr;
    used = align_up(used + bytes, 256);
    return p;
  }
};

// Route-major buffer dtype / reduce rules shared by the workspace query and
// the compute entry point.
bool reduce_needed(int32_t weighted, int32_t token_input, int64_t top_k) {
  return token_input && (weighted || top_k > 1);
}

int64_t ntiles_of(int64_t n, int64_t bn) { return (n + bn - 1) / bn; }

// Dense top-k sum (cvmm_topk_gemm.hip) for a sum over top_k routes per token
// of [K] x [K, N] products: the shapes it handles ...
bool dense_topk_shape_ok(int32_t op_dtype, int64_t n_tokens, int32_t n_experts, int64_t K, int64_t N,
                         int64_t top_k) {
  const int64_t lim = 0x7fffffffll;
  if (!((op_dtype == kBF16 || op_dtype == kF16) && K % 8 == 0 && N % 8 == 0 && top_k >= 2 && top_k <= 64 &&
        n_experts <= kTopkMaxExperts && n_tokens > 0 && n_tokens <= lim && N <= lim &&
        (int64_t)n_experts * K <= lim && n_tokens * top_k <= lim))
    return false;
  // the GEMM's 32-bit offsets reach the workspace copies (rows of K, weights
  // [E][N][K]) and the slot table
  return topk_gemm_a_fits(n_tokens * top_k, K, K) && topk_gemm_b_fits(n_experts, K * N, K, K) &&
         topk_gemm_table_fits(n_experts, n_tokens);
}
// ... and when it is the faster way (rates measured on MI355X: the dense GEMM
// at ~1.2 PFLOP/s over E/top_k times the useful flops, against the routed
// GEMM at ~0.5 PFLOP/s plus the [R, N] route buffer written and read at ~5
// TB/s); the CVMM_TUNE_DENSE_TOPK knob overrides it (1 never, 2 whenever the
// shapes fit).
bool use_dense_topk(int32_t op_dtype, int64_t n_tokens, int32_t n_experts, int64_t K, int64_t N, int64_t top_k) {
  if (!dense_topk_shape_ok(op_dtype, n_tokens, n_experts, K, N, top_k)) return false;
  const int32_t knob = g_dense_topk.load();
  if (knob == 1) return false;
  if (knob == 2) return true;
  const double T = (double)n_tokens, R = T * (double)top_k;
  const double t_dense = 2.0 * T * n_experts * K * N / 1.2e15;
  const double t_route = R * N * 2 * 2 / 5e12 + 2.0 * R * K * N / 0.5e15;
  return t_dense < t_route;
}

// Workspace of a dense top-k sum: a weight copy in a layout the GEMM reads
// (used when the caller's keys are not one), the inverse route permutation
// (when not given), the slot table, and [R][K] op-dtype operand rows (the
// weight-scaled route rows of a weighted sum, or a copy of rows that cannot
// be moved 16 bytes at a time).
struct DenseWs {
  void* b;
  int32_t* inv;
  uint32_t* offs;
  uint8_t* slots;
  uint8_t* nxt;
  uint8_t* mult;
  void* src;
};
DenseWs carve_dense(Carver& c, int64_t n_tokens, int32_t n_experts, int64_t K, int64_t N, int64_t n_routes,
                    int32_t op_dtype) {
  const size_t esz = dtype_size(op_dtype), e16 = (size_t)topk_e16(n_experts);
  DenseWs w;
  w.b = c.take((size_t)n_experts * K * N * esz);
  w.inv = (int32_t*)c.take((size_t)n_routes * 4);
  w.offs = (uint32_t*)c.take((size_t)topk_slot_rows(n_tokens) * e16 * 4);
  w.slots = (uint8_t*)c.take((size_t)topk_slot_rows(n_tokens) * e16);
  w.nxt = (uint8_t*)c.take((size_t)n_routes);
  w.mult = (uint8_t*)c.take((size_t)n_tokens);
  w.src = c.take((size_t)n_routes * K * esz);
  return w;
}

// The dense top-k sum: out[t] = sum_j s_tj src[row(t, j)] @ B_e, with K =
// d_in, N = d_out for the forward (`fwd`), K = d_out, N = d_in for the
// grad-input.  `keys` (the logical [E, d_in, d_out] view with its strides) is
// read as it stands when it is an op-dtype copy whose K dimension has unit
// stride (the per-expert copy of this product's orientation, or its
// expert-interleaved form); other keys are cast into the workspace.
int run_dense_topk(const DenseWs& w, const void* src, int32_t src_dtype, int64_t src_ld, bool src_per_route,
                   const int32_t* sorted_sel, const int32_t* route_pos, const int64_t* rp, const int64_t* offs,
                   int64_t n_routes, int64_t n_tokens, int64_t top_k, int32_t n_experts, const void* keys,
                   int32_t keys_dtype, int64_t d_in, int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj,
                   bool fwd, const void* rw, int32_t rw_dtype, int32_t w_round, int32_t op_dtype, void* out,
                   int32_t out_dtype, int64_t out_ld, uint32_t gemm_class, const char* what, hipStream_t s,
                   void* scaled_rows = nullptr) {
  const int64_t K = fwd ? d_in : d_out, N = fwd ? d_out : d_in;
  const int64_t esz = (int64_t)dtype_size(op_dtype);
  // B_e[k][n] = b[e * b_se + n * b_sn + k]: keys[e][k][n] for the forward,
  // keys[e][n][k] for the grad-input
  const void* B = keys;
  int64_t b_se = k_se, b_sn = fwd ? k_sj : k_si;
  const int64_t k_unit = fwd ? k_si : k_sj;
  if (!(keys_dtype == op_dtype && k_unit == 1 && aligned16(keys) && (k_se * esz) % 16 == 0 &&
        (b_sn * esz) % 16 == 0 && topk_gemm_b_fits(n_experts, b_se, b_sn, K))) {
    // the per-expert copy of this orientation: kt [E][d_out][d_in] or kn [E][d_in][d_out]
    int r = check_launch(timed(CVMM_KC_CAST_KEYS, s, [&] {
      return launch_cast_keys(keys, keys_dtype, k_se, k_si, k_sj, n_experts, d_in, d_out, op_dtype,
                              fwd ? w.b : nullptr, fwd ? nullptr : w.b, 0, s);
    }), what);
    if (r) return r;
    B = w.b;
    b_se = K * N;
    b_sn = K;
  }
  const int32_t* inv = route_pos;
  if (!inv) {
    int r = check_launch(timed_combine(s, [&] { return launch_invert_rows(rp, n_routes, w.inv, s); }), what);
    if (r) return r;
    inv = w.inv;
  }
  // operand rows: with routing weights the scaled route rows (a launch of
  // their own); else the rows as given when they are 16-byte pieces of the op
  // dtype, or an op-dtype copy
  const void* A = src;
  int64_t a_ld = src_ld;
  if (rw != nullptr) {
    // (into the caller's buffer when it keeps them: [n_routes][K])
    void* dst = scaled_rows != nullptr ? scaled_rows : w.src;
    int r = check_launch(timed_combine(s, [&] {
      return launch_scale_rows(src, src_dtype, src_ld, src_per_route, rw, rw_dtype, w_round, n_routes, top_k, K,
                               op_dtype, dst, s);
    }), what);
    if (r) return r;
    A = dst;
    a_ld = K;
  } else if (!(src_dtype == op_dtype && src_per_route && aligned16(src) && (src_ld * esz) % 16 == 0 &&
                topk_gemm_a_fits(n_routes, src_ld, K))) {
    // (an unweighted sum always comes with route rows: the token gradient)
    int r = check_launch(timed_combine(s, [&] {
      return launch_copy_rows_op(src, src_dtype, src_ld, n_routes, K, op_dtype, w.src, s);
    }), what);
    if (r) return r;
    A = w.src;
    a_ld = K;
  }
  int r = check_launch(timed_combine(s, [&] {
    return launch_topk_slot_table(sorted_sel, inv, rp, offs + (n_experts - 1), n_tokens, top_k, n_experts, a_ld,
                                  K, w.offs, w.slots, w.nxt, w.mult, s);
  }), what);
  if (r) return r;
  TopkGemmParams p{};
  p.src = A;
  p.src_ld = a_ld;
  p.offs = w.offs;
  p.slots = w.slots;
  p.t_pad = topk_slot_rows(n_tokens);
  p.nxt = w.nxt;
  p.mult = w.mult;
  p.b = B;
  p.b_se = b_se;
  p.b_sn = b_sn;
  p.n_tokens = n_tokens;
  p.top_k = top_k;
  p.K = K;
  p.N = N;
  p.n_experts = n_experts;
  p.e16 = topk_e16(n_experts);
  p.out = out;
  p.out_ld = out_ld;
  p.out_vec = aligned16(out) && (out_ld * (int64_t)dtype_size(out_dtype)) % 16 == 0;
  return check_launch(timed(gemm_class, s, [&] { return launch_topk_gemm(p, op_dtype, out_dtype, s); }), what);
}

// n-tile width of the routed GEMM for output width n (256x64 tiles when narrow).
int64_t gemm_bn(int64_t n) { return n <= 64 ? 64 : 128; }

}  // namespace

static int sort_routes_checked(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                               int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                               size_t workspace_bytes, void* stream, bool counts_ready);

extern "C" {

const char* cvmm_last_error(void) { return g_err.c_str(); }

int cvmm_abi_version(void) { return 13; }

int cvmm_timing_enable(uint32_t class_mask) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing_mask = class_mask;
  return CVMM_OK;
}

int cvmm_tuning_set(int32_t knob, int64_t value) {
  if (knob == CVMM_TUNE_PANEL_TILES_PER_WG) {
    if (value < 0 || value > 4096) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: tiles per workgroup out of range");
    g_panel_tpw.store((int32_t)value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_GEMM_ORDER) {
    if (value < 0 || value > 2) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: GEMM order must be 0, 1 or 2");
    g_gemm_order.store((int32_t)value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_SORT_CHUNK) {
    if (value < 0 || value > (1 << 24)) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: sort chunk out of range");
    set_sort_chunk(value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_DENSE_TOPK) {
    if (value < 0 || value > 2) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: dense top-k choice must be 0, 1 or 2");
    g_dense_topk.store((int32_t)value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_RING_TILE) {
    if (value < 0 || value > 3) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: long-K tile choice must be 0 to 3");
    g_ring_tile.store((int32_t)value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_WGRAD_ORDER) {
    if (value < 0 || value > 3) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: weight-gradient order must be 0 .. 3");
    g_wgrad_order.store((int32_t)value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_WGRAD_CHUNK) {
    if (value < 0 || value > (1ll << 30)) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: weight-gradient chunk out of range");
    g_wgrad_chunk.store(value);
    return CVMM_OK;
  }
  if (knob == CVMM_TUNE_WGRAD_TILE) {
    if (value < 0 || value > 5) return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: weight-gradient tile must be 0 .. 5");
    g_wgrad_tile.store((int32_t)value);
    return CVMM_OK;
  }
  return fail(CVMM_ERR_INVALID, "cvmm_tuning_set: unknown knob %d", knob);
}

int cvmm_topk_dense(int64_t n_tokens, int32_t n_experts, int64_t K, int64_t N, int64_t top_k, int32_t op_dtype) {
  return use_dense_topk(op_dtype, n_tokens, n_experts, K, N, top_k) ? 1 : 0;
}

int cvmm_timing_result(uint32_t kernel_class, double* total_ms, int64_t* launches) {
  if (!total_ms || !launches) return fail(CVMM_ERR_INVALID, "cvmm_timing_result: NULL output");
  std::vector<TimedLaunch> mine;
  {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    std::vector<TimedLaunch> rest;
    for (const auto& t : g_timed) (t.cls == kernel_class ? mine : rest).push_back(t);
    g_timed.swap(rest);
  }
  double sum = 0.0;
  for (const auto& t : mine) {
    float ms = 0.f;
    if (hipEventSynchronize(t.stop) == hipSuccess && hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess)
      sum += ms;
    hipEventDestroy(t.start);
    hipEventDestroy(t.stop);
  }
  *total_ms = sum;
  *launches = (int64_t)mine.size();
  return CVMM_OK;
}

// ---------------------------------------------------------------------------
size_t cvmm_sort_workspace_bytes(int64_t n_routes, int32_t n_experts) {
  return sort_workspace_bytes(n_routes, n_experts);
}

int cvmm_sort_routes(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts, int64_t top_k,
                     int32_t* sorted_sel, int64_t* perm, int64_t* token_index, int64_t* offsets,
                     int32_t* route_pos, int32_t* n_invalid, void* workspace, size_t workspace_bytes,
                     void* stream) {
  return sort_routes_checked(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index, offsets,
                             route_pos, n_invalid, workspace, workspace_bytes, stream, false);
}

}  // extern "C"

// cvmm_sort_routes; `counts_ready`: the workspace already holds the count
// matrix of these ids for n_experts (cvmm_copy_ids_count).
static int sort_routes_checked(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                               int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                               size_t workspace_bytes, void* stream, bool counts_ready) {
  if (n_experts <= 0) return fail(CVMM_ERR_INVALID, "cvmm_sort_routes: n_experts must be > 0 (got %d)", n_experts);
  if (n_experts > 32767) return fail(CVMM_ERR_UNSUPPORTED, "cvmm_sort_routes: at most 32767 experts (got %d)", n_experts);
  if (n_routes < 0 || n_routes > 0x7fffffffll)
    return fail(CVMM_ERR_INVALID, "cvmm_sort_routes: n_routes out of range (%lld)", (long long)n_routes);
  if (top_k <= 0) return fail(CVMM_ERR_INVALID, "cvmm_sort_routes: top_k must be > 0");
  if (offsets == nullptr) return fail(CVMM_ERR_INVALID, "cvmm_sort_routes: offsets is NULL");
  hipStream_t s = (hipStream_t)stream;
  if (n_routes == 0) {
    if (n_invalid) { int r = check_launch(timed_fill(s, [&] { return launch_fill_zero(n_invalid, 4, s); }), "fill"); if (r) return r; }
    return check_launch(timed_fill(s, [&] { return launch_fill_zero(offsets, (size_t)n_experts * 8, s); }), "cvmm_sort_routes(fill)");
  }
  if (!sel || !sorted_sel || !perm) return fail(CVMM_ERR_INVALID, "cvmm_sort_routes: NULL pointer");
  if (workspace == nullptr || workspace_bytes < sort_workspace_bytes(n_routes, n_experts))
    return fail(CVMM_ERR_WORKSPACE, "cvmm_sort_routes: workspace too small (%zu < %zu)", workspace_bytes,
                sort_workspace_bytes(n_routes, n_experts));
  return check_launch(timed(CVMM_KC_SORT, s, [&] { return launch_sort_routes(sel, sel_is_int64 != 0, n_routes, n_experts, top_k, sorted_sel, perm,
                                         token_index, offsets, route_pos, n_invalid, workspace, s, nullptr,
                                         counts_ready); }),
                      "cvmm_sort_routes");
}

// ---------------------------------------------------------------------------
// cvmm_sort_routes_noalloc: the sort with its histogram scratch in a
// file-scope device array instead of a caller workspace.  The sort's
// workspace is bounded by construction (chunks * (E + 1) counts <= ~96K plus
// E + 1 totals: at most 512 KiB for the 32767 experts the ABI accepts), so
// 1 MiB holds every call.  Each GPU holds its own copy until the process
// ends; its address is looked up once per device (hipGetSymbolAddress) and
// only that address is ever passed to kernels.  Nothing in it needs to start
// at zero: every call writes the histogram before reading it.  Calls that
// overlap on one GPU (different streams) share the array and race.
// ---------------------------------------------------------------------------
constexpr size_t kSortScratchBytes = size_t(1) << 20;
static __device__ __align__(256) uint8_t scratch[kSortScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's copy of `scratch` (looked up on its first use there).
int sort_scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(CVMM_ERR_LAUNCH, "cvmm_sort_routes_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_sort_routes_noalloc: device %d beyond the %d supported", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(CVMM_ERR_LAUNCH, "cvmm_sort_routes_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CVMM_OK;
}
}  // namespace

extern "C" {

int cvmm_sort_routes_noalloc(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                             int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                             int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* stream) {
  if (n_experts <= 0 || n_experts > 32767 || n_routes < 0 || n_routes > 0x7fffffffll || top_k <= 0 ||
      offsets == nullptr)  // cvmm_sort_routes names the bad argument (before any HIP call)
    return cvmm_sort_routes(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index, offsets,
                            route_pos, n_invalid, nullptr, 0, stream);
  const size_t need = sort_workspace_bytes(n_routes, n_experts);
  if (need > kSortScratchBytes)
    return fail(CVMM_ERR_WORKSPACE, "cvmm_sort_routes_noalloc: %lld routes over %d experts need %zu bytes of scratch, "
                "the static scratch holds %zu", (long long)n_routes, n_experts, need, kSortScratchBytes);
  void* ws = nullptr;
  int r = sort_scratch_of_current_device(&ws);
  if (r) return r;
  return cvmm_sort_routes(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index, offsets,
                          route_pos, n_invalid, ws, kSortScratchBytes, stream);
}

int cvmm_copy_ids(const void* sel, int32_t sel_is_int64, int64_t n, int32_t* out, void* stream) {
  if (n < 0) return fail(CVMM_ERR_INVALID, "cvmm_copy_ids: n < 0");
  if (n > 0 && (!sel || !out)) return fail(CVMM_ERR_INVALID, "cvmm_copy_ids: NULL pointer");
  return check_launch(timed(CVMM_KC_SORT, (hipStream_t)stream, [&] {
    return launch_copy_ids(sel, sel_is_int64 != 0, n, out, (hipStream_t)stream);
  }), "cvmm_copy_ids");
}

int cvmm_expert_offsets(const int32_t* sorted_sel, int64_t n_routes, int32_t n_experts, int64_t* offsets,
                        void* stream) {
  if (n_experts <= 0 || offsets == nullptr) return fail(CVMM_ERR_INVALID, "cvmm_expert_offsets: bad arguments");
  if (n_routes > 0 && sorted_sel == nullptr) return fail(CVMM_ERR_INVALID, "cvmm_expert_offsets: sorted_sel NULL");
  return check_launch(timed(CVMM_KC_OFFSETS, (hipStream_t)stream, [&] { return launch_expert_offsets(sorted_sel, n_routes, n_experts, offsets, (hipStream_t)stream); }),
                      "cvmm_expert_offsets");
}

// ---------------------------------------------------------------------------
size_t cvmm_route_topk_workspace_bytes(int64_t n_tokens, int32_t n_experts, int64_t top_k) {
  if (n_tokens < 0 || n_experts <= 0 || top_k <= 0) return 0;
  return route_workspace_bytes(n_tokens, n_experts, top_k);
}

static int route_args_ok(const char* what, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                         int32_t n_experts, int64_t top_k) {
  if (!valid_dtype(logits_dtype)) return fail(CVMM_ERR_INVALID, "%s: invalid logits dtype", what);
  if (n_tokens < 0 || n_experts <= 0 || top_k <= 0 || top_k > n_experts || logits_ld < n_experts)
    return fail(CVMM_ERR_INVALID, "%s: bad sizes (T=%lld, E=%d, k=%lld, ld=%lld)", what, (long long)n_tokens,
                n_experts, (long long)top_k, (long long)logits_ld);
  if (n_experts > kRouteMaxExperts || top_k > kRouteMaxK)
    return fail(CVMM_ERR_UNSUPPORTED, "%s: at most %d experts and top-%lld", what, kRouteMaxExperts,
                (long long)kRouteMaxK);
  if (n_tokens > (int64_t)0x7fffffff / top_k) return fail(CVMM_ERR_UNSUPPORTED, "%s: too many routes", what);
  return CVMM_OK;
}

int cvmm_route_topk(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                    int32_t n_experts, int64_t top_k, int32_t renormalize, float* weights, int64_t* sel,
                    int32_t* sorted_sel, int64_t* perm, int64_t* token_index, int64_t* offsets,
                    int32_t* route_pos, void* workspace, size_t workspace_bytes, void* stream) {
  int r = route_args_ok("cvmm_route_topk", logits_dtype, n_tokens, logits_ld, n_experts, top_k);
  if (r) return r;
  const size_t need = route_workspace_bytes(n_tokens, n_experts, top_k);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CVMM_ERR_WORKSPACE, "cvmm_route_topk: workspace too small (%zu < %zu)", workspace_bytes, need);
  if (n_tokens == 0) return CVMM_OK;
  if (!logits || !weights || !sel || !sorted_sel || !perm || !offsets)
    return fail(CVMM_ERR_INVALID, "cvmm_route_topk: NULL pointer");
  hipStream_t s = (hipStream_t)stream;
  return check_launch(timed(CVMM_KC_ROUTE, s, [&] { return launch_route_topk(logits, logits_dtype, n_tokens, logits_ld, n_experts, top_k,
                                                               renormalize, weights, sel, sorted_sel, perm,
                                                               token_index, offsets, route_pos, workspace, s); }),
                      "cvmm_route_topk");
}

int cvmm_route_topk_backward(const void* logits, int32_t logits_dtype, int64_t n_tokens, int64_t logits_ld,
                             int32_t n_experts, int64_t top_k, int32_t renormalize, const int64_t* sel,
                             const float* grad_weights, void* grad_logits, int64_t grad_ld, void* stream) {
  int r = route_args_ok("cvmm_route_topk_backward", logits_dtype, n_tokens, logits_ld, n_experts, top_k);
  if (r) return r;
  if (grad_ld < n_experts) return fail(CVMM_ERR_INVALID, "cvmm_route_topk_backward: grad row stride too small");
  if (n_tokens == 0) return CVMM_OK;
  if (!logits || !sel || !grad_weights || !grad_logits)
    return fail(CVMM_ERR_INVALID, "cvmm_route_topk_backward: NULL pointer");
  hipStream_t s = (hipStream_t)stream;
  return check_launch(timed(CVMM_KC_ROUTE, s, [&] { return launch_route_topk_backward(logits, logits_dtype, n_tokens, logits_ld, n_experts,
                                                                        top_k, renormalize, sel, grad_weights,
                                                                        grad_logits, grad_ld, s); }),
                      "cvmm_route_topk_backward");
}

// ---------------------------------------------------------------------------
int cvmm_cast_keys(const void* keys, int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out,
                   int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype, void* keys_t, void* keys_n,
                   int32_t layout, void* stream) {
  if (!valid_dtype(keys_dtype) || (out_dtype != kBF16 && out_dtype != kF16))
    return fail(CVMM_ERR_INVALID, "cvmm_cast_keys: keys dtype must be float, output bf16 or f16");
  if (layout & ~(kCastTInterleaved | kCastNInterleaved))
    return fail(CVMM_ERR_INVALID, "cvmm_cast_keys: unknown layout bits %d", layout);
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0) return fail(CVMM_ERR_INVALID, "cvmm_cast_keys: bad sizes");
  if (n_experts > 65535 || (d_in + 63) / 64 > 65535)
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_cast_keys: too many experts / rows");
  if (!keys) return fail(CVMM_ERR_INVALID, "cvmm_cast_keys: keys NULL");
  if (!keys_t && !keys_n) return CVMM_OK;
  return check_launch(timed(CVMM_KC_CAST_KEYS, (hipStream_t)stream, [&] {
                        return launch_cast_keys(keys, keys_dtype, k_se, k_si, k_sj, n_experts, d_in, d_out,
                                                out_dtype, keys_t, keys_n, layout, (hipStream_t)stream);
                      }),
                      "cvmm_cast_keys");
}

int cvmm_sort_routes_cast_keys(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                               int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                               int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                               size_t workspace_bytes, const void* keys, int32_t keys_dtype, int64_t d_in,
                               int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype,
                               void* keys_t, void* keys_n, int32_t layout, void* stream) {
  return cvmm_sort_routes_cast_keys_ex(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index,
                                       offsets, route_pos, n_invalid, workspace, workspace_bytes, keys, keys_dtype,
                                       d_in, d_out, k_se, k_si, k_sj, out_dtype, keys_t, keys_n, layout, 0, stream);
}

}  // extern "C"

// Count matrices cvmm_copy_ids_count has written: a workspace, the ids'
// count and the expert count it counted for, and the sort chunk it used.  A
// sort with CVMM_FLAG_COUNTS_READY trusts the workspace only while a record
// matches its own call and its current chunk (the chunk knob may have changed
// in between); the record is used up, as the sort turns the counts into
// prefixes.  Without a matching record the sort counts again.
namespace {
struct CountedRecord {
  const void* ws;
  int64_t n_routes;
  int32_t n_experts;
  int64_t chunk;
};
std::mutex g_counted_mu;
std::vector<CountedRecord> g_counted;  // the most recent last, at most kCountedKeep
constexpr size_t kCountedKeep = 64;

void counted_record(const void* ws, int64_t n_routes, int32_t n_experts) {
  std::lock_guard<std::mutex> lk(g_counted_mu);
  for (size_t i = 0; i < g_counted.size(); ++i)
    if (g_counted[i].ws == ws) {
      g_counted.erase(g_counted.begin() + (std::ptrdiff_t)i);
      break;
    }
  if (g_counted.size() == kCountedKeep) g_counted.erase(g_counted.begin());
  g_counted.push_back({ws, n_routes, n_experts, sort_chunk_size(n_routes, n_experts)});
}

bool counted_take(const void* ws, int64_t n_routes, int32_t n_experts) {
  std::lock_guard<std::mutex> lk(g_counted_mu);
  for (size_t i = 0; i < g_counted.size(); ++i) {
    const CountedRecord r = g_counted[i];
    if (r.ws != ws) continue;
    g_counted.erase(g_counted.begin() + (std::ptrdiff_t)i);
    return r.n_routes == n_routes && r.n_experts == n_experts && r.chunk == sort_chunk_size(n_routes, n_experts);
  }
  return false;
}
}  // namespace

extern "C" {

int cvmm_copy_ids_count(const void* sel, int32_t sel_is_int64, int64_t n, int32_t n_experts, int32_t* out,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (n_experts <= 0 || n_experts > 32767)
    return fail(CVMM_ERR_INVALID, "cvmm_copy_ids_count: n_experts must be in 1 .. 32767 (got %d)", n_experts);
  if (n < 0 || n > 0x7fffffffll) return fail(CVMM_ERR_INVALID, "cvmm_copy_ids_count: n out of range");
  if (n > 0 && (!sel || !out)) return fail(CVMM_ERR_INVALID, "cvmm_copy_ids_count: NULL pointer");
  if (n > 0 && (workspace == nullptr || workspace_bytes < sort_workspace_bytes(n, n_experts)))
    return fail(CVMM_ERR_WORKSPACE, "cvmm_copy_ids_count: workspace too small (%zu < %zu)", workspace_bytes,
                sort_workspace_bytes(n, n_experts));
  const int r = check_launch(timed(CVMM_KC_SORT, (hipStream_t)stream, [&] {
    return launch_copy_ids_count(sel, sel_is_int64 != 0, n, n_experts, out, workspace, (hipStream_t)stream);
  }), "cvmm_copy_ids_count");
  if (r == 0 && n > 0) counted_record(workspace, n, n_experts);
  return r;
}

int cvmm_sort_routes_cast_keys_ex(const void* sel, int32_t sel_is_int64, int64_t n_routes, int32_t n_experts,
                                  int64_t top_k, int32_t* sorted_sel, int64_t* perm, int64_t* token_index,
                                  int64_t* offsets, int32_t* route_pos, int32_t* n_invalid, void* workspace,
                                  size_t workspace_bytes, const void* keys, int32_t keys_dtype, int64_t d_in,
                                  int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj, int32_t out_dtype,
                                  void* keys_t, void* keys_n, int32_t layout, int32_t flags, void* stream) {
  if (flags & ~CVMM_FLAG_COUNTS_READY)
    return fail(CVMM_ERR_INVALID, "cvmm_sort_routes_cast_keys_ex: unknown flags %d", flags);
  const bool counts_ready =
      (flags & CVMM_FLAG_COUNTS_READY) != 0 && counted_take(workspace, n_routes, n_experts);
  if (!keys || (!keys_t && !keys_n))  // no cast asked for: the sort alone
    return sort_routes_checked(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index,
                               offsets, route_pos, n_invalid, workspace, workspace_bytes, stream, counts_ready);
  const bool fuse = n_routes > 0 && n_routes <= 0x7fffffffll && n_experts > 0 && n_experts <= 32767 && top_k > 0 &&
                    sel && sorted_sel && perm && offsets && keys && (keys_t || keys_n) && d_in > 0 && d_out > 0 &&
                    n_experts <= 65535 && (int64_t)n_experts * (d_in / 64) * (d_out / 64) < 0x7f000000ll &&
                    sort_cast_fusable(n_experts) && !(layout & ~(kCastTInterleaved | kCastNInterleaved)) &&
                    cast_vec_ok(keys, keys_dtype, k_se, k_si, k_sj, d_in, d_out, out_dtype, keys_t, keys_n) &&
                    workspace != nullptr && workspace_bytes >= sort_workspace_bytes(n_routes, n_experts);
  if (!fuse) {
    // separate calls, each with its own argument checks
    int r = sort_routes_checked(sel, sel_is_int64, n_routes, n_experts, top_k, sorted_sel, perm, token_index,
                                offsets, route_pos, n_invalid, workspace, workspace_bytes, stream, counts_ready);
    if (r) return r;
    return cvmm_cast_keys(keys, keys_dtype, n_experts, d_in, d_out, k_se, k_si, k_sj, out_dtype, keys_t, keys_n,
                          layout, stream);
  }
  hipStream_t s = (hipStream_t)stream;
  const CastRequest cr{keys, k_se, k_si, n_experts, d_in, d_out, out_dtype, keys_t, keys_n, layout};
  return check_launch(timed(CVMM_KC_SORT, s, [&] { return launch_sort_routes(sel, sel_is_int64 != 0, n_routes, n_experts, top_k, sorted_sel, perm,
                                         token_index, offsets, route_pos, n_invalid, workspace, s, &cr,
                                         counts_ready); }),
                      "cvmm_sort_routes_cast_keys");
}

// ---------------------------------------------------------------------------
size_t cvmm_fwd_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t out_rows,
                                int32_t out_dtype, int32_t op_dtype, int32_t has_offsets, int32_t weighted,
                                int32_t flags) {
  Carver c(nullptr);
  const int64_t k = weighted && out_rows > 0 ? n_routes / out_rows : 0;
  const bool dense = weighted && !(flags & CVMM_FLAG_ATOMIC_REDUCE) &&
                     use_dense_topk(op_dtype, out_rows, n_experts, d_in, d_out, k);
  if (dense) carve_dense(c, out_rows, n_experts, d_in, d_out, n_routes, op_dtype);
  if (!has_offsets) c.take((size_t)n_experts * 8);
  if (weighted && !dense) {
    if (flags & CVMM_FLAG_ATOMIC_REDUCE) {
      c.take((size_t)out_rows * d_out * 4);
    } else {
      c.take((size_t)n_routes * d_out * dtype_size(out_dtype));
      c.take((size_t)n_routes * 4);
    }
  }
  return c.used;
}

}  // extern "C"

// cvmm_fwd; with pre_act != NULL (unweighted only) the stored values go
// through the GELU: out = gelu(h), pre_act = h.
static int fwd_core(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, const void* keys,
                    int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t k_se, int64_t k_si,
                    int64_t k_sj, const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index,
                    int64_t n_routes, const int64_t* offsets, const int32_t* route_pos, const void* rw,
                    int32_t rw_dtype, int64_t reduce_k, int32_t op_dtype, void* out, int32_t out_dtype,
                    int64_t out_rows, int64_t out_ld, void* pre_act, int32_t flags, void* workspace,
                    size_t workspace_bytes, void* stream, void* scaled_rows = nullptr,
                    int32_t* scaled_written = nullptr) {
  if (scaled_written != nullptr) *scaled_written = 0;
  if (!valid_dtype(x_dtype) || !valid_dtype(keys_dtype) || !valid_dtype(op_dtype) || !valid_dtype(out_dtype) ||
      (rw && !valid_dtype(rw_dtype)))
    return fail(CVMM_ERR_INVALID, "cvmm_fwd: invalid dtype id");
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0 || n_routes < 0)
    return fail(CVMM_ERR_INVALID, "cvmm_fwd: bad sizes (E=%d, d_in=%lld, d_out=%lld, R=%lld)", n_experts,
                (long long)d_in, (long long)d_out, (long long)n_routes);
  if (x_ld < d_in || out_ld < d_out) return fail(CVMM_ERR_INVALID, "cvmm_fwd: row stride smaller than width");
  const bool weighted = rw != nullptr;
  if (weighted && (reduce_k <= 0 || n_routes % reduce_k != 0 || out_rows != n_routes / reduce_k))
    return fail(CVMM_ERR_INVALID, "cvmm_fwd: weighted output needs out_rows = R / reduce_k");
  if (!weighted && out_rows != n_routes) return fail(CVMM_ERR_INVALID, "cvmm_fwd: out_rows must equal R");
  const size_t need = cvmm_fwd_workspace_bytes(n_routes, n_experts, d_in, d_out, out_rows, out_dtype, op_dtype,
                                               offsets != nullptr, weighted, flags);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(CVMM_ERR_WORKSPACE, "cvmm_fwd: workspace too small (%zu < %zu)", workspace_bytes, need);
  if (n_routes == 0) return CVMM_OK;
  if (!x || !keys || !sorted_sel || !sel_index || !out) return fail(CVMM_ERR_INVALID, "cvmm_fwd: NULL pointer");
  if (op_dtype != kF32 && !((x_dtype == kF32 || x_dtype == op_dtype) && (keys_dtype == kF32 || keys_dtype == op_dtype)))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_fwd: x/keys storage must be fp32 or the op dtype");
  if (op_dtype == kF32 && (x_dtype != kF32 || keys_dtype != kF32))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_fwd: fp32 op needs fp32 x and keys");
  hipStream_t s = (hipStream_t)stream;
  Carver c(workspace);
  const bool dense = weighted && !(flags & CVMM_FLAG_ATOMIC_REDUCE) &&
                     use_dense_topk(op_dtype, out_rows, n_experts, d_in, d_out, reduce_k);
  DenseWs dws{};
  if (dense) dws = carve_dense(c, out_rows, n_experts, d_in, d_out, n_routes, op_dtype);
  const int64_t* offs = offsets;
  if (!offs) {
    int64_t* o = (int64_t*)c.take((size_t)n_experts * 8);
    int r = check_launch(timed(CVMM_KC_OFFSETS, s, [&] { return launch_expert_offsets(sorted_sel, n_routes, n_experts, o, s); }), "cvmm_fwd(offsets)");
    if (r) return r;
    offs = o;
  }
  const int64_t* rp = out_index ? out_index : sel_index;

  GemmParams p{};
  p.a = x; p.a_dtype = x_dtype; p.a_ld = x_ld; p.a_rows = x_rows;
  p.a_vec = aligned16(x) && (x_ld * (int64_t)dtype_size(x_dtype)) % 16 == 0;
  p.a_idx = sel_index; p.a_div = 1;
  p.b = keys; p.b_dtype = keys_dtype; p.b_se = k_se; p.b_sk = k_si; p.b_sn = k_sj;
  const int64_t bsz = (int64_t)dtype_size(keys_dtype);
  p.b_vec = aligned16(keys) && (k_se * bsz) % 16 == 0 &&
            ((k_sj == 1 && (k_si * bsz) % 16 == 0) || (k_sj != 1 && k_si == 1 && (k_sj * bsz) % 16 == 0));
  p.K = d_in; p.N = d_out;
  p.offsets = offs; p.n_experts = n_experts; p.n_routes = n_routes;
  const int64_t bm = routed_gemm_bm(d_out);
  p.grid_tiles = (n_routes + bm - 1) / bm + (n_experts < n_routes ? n_experts : n_routes);
  p.o_idx = rp; p.o_div = 1;
  p.val_dtype = out_dtype;
  p.prod_dtype = -1;
  p.w_idx = rp;
  p.panel_tpw = g_panel_tpw.load();
  p.ring_tile = g_ring_tile.load();
  p.token_major = gemm_token_major(n_experts);

  if (!weighted) {
    // rows of routes with an expert id outside [0, E): zeroed by the GEMM's
    // workgroups past its last m-tile
    p.zero_unrouted = 1;
    p.epi = kEpiStore; p.out = out; p.out_dtype = out_dtype; p.out_ld = out_ld; p.out_rows = out_rows;
    if (pre_act != nullptr) {
      p.act = 1; p.aux = pre_act;
      if (!(nt_eligible(p, op_dtype) && routed_gemm_ring_applies(p, op_dtype))) {
        // not the ring kernel: the products to pre_act, then a GELU pass
        p.act = 0; p.aux = nullptr; p.out = pre_act;
        int r = check_launch(timed(CVMM_KC_GEMM_FWD, s, [&] { return launch_routed_gemm(p, op_dtype, s); }), "cvmm_fwd(gemm)");
        if (r) return r;
        return check_launch(timed_combine(s, [&] { return launch_gelu_rows(pre_act, out_dtype, out_ld, out_rows, d_out, out, out_dtype, out_ld, s); }),
                            "cvmm_fwd_gelu(gelu)");
      }
    }
    return check_launch(timed(CVMM_KC_GEMM_FWD, s, [&] { return launch_routed_gemm(p, op_dtype, s); }), "cvmm_fwd(gemm)");
  }
  if (dense) {
    // high fan-out: one GEMM over expert slots of the x rows (scaled by
    // rnd_out(w)), no route buffer.  Route input with out == op dtype: the
    // scaled rows are those the weight gradient scales, kept when asked for.
    const bool keep = scaled_rows != nullptr && scaled_written != nullptr && out_index == nullptr &&
                      x_rows == n_routes && out_dtype == op_dtype && (op_dtype == kBF16 || op_dtype == kF16);
    const int r = run_dense_topk(dws, x, x_dtype, x_ld, out_index == nullptr, sorted_sel, route_pos, rp, offs,
                                 n_routes, out_rows, reduce_k, n_experts, keys, keys_dtype, d_in, d_out, k_se, k_si,
                                 k_sj, true, rw, rw_dtype, out_dtype, op_dtype, out, out_dtype, out_ld,
                                 CVMM_KC_GEMM_FWD, "cvmm_fwd(dense)", s, keep ? scaled_rows : nullptr);
    if (r == 0 && keep) *scaled_written = 1;
    return r;
  }
  if (flags & CVMM_FLAG_ATOMIC_REDUCE) {
    // fused combine: y rounded to the output dtype, times rnd_out(w), fp32 atomics per token row
    float* acc = (float*)c.take((size_t)out_rows * d_out * 4);
    int r = check_launch(timed_fill(s, [&] { return launch_fill_zero(acc, (size_t)out_rows * d_out * 4, s); }), "cvmm_fwd(zero)");
    if (r) return r;
    p.epi = kEpiAtomic; p.out = acc; p.out_dtype = kF32; p.out_ld = d_out; p.out_rows = out_rows;
    p.o_div = reduce_k;
    p.w = rw; p.w_dtype = rw_dtype; p.w_round = out_dtype;
    r = check_launch(timed(CVMM_KC_GEMM_FWD, s, [&] { return launch_routed_gemm(p, op_dtype, s); }), "cvmm_fwd(gemm)");
    if (r) return r;
    return check_launch(timed_combine(s, [&] { return launch_cast_rows(acc, d_out, out_rows, d_out, -1, out, out_dtype, out_ld, s); }),
                        "cvmm_fwd(cast)");
  }
  // y in the output dtype, row q = sorted route q (contiguous rows per expert
  // tile), then the per-token combine in route order through the inverse
  void* ybuf = c.take((size_t)n_routes * d_out * dtype_size(out_dtype));
  int32_t* inv_ws = (int32_t*)c.take((size_t)n_routes * 4);
  const int32_t* inv = route_pos;
  int r = 0;
  if (!inv) {
    r = check_launch(timed_combine(s, [&] { return launch_invert_rows(rp, n_routes, inv_ws, s); }), "cvmm_fwd(invert)");
    if (r) return r;
    inv = inv_ws;
  }
  p.epi = kEpiStore; p.out = ybuf; p.out_dtype = out_dtype; p.out_ld = d_out; p.out_rows = n_routes;
  p.o_idx = nullptr;
  // route input kept for the weight gradient: the small-K kernel writes the
  // scaled rows from its activation fragments (the rows cvmm_bwd_w scales)
  const bool keep = scaled_rows != nullptr && scaled_written != nullptr && out_index == nullptr &&
                    x_rows == n_routes && out_dtype == op_dtype && (op_dtype == kBF16 || op_dtype == kF16) &&
                    routed_gemm_is_panel(p, op_dtype);
  if (keep) {
    p.xs_out = scaled_rows;
    p.xs_w = rw;
    p.xs_w_dtype = rw_dtype;
  }
  r = check_launch(timed(CVMM_KC_GEMM_FWD, s, [&] { return launch_routed_gemm(p, op_dtype, s); }), "cvmm_fwd(gemm)");
  if (r) return r;
  if (keep) *scaled_written = 1;
  return check_launch(timed_combine(s, [&] { return launch_combine_rows(ybuf, out_dtype, d_out, inv, rp, offs + (n_experts - 1), rw, rw_dtype, out_dtype, out_rows, reduce_k, d_out,
                                          out_dtype, out, out_dtype, out_ld, s); }),
                      "cvmm_fwd(combine)");
}


extern "C" {

int cvmm_fwd(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, const void* keys, int32_t keys_dtype,
             int32_t n_experts, int64_t d_in, int64_t d_out, int64_t k_se, int64_t k_si, int64_t k_sj,
             const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
             const int64_t* offsets, const int32_t* route_pos, const void* rw, int32_t rw_dtype, int64_t reduce_k,
             int32_t op_dtype,
             void* out, int32_t out_dtype, int64_t out_rows, int64_t out_ld, int32_t flags, void* workspace,
             size_t workspace_bytes, void* stream) {
  return fwd_core(x, x_dtype, x_rows, x_ld, keys, keys_dtype, n_experts, d_in, d_out, k_se, k_si, k_sj, sorted_sel,
                  sel_index, out_index, n_routes, offsets, route_pos, rw, rw_dtype, reduce_k, op_dtype, out,
                  out_dtype, out_rows, out_ld, nullptr, flags, workspace, workspace_bytes, stream);
}

int cvmm_fwd_keep_scaled(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, const void* keys,
                         int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t k_se,
                         int64_t k_si, int64_t k_sj, const int32_t* sorted_sel, const int64_t* sel_index,
                         const int64_t* out_index, int64_t n_routes, const int64_t* offsets,
                         const int32_t* route_pos, const void* rw, int32_t rw_dtype, int64_t reduce_k,
                         int32_t op_dtype, void* out, int32_t out_dtype, int64_t out_rows, int64_t out_ld,
                         void* scaled_rows, int32_t* scaled_written, int32_t flags, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (scaled_written == nullptr) return fail(CVMM_ERR_INVALID, "cvmm_fwd_keep_scaled: scaled_written NULL");
  return fwd_core(x, x_dtype, x_rows, x_ld, keys, keys_dtype, n_experts, d_in, d_out, k_se, k_si, k_sj, sorted_sel,
                  sel_index, out_index, n_routes, offsets, route_pos, rw, rw_dtype, reduce_k, op_dtype, out,
                  out_dtype, out_rows, out_ld, nullptr, flags, workspace, workspace_bytes, stream, scaled_rows,
                  scaled_written);
}

int cvmm_fwd_gelu(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, const void* keys,
                  int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t k_se, int64_t k_si,
                  int64_t k_sj, const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index,
                  int64_t n_routes, const int64_t* offsets, const int32_t* route_pos, int32_t op_dtype, void* out,
                  int32_t out_dtype, int64_t out_rows, int64_t out_ld, void* pre_act, int32_t flags,
                  void* workspace, size_t workspace_bytes, void* stream) {
  if (pre_act == nullptr && n_routes > 0) return fail(CVMM_ERR_INVALID, "cvmm_fwd_gelu: pre_act NULL");
  return fwd_core(x, x_dtype, x_rows, x_ld, keys, keys_dtype, n_experts, d_in, d_out, k_se, k_si, k_sj, sorted_sel,
                  sel_index, out_index, n_routes, offsets, route_pos, nullptr, 0, 1, op_dtype, out, out_dtype,
                  out_rows, out_ld, pre_act, flags, workspace, workspace_bytes, stream);
}

int cvmm_gelu_backward(const void* grad, int32_t grad_dtype, int64_t grad_ld, const void* pre_act,
                       int32_t pre_dtype, int64_t pre_ld, int64_t rows, int64_t cols, void* grad_pre,
                       int32_t grad_pre_dtype, int64_t grad_pre_ld, void* stream) {
  if (!valid_dtype(grad_dtype) || !valid_dtype(pre_dtype) || !valid_dtype(grad_pre_dtype))
    return fail(CVMM_ERR_INVALID, "cvmm_gelu_backward: invalid dtype id");
  if (rows < 0 || cols < 0 || grad_ld < cols || pre_ld < cols || grad_pre_ld < cols)
    return fail(CVMM_ERR_INVALID, "cvmm_gelu_backward: bad sizes");
  if (rows == 0 || cols == 0) return CVMM_OK;
  if (!grad || !pre_act || !grad_pre) return fail(CVMM_ERR_INVALID, "cvmm_gelu_backward: NULL pointer");
  hipStream_t s = (hipStream_t)stream;
  return check_launch(timed_combine(s, [&] { return launch_gelu_backward(grad, grad_dtype, grad_ld, pre_act, pre_dtype, pre_ld, rows, cols,
                                                            grad_pre, grad_pre_dtype, grad_pre_ld, s); }),
                      "cvmm_gelu_backward");
}

// ---------------------------------------------------------------------------
size_t cvmm_bwd_x_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                  int64_t grad_x_rows, int32_t has_offsets, int32_t weighted, int32_t token_input,
                                  int64_t top_k, int32_t grad_x_dtype, int32_t op_dtype, int32_t need_grad_rw,
                                  int32_t flags) {
  Carver c(nullptr);
  const bool reduce = reduce_needed(weighted, token_input, top_k) ||
                      ((flags & CVMM_FLAG_ACCUMULATE) && token_input && !weighted);
  const bool dense = reduce && !weighted && !(flags & (CVMM_FLAG_ATOMIC_REDUCE | CVMM_FLAG_ACCUMULATE)) &&
                     use_dense_topk(op_dtype, grad_x_rows, n_experts, d_out, d_in, top_k);
  if (dense) carve_dense(c, grad_x_rows, n_experts, d_out, d_in, n_routes, op_dtype);
  if (!has_offsets) c.take((size_t)n_experts * 8);
  if (reduce && !dense) {
    if (flags & CVMM_FLAG_ATOMIC_REDUCE) {
      c.take((size_t)grad_x_rows * d_in * 4);
    } else {
      c.take((size_t)n_routes * d_in * dtype_size(weighted ? op_dtype : grad_x_dtype));
      c.take((size_t)n_routes * 4);
    }
  }
  if (weighted && need_grad_rw) c.take((size_t)n_routes * ntiles_of(d_in, gemm_bn(d_in)) * 4);
  return c.used;
}

int cvmm_bwd_x(const void* grad, int32_t grad_dtype, int64_t grad_rows, int64_t grad_ld, const void* keys,
               int32_t keys_dtype, int32_t n_experts, int64_t d_in, int64_t d_out, int64_t k_se, int64_t k_si,
               int64_t k_sj, const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index,
               int64_t n_routes, const int64_t* offsets, const int32_t* route_pos, const void* rw, int32_t rw_dtype,
               int64_t top_k,
               const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, int32_t op_dtype, void* grad_x,
               int32_t grad_x_dtype, int64_t grad_x_rows, int64_t grad_x_ld, void* grad_rw, int32_t grad_rw_dtype,
               int32_t flags, void* workspace, size_t workspace_bytes, void* stream) {
  const bool weighted = rw != nullptr;
  const bool token_input = out_index != nullptr;
  if (!valid_dtype(grad_dtype) || !valid_dtype(keys_dtype) || !valid_dtype(op_dtype) ||
      (grad_x && !valid_dtype(grad_x_dtype)) || (weighted && !valid_dtype(rw_dtype)) ||
      (grad_rw && !valid_dtype(grad_rw_dtype)) || (x && !valid_dtype(x_dtype)))
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: invalid dtype id");
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0 || n_routes < 0 || top_k <= 0)
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: bad sizes");
  if (grad_ld < d_out || (grad_x && grad_x_ld < d_in)) return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: bad row stride");
  if (grad_rw && !weighted) return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: grad_rw needs reduction_weight");
  if (grad_rw && (!x || x_ld < d_in)) return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: grad_rw needs x");
  if (weighted && n_routes % top_k != 0) return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: R not a multiple of top_k");
  // CVMM_FLAG_ACCUMULATE: grad_x is an fp32 running sum; the route rows are
  // rounded to x_dtype, the dtype the final gradient will be stored in (a
  // slice of one top-k column still adds its rows to the sum)
  const bool accumulate = (flags & CVMM_FLAG_ACCUMULATE) != 0;
  const bool reduce = reduce_needed(weighted, token_input, top_k) || (accumulate && token_input && !weighted);
  if (accumulate && !(reduce && !weighted && grad_x && grad_x_dtype == kF32 && !(flags & CVMM_FLAG_ATOMIC_REDUCE) &&
                      (x_dtype == kBF16 || x_dtype == kF16) && d_in % 8 == 0 && top_k <= 64))
    return fail(CVMM_ERR_UNSUPPORTED,
                "cvmm_bwd_x: CVMM_FLAG_ACCUMULATE takes a token-input unweighted top-k sum (top_k <= 64, d_in %% 8 "
                "== 0) into fp32 grad_x, with x_dtype bf16 or f16 the dtype of its rows");
  if (grad_x) {
    const int64_t want = reduce ? n_routes / top_k : n_routes;
    if (grad_x_rows != want)
      return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: grad_x has %lld rows, expected %lld", (long long)grad_x_rows,
                  (long long)want);
  }
  const size_t need = cvmm_bwd_x_workspace_bytes(n_routes, n_experts, d_in, d_out, grad_x_rows, offsets != nullptr,
                                                 weighted, token_input, top_k, accumulate ? x_dtype : grad_x_dtype,
                                                 op_dtype, grad_rw != nullptr, flags);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(CVMM_ERR_WORKSPACE, "cvmm_bwd_x: workspace too small (%zu < %zu)", workspace_bytes, need);
  if (n_routes == 0 || (!grad_x && !grad_rw)) return CVMM_OK;
  if (!grad || !keys || !sorted_sel || !sel_index) return fail(CVMM_ERR_INVALID, "cvmm_bwd_x: NULL pointer");
  if (op_dtype != kF32 && !((grad_dtype == kF32 || grad_dtype == op_dtype) && (keys_dtype == kF32 || keys_dtype == op_dtype)))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_bwd_x: grad/keys storage must be fp32 or the op dtype");
  if (op_dtype == kF32 && (grad_dtype != kF32 || keys_dtype != kF32))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_bwd_x: fp32 op needs fp32 grad and keys");

  hipStream_t s = (hipStream_t)stream;
  Carver c(workspace);
  const bool dense = reduce && !weighted && !(flags & (CVMM_FLAG_ATOMIC_REDUCE | CVMM_FLAG_ACCUMULATE)) &&
                     use_dense_topk(op_dtype, grad_x_rows, n_experts, d_out, d_in, top_k);
  DenseWs dws{};
  if (dense) dws = carve_dense(c, grad_x_rows, n_experts, d_out, d_in, n_routes, op_dtype);
  const int64_t* offs = offsets;
  if (!offs) {
    int64_t* o = (int64_t*)c.take((size_t)n_experts * 8);
    int r = check_launch(timed(CVMM_KC_OFFSETS, s, [&] { return launch_expert_offsets(sorted_sel, n_routes, n_experts, o, s); }), "cvmm_bwd_x(offsets)");
    if (r) return r;
    offs = o;
  }
  const int64_t* rp = token_input ? out_index : sel_index;

  if (dense && grad_x) {
    // high fan-out: one GEMM over expert slots of the dY rows, no route buffer
    return run_dense_topk(dws, grad, grad_dtype, grad_ld, true, sorted_sel, route_pos, rp, offs, n_routes,
                          grad_x_rows, top_k, n_experts, keys, keys_dtype, d_in, d_out, k_se, k_si, k_sj, false,
                          nullptr, 0, 0, op_dtype, grad_x, grad_x_dtype, grad_x_ld, CVMM_KC_GEMM_BWDX,
                          "cvmm_bwd_x(dense)", s);
  }

  // grad @ keys[e]^T: K = d_out, N = d_in, B[k][n] = keys[e][n][k]
  GemmParams p{};
  p.a = grad; p.a_dtype = grad_dtype; p.a_ld = grad_ld; p.a_rows = grad_rows;
  p.a_vec = aligned16(grad) && (grad_ld * (int64_t)dtype_size(grad_dtype)) % 16 == 0;
  p.a_idx = rp; p.a_div = weighted ? top_k : 1;
  p.b = keys; p.b_dtype = keys_dtype; p.b_se = k_se; p.b_sk = k_sj; p.b_sn = k_si;
  const int64_t bsz = (int64_t)dtype_size(keys_dtype);
  p.b_vec = aligned16(keys) && (k_se * bsz) % 16 == 0 &&
            ((k_si == 1 && (k_sj * bsz) % 16 == 0) || (k_si != 1 && k_sj == 1 && (k_si * bsz) % 16 == 0));
  p.K = d_out; p.N = d_in;
  p.offsets = offs; p.n_experts = n_experts; p.n_routes = n_routes;
  const int64_t bm = routed_gemm_bm(d_in);
  p.grid_tiles = (n_routes + bm - 1) / bm + (n_experts < n_routes ? n_experts : n_routes);
  p.o_idx = rp; p.o_div = 1;
  p.w_idx = rp;
  p.prod_dtype = -1;
  p.role = 1;
  p.panel_tpw = g_panel_tpw.load();
  p.ring_tile = g_ring_tile.load();
  p.token_major = gemm_token_major(n_experts);

  void* route_buf = nullptr;
  const int32_t* inv = nullptr;
  float* acc = nullptr;
  if (grad_x) {
    if (!reduce) {
      p.epi = kEpiStore; p.out = grad_x; p.out_dtype = grad_x_dtype; p.out_ld = grad_x_ld; p.out_rows = grad_x_rows;
      p.zero_unrouted = 1;  // per-route rows of out-of-range expert ids: zero
      if (weighted) {  // route-major weighted: rnd_op(rnd_op(g) * rnd_op(w))
        p.val_dtype = op_dtype; p.w = rw; p.w_dtype = rw_dtype; p.w_round = op_dtype; p.prod_dtype = op_dtype;
      } else {
        p.val_dtype = grad_x_dtype;
      }
    } else if (flags & CVMM_FLAG_ATOMIC_REDUCE) {
      acc = (float*)c.take((size_t)grad_x_rows * d_in * 4);
      int r = check_launch(timed_fill(s, [&] { return launch_fill_zero(acc, (size_t)grad_x_rows * d_in * 4, s); }), "cvmm_bwd_x(zero)");
      if (r) return r;
      p.epi = kEpiAtomic; p.out = acc; p.out_dtype = kF32; p.out_ld = d_in; p.out_rows = grad_x_rows;
      p.o_div = top_k;
      if (weighted) { p.val_dtype = op_dtype; p.w = rw; p.w_dtype = rw_dtype; p.w_round = op_dtype; }
      else p.val_dtype = grad_x_dtype;
    } else {
      // row q = sorted route q; the combine gathers each token's routes
      const int32_t bdt = weighted ? op_dtype : accumulate ? x_dtype : grad_x_dtype;
      route_buf = c.take((size_t)n_routes * d_in * dtype_size(bdt));
      int32_t* inv_ws = (int32_t*)c.take((size_t)n_routes * 4);
      inv = route_pos;
      if (!inv) {
        int r = check_launch(timed_combine(s, [&] { return launch_invert_rows(rp, n_routes, inv_ws, s); }),
                             "cvmm_bwd_x(invert)");
        if (r) return r;
        inv = inv_ws;
      }
      p.epi = kEpiStore; p.out = route_buf; p.out_dtype = bdt; p.out_ld = d_in; p.out_rows = n_routes;
      p.o_idx = nullptr;
      p.val_dtype = bdt;
    }
  } else {
    p.epi = kEpiStore; p.out = nullptr;
  }

  float* dg_part = nullptr;
  bool dg_direct = false;
  const int64_t dg_nt = ntiles_of(d_in, gemm_bn(d_in));
  if (weighted && grad_rw) {
    // no fill: the GEMM writes every (route, n tile) partial -- covered
    // routes from their tile's epilogue, out-of-range expert ids as zeros
    // from the workgroups past the last m-tile.  One n tile and an fp32
    // gradient: the partial is the gradient, written in place.
    dg_part = (float*)c.take((size_t)n_routes * dg_nt * 4);
    dg_direct = dg_nt == 1 && grad_rw_dtype == kF32;
    p.dg = dg_direct ? (float*)grad_rw : dg_part; p.dg_ntiles = (int32_t)dg_nt;
    p.dg_x = x; p.dg_x_dtype = x_dtype; p.dg_x_ld = x_ld; p.dg_x_rows = x_rows; p.dg_x_idx = sel_index;
    p.dg_val_dtype = op_dtype;
  }

  int r = check_launch(timed(CVMM_KC_GEMM_BWDX, s, [&] { return launch_routed_gemm(p, op_dtype, s); }), "cvmm_bwd_x(gemm)");
  if (r) return r;
  if (grad_x && reduce) {
    if (acc) {
      r = check_launch(timed_combine(s, [&] { return launch_cast_rows(acc, d_in, grad_x_rows, d_in, weighted ? op_dtype : -1, grad_x,
                                        grad_x_dtype, grad_x_ld, s); }),
                       "cvmm_bwd_x(cast)");
    } else {
      const int32_t bdt = weighted ? op_dtype : accumulate ? x_dtype : grad_x_dtype;
      r = check_launch(timed_combine(s, [&] { return launch_combine_rows(route_buf, bdt, d_in, inv, rp, offs + (n_experts - 1), weighted ? rw : nullptr, rw_dtype, op_dtype,
                                           grad_x_rows, top_k, d_in, weighted ? op_dtype : -1, grad_x, grad_x_dtype,
                                           grad_x_ld, s, accumulate); }),
                       "cvmm_bwd_x(combine)");
    }
    if (r) return r;
  }
  if (dg_part && !dg_direct) {
    r = check_launch(timed_combine(s, [&] { return launch_sum_partials(dg_part, n_routes, (int32_t)dg_nt, grad_rw, grad_rw_dtype, s); }),
                     "cvmm_bwd_x(dgate)");
    if (r) return r;
  }
  return CVMM_OK;
}

// ---------------------------------------------------------------------------
size_t cvmm_bwd_w_counter_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                int32_t op_dtype) {
  int64_t split, grid_chunks, max_slots, tiles;
  wgrad_geometry(d_in, d_out, n_routes, n_experts, op_dtype, &split, &grid_chunks, &max_slots, &tiles);
  Carver c(nullptr);
  c.take((size_t)n_experts * tiles * 4);
  return c.used;
}

}  // extern "C"

// The weight gradient of a weighted route-input selection scales the route
// rows beforehand (16-bit op, rows of whole 16-byte pieces).
static bool wgrad_scales_rows(int32_t op_dtype, int64_t d_in) {
  return (op_dtype == kBF16 || op_dtype == kF16) && d_in % 8 == 0;
}

extern "C" {

size_t cvmm_bwd_w_workspace_bytes(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                  int32_t op_dtype, int32_t has_offsets) {
  int64_t split, grid_chunks, max_slots, tiles;
  wgrad_geometry(d_in, d_out, n_routes, n_experts, op_dtype, &split, &grid_chunks, &max_slots, &tiles);
  Carver c(nullptr);
  c.take((size_t)n_experts * tiles * 4);  // counters first: see CVMM_FLAG_COUNTERS_ZEROED
  if (!has_offsets) c.take((size_t)n_experts * 8);
  c.take((size_t)max_slots * wgrad_partial_elems(d_in, d_out) * 4);
  return c.used;
}

size_t cvmm_bwd_w_workspace_bytes_ex(int64_t n_routes, int32_t n_experts, int64_t d_in, int64_t d_out,
                                     int32_t op_dtype, int32_t has_offsets, int32_t weighted_route_input) {
  size_t need = cvmm_bwd_w_workspace_bytes(n_routes, n_experts, d_in, d_out, op_dtype, has_offsets);
  if (weighted_route_input && wgrad_scales_rows(op_dtype, d_in))
    need = align_up(need, 256) + (size_t)n_routes * d_in * dtype_size(op_dtype);
  return need;
}

int cvmm_bwd_w(const void* x, int32_t x_dtype, int64_t x_rows, int64_t x_ld, const void* grad, int32_t grad_dtype,
               int64_t grad_rows, int64_t grad_ld, int32_t n_experts, int64_t d_in, int64_t d_out,
               const int32_t* sorted_sel, const int64_t* sel_index, const int64_t* out_index, int64_t n_routes,
               const int64_t* offsets, const void* rw, int32_t rw_dtype, int64_t top_k, int32_t op_dtype,
               void* grad_keys, int32_t grad_keys_dtype, int64_t gk_se, int64_t gk_si, int64_t gk_sj, int32_t flags,
               void* workspace, size_t workspace_bytes, void* stream) {
  const bool weighted = rw != nullptr;
  if (!valid_dtype(x_dtype) || !valid_dtype(grad_dtype) || !valid_dtype(op_dtype) || !valid_dtype(grad_keys_dtype) ||
      (weighted && !valid_dtype(rw_dtype)))
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: invalid dtype id");
  if (n_experts <= 0 || d_in <= 0 || d_out <= 0 || n_routes < 0 || top_k <= 0)
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: bad sizes");
  if (x_ld < d_in || grad_ld < d_out) return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: bad row stride");
  if (!grad_keys) return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: grad_keys NULL");
  const size_t need = cvmm_bwd_w_workspace_bytes(n_routes, n_experts, d_in, d_out, op_dtype, offsets != nullptr);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CVMM_ERR_WORKSPACE, "cvmm_bwd_w: workspace too small (%zu < %zu)", workspace_bytes, need);
  if (n_routes > 0 && (!x || !grad || !sorted_sel || !sel_index))
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: NULL pointer");
  if (op_dtype != kF32 && !((x_dtype == kF32 || x_dtype == op_dtype) && (grad_dtype == kF32 || grad_dtype == op_dtype)))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_bwd_w: x/grad storage must be fp32 or the op dtype");
  if (op_dtype == kF32 && (x_dtype != kF32 || grad_dtype != kF32))
    return fail(CVMM_ERR_UNSUPPORTED, "cvmm_bwd_w: fp32 op needs fp32 x and grad");
  // x already scaled by the routes' weights (the rows cvmm_fwd_keep_scaled
  // kept): a weighted selection with route input, rows in the 16-bit op dtype
  const bool rows_scaled = (flags & CVMM_FLAG_ROWS_SCALED) != 0;
  if (rows_scaled && !(weighted && out_index == nullptr && x_dtype == op_dtype &&
                       (op_dtype == kBF16 || op_dtype == kF16) && x_rows == n_routes))
    return fail(CVMM_ERR_INVALID, "cvmm_bwd_w: CVMM_FLAG_ROWS_SCALED needs a weighted selection with route input "
                                  "and x in the 16-bit op dtype, one row per route");

  hipStream_t s = (hipStream_t)stream;
  WgradParams p{};
  int64_t tiles;
  wgrad_geometry(d_in, d_out, n_routes, n_experts, op_dtype, &p.split, &p.grid_chunks, &p.max_slots, &tiles);
  Carver c(workspace);
  // The kernel's last arriver on each tile resets its counter, so the region
  // is zero again when the kernel ends; callers that keep the workspace can
  // pass CVMM_FLAG_COUNTERS_ZEROED and skip the fill.
  p.counters = (int32_t*)c.take((size_t)n_experts * tiles * 4);
  if (!(flags & CVMM_FLAG_COUNTERS_ZEROED)) {
    int r = check_launch(timed_fill(s, [&] { return launch_fill_zero(p.counters, (size_t)n_experts * tiles * 4, s); }),
                         "cvmm_bwd_w(zero)");
    if (r) return r;
  }
  const int64_t* offs = offsets;
  if (!offs) {
    int64_t* o = (int64_t*)c.take((size_t)n_experts * 8);
    int r = n_routes > 0 ? check_launch(timed(CVMM_KC_OFFSETS, s, [&] { return launch_expert_offsets(sorted_sel, n_routes, n_experts, o, s); }), "offsets")
                         : check_launch(timed_fill(s, [&] { return launch_fill_zero(o, (size_t)n_experts * 8, s); }), "offsets");
    if (r) return r;
    offs = o;
  }
  p.partial = (float*)c.take((size_t)p.max_slots * wgrad_partial_elems(d_in, d_out) * 4);

  const int64_t* rp = out_index ? out_index : sel_index;
  // A weighted selection with route input (x row = route) whose workspace
  // holds the rows: x scaled by its routes' weights once, rnd_op(rnd_op(w_r)
  // * rnd_op(x_r)), then the unweighted kernel with the token's gradient row
  // (the weight moves from the d_out-wide gradient slices of every dW tile to
  // one pass over the d_in-wide route rows).
  const size_t rows_bytes = (size_t)x_rows * d_in * dtype_size(op_dtype);
  const bool scale_rows = !rows_scaled && weighted && out_index == nullptr && x_rows <= n_routes && n_routes > 0 &&
                          wgrad_scales_rows(op_dtype, d_in) && align_up(c.used, 256) + rows_bytes <= workspace_bytes;
  if (rows_scaled) {
    rw = nullptr;  // (the selection stays weighted: one gradient row per token)
  } else if (scale_rows) {
    void* xs = c.take(rows_bytes);
    // timed with the row work (combine class): the weight-gradient class
    // times the GEMM alone, one launch per call
    int r = check_launch(timed_combine(s, [&] {
      return launch_scale_rows(x, x_dtype, x_ld, true, rw, rw_dtype, op_dtype, x_rows, top_k, d_in, op_dtype, xs,
                               s);
    }), "cvmm_bwd_w(scale)");
    if (r) return r;
    x = xs;
    x_dtype = op_dtype;
    x_ld = d_in;
    rw = nullptr;
  }
  p.x = x; p.x_dtype = x_dtype; p.x_ld = x_ld; p.x_rows = x_rows;
  p.x_vec = aligned16(x) && (x_ld * (int64_t)dtype_size(x_dtype)) % 16 == 0;
  p.x_idx = sel_index;
  p.g = grad; p.g_dtype = grad_dtype; p.g_ld = grad_ld; p.g_rows = grad_rows;
  p.g_vec = aligned16(grad) && (grad_ld * (int64_t)dtype_size(grad_dtype)) % 16 == 0;
  p.g_idx = rp; p.g_div = weighted ? top_k : 1;
  p.g_fdiv = make_fast_div(p.g_div);
  p.w = rw; p.w_dtype = rw_dtype; p.w_idx = rp;
  p.M = d_in; p.N = d_out;
  p.offsets = offs; p.n_experts = n_experts; p.n_routes = n_routes;
  p.dw = grad_keys; p.dw_dtype = grad_keys_dtype; p.dw_se = gk_se; p.dw_sm = gk_si; p.dw_sn = gk_sj;
  // dW tile: the knob, else 256 x 256 where both sides fill it and the grid
  // still holds >= 4 workgroups per CU (the FFN stack's 2048 x 512: 1.6 -> 0.8 ms per
  // launch; the gathered bytes per flop halve against 128 x 128)
  const int32_t tile = g_wgrad_tile.load();
  p.tile_choice = tile > 0 ? tile - 1 : wgrad_auto_tile(d_in, d_out, p.grid_chunks);
  // Workgroup order: the knob, else chunk-xcd for the 16-bit kernel's 128 x
  // 128 tile (ff_up 38.5 -> 35.0 us, ff_down 52.9 -> 50.8 us per launch: the
  // eight dW tiles of a chunk share its routes' gradient rows in one L2) and
  // tile-major for the other tiles (the activation column slice of one tile,
  // shared by the top-k experts of each token, stays in one XCD's L2:
  // switch_v 223 us against 249 with chunk-xcd, the FFN stack 4.49 against
  // 4.55 ms).  Every order gives the same bits.
  const int32_t order = g_wgrad_order.load();
  if (order == 0) {
    int bm, bn;
    wgrad_fast_tile(d_in, d_out, p.tile_choice, &bm, &bn);
    p.order = wgrad_fast_eligible(p, op_dtype) && bm == 128 && bn == 128 ? kWgOrderChunkXcd : kWgOrderTile;
  } else {
    p.order = order == 1 ? kWgOrderChunk : order == 3 ? kWgOrderChunkXcd : kWgOrderTile;
  }
  return check_launch(timed(CVMM_KC_WGRAD, s, [&] { return launch_wgrad(p, op_dtype, s); }), "cvmm_bwd_w(gemm)");
}

}  // extern "C"
