// Host glue between the Python API (cvmm_codex_amd/api.py) and the C ABI of
// libcvmm_hip.so (include/cvmm_hip.h): output allocation, the storage and
// layout rules for each operand, workspace sizing and the ABI calls.  One call
// per phase replaces a few dozen Python-level tensor operations, which at the
// sizes of an MoE projection cost as much host time as the kernels take on the
// GPU.  Streams come from Python (the raw handle of torch's current stream);
// every call here is asynchronous.
//
// Mirrors the reference's per-phase host logic: cvmm_prepare_sel2's sort
// (cvmm.py:1796-1803), cvmm_triton (cvmm.py:814-867) with the weighted combine
// (cvmm.py:1543-1545), and CVMM.backward's products (cvmm.py:1552-1755).
#include <torch/extension.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <optional>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "cvmm_hip.h"

namespace py = pybind11;

namespace {

using at::Tensor;
using OptT = std::optional<Tensor>;

int32_t dtype_id(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return 0;
    case at::kHalf: return 1;
    case at::kBFloat16: return 2;
    default: throw py::type_error(std::string("cvmm: unsupported dtype ") + c10::toString(t));
  }
}

at::ScalarType dtype_of(int64_t id) {
  switch (id) {
    case 0: return at::kFloat;
    case 1: return at::kHalf;
    case 2: return at::kBFloat16;
    default: throw py::value_error("cvmm: bad dtype id");
  }
}

void check(int rc, const char* what) {
  if (rc != 0)
    throw std::runtime_error(std::string(what) + " failed (code " + std::to_string(rc) + "): " + cvmm_last_error());
}

void* ptr(const Tensor& t) { return t.data_ptr(); }
void* ptr(const OptT& t) { return t.has_value() ? t->data_ptr() : nullptr; }
template <typename T> T* tptr(const OptT& t) { return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr; }
template <typename T> T* tptr(const Tensor& t) { return static_cast<T*>(t.data_ptr()); }

void require_device(const Tensor& t, const char* what) {
  if (!t.is_cuda())
    throw std::runtime_error(std::string("cvmm_codex_amd: ") + what +
                             " must be a ROCm GPU tensor (there is no CPU fallback)");
}

// Kernels read fp32 or op-dtype storage; other float types are widened to
// fp32 (exact), which leaves the in-kernel rounding to the op dtype unchanged.
Tensor storage_for(const Tensor& t, at::ScalarType op) {
  if (t.scalar_type() == at::kFloat || (op != at::kFloat && t.scalar_type() == op)) return t;
  return t.to(at::kFloat);
}

// [rows, width] view with unit column stride and a row stride >= width.
Tensor rows_of(const Tensor& t, int64_t width) {
  Tensor f = t.reshape({-1, width});
  if (f.stride(1) != 1 || (f.size(0) > 1 && f.stride(0) < width)) f = f.contiguous();
  return f;
}

Tensor keys_view(const Tensor& keys) {
  if (keys.stride(2) == 1 || keys.stride(1) == 1) return keys;
  return keys.contiguous();
}

Tensor as_i64(const Tensor& t) {
  Tensor f = t.reshape({-1});
  if (f.scalar_type() != at::kLong) f = f.to(at::kLong);
  return f.contiguous();
}

OptT as_i64(const OptT& t) {
  if (!t.has_value()) return std::nullopt;
  return as_i64(*t);
}

Tensor sorted_i32(const Tensor& s) {
  Tensor f = s.reshape({-1});
  if (f.scalar_type() != at::kInt) f = f.to(at::kInt);
  return f.contiguous();
}

bool fast_path(at::ScalarType op, int64_t d_in, int64_t d_out) {
  return (op == at::kBFloat16 || op == at::kHalf) && d_in % 8 == 0 && d_out % 8 == 0;
}

at::TensorOptions opts(const Tensor& like, at::ScalarType dt) {
  return at::TensorOptions().dtype(dt).device(like.device());
}

// Scratch kept per (device, stream): calls on one stream run in stream order,
// so they can share it.
struct Scratch {
  Tensor buf;
  size_t clean = 0;       // length of the prefix known to be zero
  bool captured = false;  // a HIP graph capture recorded kernels that use buf
};
std::mutex g_mu;
std::map<std::pair<int, int64_t>, Scratch> g_sort_ws, g_wgrad_ws;
// Kept buffers replaced by larger ones after a graph capture used them: the
// graph's replays still read and write them, so they stay allocated until the
// process ends instead of going back to the allocator.
std::vector<Tensor> g_retired;

bool stream_capturing(int64_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing((hipStream_t)(uintptr_t)stream, &st) == hipSuccess &&
         st == hipStreamCaptureStatusActive;
}

// The kept scratch of `s` with at least `bytes`, (re)allocated -- and zeroed
// when `zero` -- on `stream` itself, the stream the kernels that use it run on.
// Call with g_mu held.
Tensor& kept_scratch(Scratch& s, const Tensor& like, int64_t stream, size_t bytes, bool zero) {
  if (!s.buf.defined() || (size_t)s.buf.numel() < bytes) {
    if (s.buf.defined() && s.captured) g_retired.push_back(s.buf);
    c10::hip::HIPStreamGuard guard(
        c10::hip::getStreamFromExternal((hipStream_t)(uintptr_t)stream, like.get_device()));
    const int64_t n = (int64_t)std::max<size_t>(bytes, 1);
    s.buf = zero ? at::zeros({n}, opts(like, at::kByte)) : at::empty({n}, opts(like, at::kByte));
    s.clean = zero ? (size_t)n : 0;
    s.captured = false;
  }
  if (stream_capturing(stream)) s.captured = true;
  return s.buf;
}

Tensor sort_workspace(const Tensor& like, int64_t stream, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  return kept_scratch(g_sort_ws[{(int)like.get_device(), stream}], like, stream, bytes, false);
}

// ---------------------------------------------------------------------------
// selector preparation: stable counting sort (cvmm.py:24-27, :1796-1803)
// returns (sorted int32, perm int64, perm // top_k int64, offsets int64[E],
// route_pos int32 = inverse of perm)
// ---------------------------------------------------------------------------
std::vector<Tensor> sort_routes(const Tensor& raw, int64_t n_experts, int64_t top_k, int64_t stream,
                                const OptT& counted_ws) {
  require_device(raw, "sel");
  Tensor flat = raw.reshape({-1});
  if (flat.scalar_type() != at::kInt && flat.scalar_type() != at::kLong) flat = flat.to(at::kInt);
  flat = flat.contiguous();
  const int64_t R = flat.numel();
  Tensor i32 = at::empty({2 * R}, opts(flat, at::kInt));
  Tensor i64 = at::empty({2 * R + n_experts}, opts(flat, at::kLong));
  Tensor ssel = i32.narrow(0, 0, R), pos = i32.narrow(0, R, R);
  Tensor perm = i64.narrow(0, 0, R), tok = i64.narrow(0, R, R), off = i64.narrow(0, 2 * R, n_experts);
  const size_t ws_bytes = cvmm_sort_workspace_bytes(R, (int32_t)n_experts);
  Tensor ws = counted_ws.has_value() ? *counted_ws : sort_workspace(flat, stream, ws_bytes);
  check(cvmm_sort_routes_cast_keys_ex(ptr(flat), flat.scalar_type() == at::kLong ? 1 : 0, R, (int32_t)n_experts,
                                      std::max<int64_t>(top_k, 1), tptr<int32_t>(ssel), tptr<int64_t>(perm),
                                      tptr<int64_t>(tok), tptr<int64_t>(off), tptr<int32_t>(pos), nullptr, ptr(ws),
                                      (size_t)ws.numel(), nullptr, 0, 0, 0, 0, 0, 0, 0, nullptr, nullptr, 0,
                                      counted_ws.has_value() ? CVMM_FLAG_COUNTS_READY : 0, (void*)stream),
        "cvmm_sort_routes");
  return {ssel, perm, tok, off, pos};
}

// The op-dtype weight copies of a cast (`layout`: CVMM_CAST_* bits): kt
// [E, d_out, d_in] or, interleaved, [d_out, E, d_in]; kn [E, d_in, d_out] or
// [d_in, E, d_out].
std::tuple<OptT, OptT> cast_outputs(const Tensor& keys, at::ScalarType op, bool want_t, bool want_n,
                                    int64_t layout) {
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  OptT kt, kn;
  if (want_t)
    kt = (layout & CVMM_CAST_T_INTERLEAVED) ? at::empty({d_out, E, d_in}, opts(keys, op))
                                            : at::empty({E, d_out, d_in}, opts(keys, op));
  if (want_n)
    kn = (layout & CVMM_CAST_N_INTERLEAVED) ? at::empty({d_in, E, d_out}, opts(keys, op))
                                            : at::empty({E, d_in, d_out}, opts(keys, op));
  return {kt, kn};
}

// The sort and the same step's weight cast in one call (the cast runs in the
// scatter launch): (sorted, perm, perm // top_k, offsets, route_pos), kt, kn.
std::tuple<std::vector<Tensor>, OptT, OptT> sort_routes_cast(const Tensor& raw, int64_t n_experts, int64_t top_k,
                                                             const Tensor& keys, int64_t op_id, bool want_t,
                                                             bool want_n, int64_t layout, int64_t stream,
                                                             const OptT& counted_ws) {
  require_device(raw, "sel");
  require_device(keys, "keys");
  Tensor flat = raw.reshape({-1});
  if (flat.scalar_type() != at::kInt && flat.scalar_type() != at::kLong) flat = flat.to(at::kInt);
  flat = flat.contiguous();
  const int64_t R = flat.numel();
  Tensor i32 = at::empty({2 * R}, opts(flat, at::kInt));
  Tensor i64 = at::empty({2 * R + n_experts}, opts(flat, at::kLong));
  Tensor ssel = i32.narrow(0, 0, R), pos = i32.narrow(0, R, R);
  Tensor perm = i64.narrow(0, 0, R), tok = i64.narrow(0, R, R), off = i64.narrow(0, 2 * R, n_experts);
  const auto op = dtype_of(op_id);
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  if (E != n_experts) throw py::value_error("cvmm: keys.shape[0] differs from the expert count");
  auto [kt, kn] = cast_outputs(keys, op, want_t, want_n, layout);
  const size_t ws_bytes = cvmm_sort_workspace_bytes(R, (int32_t)n_experts);
  Tensor ws = counted_ws.has_value() ? *counted_ws : sort_workspace(flat, stream, ws_bytes);
  check(cvmm_sort_routes_cast_keys_ex(ptr(flat), flat.scalar_type() == at::kLong ? 1 : 0, R, (int32_t)n_experts,
                                      std::max<int64_t>(top_k, 1), tptr<int32_t>(ssel), tptr<int64_t>(perm),
                                      tptr<int64_t>(tok), tptr<int64_t>(off), tptr<int32_t>(pos), nullptr, ptr(ws),
                                      (size_t)ws.numel(), ptr(keys), dtype_id(keys.scalar_type()), d_in, d_out,
                                      keys.stride(0), keys.stride(1), keys.stride(2), (int32_t)op_id, ptr(kt),
                                      ptr(kn), (int32_t)layout, counted_ws.has_value() ? CVMM_FLAG_COUNTS_READY : 0,
                                      (void*)stream),
        "cvmm_sort_routes_cast_keys");
  return {{ssel, perm, tok, off, pos}, kt, kn};
}

// ---------------------------------------------------------------------------
// router (no counterpart in cvmm.py; its callers' softmax -> top-k ->
// renormalise -> cvmm_prepare_sel2): (weights fp32 [T, k], sel int64 [T, k],
// sorted int32, perm, perm // k, offsets, route_pos)
// ---------------------------------------------------------------------------
std::vector<Tensor> route_topk(const Tensor& logits, int64_t top_k, bool renormalize, int64_t stream) {
  require_device(logits, "logits");
  Tensor l = logits.reshape({-1, logits.size(-1)});
  if (l.stride(-1) != 1) l = l.contiguous();
  const int64_t T = l.size(0), E = l.size(1);
  const int64_t R = T * top_k;
  Tensor w = at::empty({T, top_k}, opts(l, at::kFloat));
  Tensor sel = at::empty({T, top_k}, opts(l, at::kLong));
  Tensor i32 = at::empty({2 * R}, opts(l, at::kInt));
  Tensor i64 = at::empty({2 * R + E}, opts(l, at::kLong));
  Tensor ssel = i32.narrow(0, 0, R), pos = i32.narrow(0, R, R);
  Tensor perm = i64.narrow(0, 0, R), tok = i64.narrow(0, R, R), off = i64.narrow(0, 2 * R, E);
  const size_t ws_bytes = cvmm_route_topk_workspace_bytes(T, (int32_t)E, top_k);
  Tensor ws = sort_workspace(l, stream, ws_bytes);
  check(cvmm_route_topk(ptr(l), dtype_id(l.scalar_type()), T, l.stride(0), (int32_t)E, top_k, renormalize ? 1 : 0,
                        tptr<float>(w), tptr<int64_t>(sel), tptr<int32_t>(ssel), tptr<int64_t>(perm),
                        tptr<int64_t>(tok), tptr<int64_t>(off), tptr<int32_t>(pos), ptr(ws), (size_t)ws.numel(),
                        (void*)stream),
        "cvmm_route_topk");
  return {w, sel, ssel, perm, tok, off, pos};
}

Tensor route_topk_backward(const Tensor& logits, const Tensor& sel, const Tensor& grad_weights, int64_t top_k,
                           bool renormalize, int64_t stream) {
  require_device(logits, "logits");
  Tensor l = logits.reshape({-1, logits.size(-1)});
  if (l.stride(-1) != 1) l = l.contiguous();
  const int64_t T = l.size(0), E = l.size(1);
  Tensor s = sel.reshape({-1}).contiguous();
  Tensor g = grad_weights.reshape({-1}).to(at::kFloat).contiguous();
  if (s.numel() != T * top_k || g.numel() != T * top_k)
    throw py::value_error("cvmm_route_topk: sel / grad have the wrong size");
  Tensor out = at::empty({T, E}, opts(l, l.scalar_type()));
  check(cvmm_route_topk_backward(ptr(l), dtype_id(l.scalar_type()), T, l.stride(0), (int32_t)E, top_k,
                                 renormalize ? 1 : 0, tptr<int64_t>(s), tptr<float>(g), ptr(out), out.stride(0),
                                 (void*)stream),
        "cvmm_route_topk_backward");
  return out.view(logits.sizes());
}

// The int32 copy of the ids cvmm_prepare_sel2 takes (cvmm.py:1796), in the
// ids' shape.
Tensor copy_ids(const Tensor& sel, int64_t stream) {
  require_device(sel, "sel");
  Tensor flat = sel.reshape({-1});
  if (flat.scalar_type() != at::kInt && flat.scalar_type() != at::kLong) flat = flat.to(at::kLong);
  flat = flat.contiguous();
  Tensor out = at::empty(sel.sizes(), opts(flat, at::kInt));
  check(cvmm_copy_ids(ptr(flat), flat.scalar_type() == at::kLong ? 1 : 0, flat.numel(), tptr<int32_t>(out),
                      (void*)stream),
        "cvmm_copy_ids");
  return out;
}

// copy_ids plus the sort's count matrix for an expected expert count, in a
// sort workspace of its own: (ids, workspace).  A sort of the copy for that
// count passes the workspace and CVMM_FLAG_COUNTS_READY.
std::tuple<Tensor, Tensor> copy_ids_count(const Tensor& sel, int64_t n_experts, int64_t stream) {
  require_device(sel, "sel");
  Tensor flat = sel.reshape({-1});
  if (flat.scalar_type() != at::kInt && flat.scalar_type() != at::kLong) flat = flat.to(at::kLong);
  flat = flat.contiguous();
  Tensor out = at::empty(sel.sizes(), opts(flat, at::kInt));
  const size_t ws_bytes = cvmm_sort_workspace_bytes(flat.numel(), (int32_t)n_experts);
  Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 1)}, opts(flat, at::kByte));
  check(cvmm_copy_ids_count(ptr(flat), flat.scalar_type() == at::kLong ? 1 : 0, flat.numel(), (int32_t)n_experts,
                            tptr<int32_t>(out), ptr(ws), (size_t)ws.numel(), (void*)stream),
        "cvmm_copy_ids_count");
  return {out, ws};
}

Tensor expert_offsets(const Tensor& sorted, int64_t n_experts, int64_t stream) {
  require_device(sorted, "sorted_experts");
  Tensor s = sorted_i32(sorted);
  Tensor out = at::empty({n_experts}, opts(s, at::kLong));
  check(cvmm_expert_offsets(tptr<int32_t>(s), s.numel(), (int32_t)n_experts, tptr<int64_t>(out), (void*)stream),
        "cvmm_expert_offsets");
  return out;
}

// keys [E, d_in, d_out] -> op-dtype copies kt (forward) and kn (grad-input)
// in the layouts of cast_outputs, one pass.
std::tuple<OptT, OptT> cast_keys(const Tensor& keys, int64_t op_id, bool want_t, bool want_n, int64_t layout,
                                 int64_t stream) {
  require_device(keys, "keys");
  const auto op = dtype_of(op_id);
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  auto [kt, kn] = cast_outputs(keys, op, want_t, want_n, layout);
  check(cvmm_cast_keys(ptr(keys), dtype_id(keys.scalar_type()), (int32_t)E, d_in, d_out, keys.stride(0),
                       keys.stride(1), keys.stride(2), (int32_t)op_id, ptr(kt), ptr(kn), (int32_t)layout,
                       (void*)stream),
        "cvmm_cast_keys");
  return {kt, kn};
}

// ---------------------------------------------------------------------------
// forward (cvmm.py:1524-1550): returns [out_rows, d_out] in the op dtype
// ---------------------------------------------------------------------------
// The op-dtype weight copy a call reads, as the logical [E, d_in, d_out]
// view: `copy` is the [E, d_out, d_in] copy when `is_t`, else the view itself
// (a [E, d_in, d_out] copy, or an interleaved copy already viewed so).
Tensor copy_view(const Tensor& copy, bool is_t) { return is_t ? copy.transpose(1, 2) : copy; }

// `scaled` (not NULL): a weighted route-input call keeps its scaled route
// rows there for the weight gradient where the library makes them anyway
// (cvmm_fwd_keep_scaled: the dense top-k sum, or the small-K routed product's
// activation fragments); left undefined otherwise.
Tensor cvmm_forward_impl(const Tensor& x, const Tensor& keys, const OptT& keys_op, bool keys_op_is_t, const Tensor& sel,
               const Tensor& sel_index, const OptT& out_index, const Tensor& offsets, const OptT& route_pos,
               const OptT& rw, int64_t op_id, int64_t out_id, int64_t flags, int64_t stream,
               Tensor* scaled = nullptr) {
  require_device(x, "x");
  require_device(keys, "keys");
  require_device(sel, "sel");
  require_device(sel_index, "sel_index");
  const auto op = dtype_of(op_id);
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  TORCH_CHECK(x.size(-1) == d_in, "cvmm: x.shape[-1] must equal keys.shape[1]");  // cvmm.py:825
  Tensor xf, kv;
  if (keys_op.has_value()) {
    // op-dtype activations and an op-dtype weight copy: the [E, d_out, d_in]
    // copy (unit stride on d_in, the routed kernels' layout) or the
    // [E, d_in, d_out] one (the dense top-k GEMM's rows)
    xf = rows_of(x.scalar_type() == op ? x : x.to(op), d_in);
    kv = copy_view(*keys_op, keys_op_is_t);
  } else {
    xf = rows_of(storage_for(x, op), d_in);
    kv = keys_view(storage_for(keys, op));
  }
  Tensor s32 = sorted_i32(sel);
  const int64_t R = s32.numel();
  Tensor si = as_i64(sel_index);
  OptT oi = as_i64(out_index);
  if (si.numel() != R || (oi.has_value() && oi->numel() != R))
    throw py::value_error("cvmm: sel_index/out_index must have one entry per route");
  OptT rwf;
  int64_t k = 1, out_rows = R;
  if (rw.has_value()) {
    require_device(*rw, "reduction_weight");
    if (rw->numel() != R) throw py::value_error("cvmm: reduction_weight must have one entry per route");
    k = rw->size(-1);
    rwf = rw->reshape({-1}).contiguous();
    out_rows = R / k;
  }
  const int32_t od = (int32_t)op_id;
  // the output dtype: the op dtype (-1), or another one the products are
  // rounded to directly (the reference op's out_dtype, cvmm.py:832-833)
  const int32_t outd = out_id < 0 ? od : (int32_t)out_id;
  Tensor out = at::empty({out_rows, d_out}, opts(x, dtype_of(outd)));
  const size_t ws_bytes = cvmm_fwd_workspace_bytes(R, (int32_t)E, d_in, d_out, out_rows, outd, od, 1,
                                                   rw.has_value() ? 1 : 0, (int32_t)flags);
  OptT ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, opts(x, at::kByte));
  if (scaled != nullptr && rwf.has_value() && !oi.has_value() && xf.size(0) == R && outd == od &&
      (op == at::kBFloat16 || op == at::kHalf) && !(flags & CVMM_FLAG_ATOMIC_REDUCE) &&
      (cvmm_topk_dense(out_rows, (int32_t)E, d_in, d_out, k, od) == 1 || d_in <= 128)) {
    // (the dense sum, or a small-K routed product: the two that keep them)
    Tensor xs = at::empty({R, d_in}, opts(x, op));
    int32_t written = 0;
    check(cvmm_fwd_keep_scaled(ptr(xf), dtype_id(xf.scalar_type()), xf.size(0), xf.stride(0), ptr(kv),
                               dtype_id(kv.scalar_type()), (int32_t)E, d_in, d_out, kv.stride(0), kv.stride(1),
                               kv.stride(2), tptr<int32_t>(s32), tptr<int64_t>(si), nullptr, R,
                               tptr<int64_t>(offsets), tptr<int32_t>(route_pos), ptr(rwf),
                               dtype_id(rwf->scalar_type()), k, od, ptr(out), outd, out_rows, d_out, ptr(xs),
                               &written, (int32_t)flags, ptr(ws), ws_bytes, (void*)stream),
          "cvmm_fwd_keep_scaled");
    if (written) *scaled = xs;
    return out;
  }
  check(cvmm_fwd(ptr(xf), dtype_id(xf.scalar_type()), xf.size(0), xf.stride(0), ptr(kv),
                 dtype_id(kv.scalar_type()), (int32_t)E, d_in, d_out, kv.stride(0), kv.stride(1), kv.stride(2),
                 tptr<int32_t>(s32), tptr<int64_t>(si), tptr<int64_t>(oi), R, tptr<int64_t>(offsets),
                 tptr<int32_t>(route_pos), ptr(rwf), rwf.has_value() ? dtype_id(rwf->scalar_type()) : 0, k, od,
                 ptr(out), outd, out_rows, d_out, (int32_t)flags, ptr(ws), ws_bytes, (void*)stream),
        "cvmm_fwd");
  return out;
}

// ---------------------------------------------------------------------------
// forward + GELU (no counterpart in cvmm.py: its callers' F.gelu(cvmm(...)),
// benchmark_ffn_moe.py:96), unweighted selections: (gelu(h), h), [R, d_out]
// in the op dtype
// ---------------------------------------------------------------------------
std::tuple<Tensor, Tensor> forward_gelu(const Tensor& x, const Tensor& keys, const OptT& keys_t, bool keys_t_is_t,
                                        const Tensor& sel,
                                        const Tensor& sel_index, const OptT& out_index, const Tensor& offsets,
                                        const OptT& route_pos, int64_t op_id, int64_t flags, int64_t stream) {
  require_device(x, "x");
  require_device(keys, "keys");
  require_device(sel, "sel");
  require_device(sel_index, "sel_index");
  const auto op = dtype_of(op_id);
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  TORCH_CHECK(x.size(-1) == d_in, "cvmm: x.shape[-1] must equal keys.shape[1]");  // cvmm.py:825
  Tensor xf, kv;
  if (keys_t.has_value()) {
    xf = rows_of(x.scalar_type() == op ? x : x.to(op), d_in);
    kv = copy_view(*keys_t, keys_t_is_t);
  } else {
    xf = rows_of(storage_for(x, op), d_in);
    kv = keys_view(storage_for(keys, op));
  }
  Tensor s32 = sorted_i32(sel);
  const int64_t R = s32.numel();
  Tensor si = as_i64(sel_index);
  OptT oi = as_i64(out_index);
  if (si.numel() != R || (oi.has_value() && oi->numel() != R))
    throw py::value_error("cvmm: sel_index/out_index must have one entry per route");
  const int32_t od = (int32_t)op_id;
  Tensor out = at::empty({R, d_out}, opts(x, op));
  Tensor pre = at::empty({R, d_out}, opts(x, op));
  const size_t ws_bytes = cvmm_fwd_workspace_bytes(R, (int32_t)E, d_in, d_out, R, od, od, 1, 0, (int32_t)flags);
  OptT ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, opts(x, at::kByte));
  check(cvmm_fwd_gelu(ptr(xf), dtype_id(xf.scalar_type()), xf.size(0), xf.stride(0), ptr(kv),
                      dtype_id(kv.scalar_type()), (int32_t)E, d_in, d_out, kv.stride(0), kv.stride(1), kv.stride(2),
                      tptr<int32_t>(s32), tptr<int64_t>(si), tptr<int64_t>(oi), R, tptr<int64_t>(offsets),
                      tptr<int32_t>(route_pos), od, ptr(out), od, R, d_out, ptr(pre), (int32_t)flags, ptr(ws),
                      ws_bytes, (void*)stream),
        "cvmm_fwd_gelu");
  return {out, pre};
}

Tensor gelu_backward(const Tensor& grad, const Tensor& pre, int64_t stream) {
  require_device(grad, "grad");
  require_device(pre, "pre_act");
  const int64_t cols = pre.size(-1);
  Tensor g = rows_of(grad, cols);
  Tensor h = rows_of(pre, cols);
  if (g.size(0) != h.size(0)) throw py::value_error("cvmm_gelu: grad and pre-activation shapes differ");
  Tensor out = at::empty({h.size(0), cols}, opts(h, h.scalar_type()));
  check(cvmm_gelu_backward(ptr(g), dtype_id(g.scalar_type()), g.stride(0), ptr(h), dtype_id(h.scalar_type()),
                           h.stride(0), h.size(0), cols, ptr(out), dtype_id(out.scalar_type()), out.stride(0),
                           (void*)stream),
        "cvmm_gelu_backward");
  return out;
}

// ---------------------------------------------------------------------------
// backward (cvmm.py:1552-1755): (grad_x, grad_keys, grad_reduction_weight)
// ---------------------------------------------------------------------------
// Host-side flags above the ABI's 32 bits: bits 32..47 carry the low-memory
// grad-input's top-k columns per slice (cvmm_lowmem_chunk_size; 0: all).
int64_t lowmem_chunk_of(int64_t flags) { return (flags >> 32) & 0xffff; }

// Host flag (bit 48, never passed to the C ABI): the backward's weight
// gradient runs on a second stream of the device, concurrent with the
// grad-input and its top-k sum, which it does not depend on.
constexpr int64_t kHostOverlapBackward = int64_t(1) << 48;

// The second stream: one torch pool stream per device (default priority),
// and the fork / join events, created once; record-and-wait pairs under a
// lock.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
std::map<int, SideStream> g_side;

SideStream& side_stream(int dev) {
  SideStream& ss = g_side[dev];
  if (ss.stream == nullptr) {
    ss.stream = c10::hip::getStreamFromPool(false, (c10::DeviceIndex)dev).stream();
    c10::hip::HIPGuard guard((c10::DeviceIndex)dev);
    TORCH_CHECK(hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) == hipSuccess &&
                    hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) == hipSuccess,
                "cvmm: event creation failed");
  }
  return ss;
}

// Work enqueued on `main` so far -> the side stream of the device: returns it.
hipStream_t fork_to_side(int dev, hipStream_t main) {
  std::lock_guard<std::mutex> lk(g_side_mu);
  SideStream& ss = side_stream(dev);
  TORCH_CHECK(hipEventRecord(ss.fork, main) == hipSuccess && hipStreamWaitEvent(ss.stream, ss.fork, 0) == hipSuccess,
              "cvmm: stream fork failed");
  return ss.stream;
}

// Makes `main` wait for the side stream's work when it goes out of scope
// (every return and exception path of the backward after a fork).
struct SideJoin {
  int dev = -1;
  hipStream_t main = nullptr;
  ~SideJoin() {
    if (dev < 0) return;
    std::lock_guard<std::mutex> lk(g_side_mu);
    SideStream& ss = side_stream(dev);
    hipEventRecord(ss.join, ss.stream);
    hipStreamWaitEvent(main, ss.join, 0);
  }
};

// The token gradient of a token-input unweighted top-k sum taken over slices
// of `chunk` top-k columns (cvmm_grouped_backward_lowmem, cvmm.py:1228-1338):
// each slice of the selection is sorted on its own, its routes' rows go
// through a route buffer of T * chunk rows (not T * top_k), and are added in
// route order to an fp32 running sum (CVMM_FLAG_ACCUMULATE) that is rounded
// once at the end -- the bits of the one-call sum.  g: [T * top_k, d_out]
// route rows; perm: the selection's out_index; s32: its sorted ids.
Tensor grad_x_by_slices(const Tensor& g, const Tensor& kv, const Tensor& s32, const Tensor& perm, int64_t T,
                        int64_t k, int64_t E, int64_t d_in, int64_t d_out, int64_t chunk, at::ScalarType x_type,
                        int32_t od, int64_t flags, int64_t stream) {
  Tensor ids = at::empty({T * k}, s32.options());
  ids.index_put_({perm}, s32);  // the id of route t * k + j
  ids = ids.view({T, k});
  Tensor gv = g.reshape({T, k, d_out});
  Tensor acc = at::zeros({T, d_in}, g.options().dtype(at::kFloat));
  const int32_t aflags = (int32_t)flags | CVMM_FLAG_ACCUMULATE;
  for (int64_t cs = 0; cs < k; cs += chunk) {
    const int64_t c = std::min(chunk, k - cs), Rc = T * c;
    Tensor ids_c = ids.narrow(1, cs, c).contiguous();
    const std::vector<Tensor> srt = sort_routes(ids_c, E, c, stream, std::nullopt);  // ssel, perm, tok, off, pos
    Tensor g_c = gv.narrow(1, cs, c).reshape({Rc, d_out}).contiguous();
    const size_t ws_bytes = cvmm_bwd_x_workspace_bytes(Rc, (int32_t)E, d_in, d_out, T, 1, 0, 1, c, dtype_id(x_type),
                                                       od, 0, aflags);
    OptT ws;
    if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, opts(g, at::kByte));
    check(cvmm_bwd_x(ptr(g_c), dtype_id(g_c.scalar_type()), Rc, d_out, ptr(kv), dtype_id(kv.scalar_type()),
                     (int32_t)E, d_in, d_out, kv.stride(0), kv.stride(1), kv.stride(2), tptr<int32_t>(srt[0]),
                     tptr<int64_t>(srt[2]), tptr<int64_t>(srt[1]), Rc, tptr<int64_t>(srt[3]),
                     tptr<int32_t>(srt[4]), nullptr, 0, c, nullptr, dtype_id(x_type), 0, 0, od, ptr(acc),
                     dtype_id(at::kFloat), T, d_in, nullptr, 0, aflags, ptr(ws), ws_bytes, (void*)stream),
          "cvmm_bwd_x(slice)");
  }
  return acc.to(x_type);
}

std::tuple<OptT, OptT, OptT> cvmm_backward_impl(const Tensor& grad_output, const Tensor& x, const Tensor& keys,
                                      const OptT& keys_x, bool keys_x_is_t, const Tensor& sel, const Tensor& sel_index,
                                      const OptT& out_index, const Tensor& offsets, const OptT& route_pos,
                                      const OptT& rw, int64_t top_k, int64_t op_id, bool need_grad_x,
                                      bool need_grad_keys, bool need_grad_rw, int64_t flags, int64_t stream,
                                      const OptT& scaled_x = std::nullopt) {
  const auto op = dtype_of(op_id);
  const int64_t E = keys.size(0), d_in = keys.size(1), d_out = keys.size(2);
  const int64_t k = rw.has_value() ? rw->size(-1) : top_k;
  const bool fast = fast_path(op, d_in, d_out);
  Tensor g = rows_of(fast && grad_output.scalar_type() != op ? grad_output.to(op) : storage_for(grad_output, op),
                     d_out);
  Tensor s32 = sorted_i32(sel);
  const int64_t R = s32.numel();
  Tensor si = as_i64(sel_index);
  OptT oi = as_i64(out_index);
  OptT rwf;
  if (rw.has_value()) rwf = rw->reshape({-1}).contiguous();
  const int32_t rwd = rwf.has_value() ? dtype_id(rwf->scalar_type()) : 0;
  const int32_t od = (int32_t)op_id;
  OptT grad_x, grad_w, grad_rw;
  // the weight gradient's x rows: declared before the join below, so that
  // a temporary (x converted to the op dtype) outlives the side stream's use
  Tensor xs;
  // joins the side stream back into `stream` on every way out below (and,
  // destroyed before the tensors declared above, before they are freed)
  SideJoin join;

  if (need_grad_keys) {
    // the route rows the forward scaled (cvmm_fwd_keep_scaled), or x
    const bool pre_scaled = scaled_x.has_value();
    xs = pre_scaled ? *scaled_x : rows_of(fast && x.scalar_type() != op ? x.to(op) : storage_for(x, op), d_in);
    grad_w = at::empty(keys.sizes(), opts(keys, keys.scalar_type()));
    // with a grad-input to run as well, the weight gradient goes to the side
    // stream once its inputs are enqueued; its inputs (g, xs and the routing
    // tensors, all declared before `join`) are freed to the caller's stream
    // only after the join, so no later work there reuses them too early
    int64_t wstream = stream;
    if ((flags & kHostOverlapBackward) && (need_grad_x || need_grad_rw)) {
      wstream = (int64_t)(uintptr_t)fork_to_side(x.get_device(), (hipStream_t)(uintptr_t)stream);
      join.dev = x.get_device();
      join.main = (hipStream_t)(uintptr_t)stream;
    }
    // a weighted route-input selection gets room for its scaled route rows
    // (none needed when the forward kept them)
    const size_t ws_bytes = cvmm_bwd_w_workspace_bytes_ex(R, (int32_t)E, d_in, d_out, od, 1,
                                                          rw.has_value() && !oi.has_value() && !pre_scaled ? 1 : 0);
    const size_t ctr_bytes = cvmm_bwd_w_counter_bytes(R, (int32_t)E, d_in, d_out, od);
    Tensor ws;
    bool zeroed;
    {
      // the tile counters at the start of the workspace are left zero by the
      // kernel; a kept workspace is zeroed once (when allocated)
      std::lock_guard<std::mutex> lk(g_mu);
      Scratch& s = g_wgrad_ws[{(int)x.get_device(), wstream}];
      kept_scratch(s, x, wstream, ws_bytes, true);
      zeroed = ctr_bytes <= s.clean;
      s.clean = ctr_bytes;  // partial tiles follow the counter region
      ws = s.buf;
    }
    const int32_t wflags = (int32_t)flags | (zeroed ? CVMM_FLAG_COUNTERS_ZEROED : 0) |
                           (pre_scaled ? CVMM_FLAG_ROWS_SCALED : 0);
    check(cvmm_bwd_w(ptr(xs), dtype_id(xs.scalar_type()), xs.size(0), xs.stride(0), ptr(g),
                     dtype_id(g.scalar_type()), g.size(0), g.stride(0), (int32_t)E, d_in, d_out, tptr<int32_t>(s32),
                     tptr<int64_t>(si), tptr<int64_t>(oi), R, tptr<int64_t>(offsets), ptr(rwf), rwd, k, od,
                     ptr(grad_w), dtype_id(grad_w->scalar_type()), grad_w->stride(0), grad_w->stride(1),
                     grad_w->stride(2), wflags, ptr(ws), (size_t)ws.numel(), (void*)wstream),
          "cvmm_bwd_w");
  }

  if (need_grad_x || need_grad_rw) {
    // the grad-input's weight copy: [E, d_in, d_out] for the routed GEMM, the
    // transposed one for a dense top-k sum, else the keys as stored
    Tensor kv = keys_x.has_value() ? copy_view(*keys_x, keys_x_is_t) : keys_view(storage_for(keys, op));
    Tensor xr = rows_of(x, d_in);
    OptT gx;
    if (need_grad_x) gx = at::empty(xr.sizes(), opts(x, x.scalar_type()));
    if (need_grad_rw) grad_rw = at::empty(rw->sizes(), opts(*rw, rw->scalar_type()));
    const int64_t gx_rows = gx.has_value() ? gx->size(0) : xr.size(0);
    // a token-input unweighted top-k sum on the route buffer can run over
    // slices of its top-k columns: when cvmm_lowmem_chunk_size asks for it,
    // or when the one-call workspace does not fit (halving the slice until
    // it does), as the reference falls back on torch.OutOfMemoryError
    const bool sliceable = need_grad_x && !rw.has_value() && oi.has_value() && k > 1 && k <= 64 &&
                           !(flags & CVMM_FLAG_ATOMIC_REDUCE) && d_in % 8 == 0 &&
                           (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf) &&
                           cvmm_topk_dense(gx_rows, (int32_t)E, d_out, d_in, k, od) == 0;
    auto by_slices = [&](int64_t chunk) {
      return grad_x_by_slices(g, kv, s32, *oi, gx_rows, k, E, d_in, d_out, chunk, x.scalar_type(), od, flags, stream)
          .view(x.sizes());
    };
    const int64_t chunk = lowmem_chunk_of(flags);
    if (sliceable && chunk > 0 && chunk < k) {
      gx.reset();
      return {by_slices(chunk), grad_w, grad_rw};
    }
    const size_t ws_bytes = cvmm_bwd_x_workspace_bytes(R, (int32_t)E, d_in, d_out, gx_rows, 1, rw.has_value() ? 1 : 0,
                                                       oi.has_value() ? 1 : 0, k, dtype_id(x.scalar_type()), od,
                                                       need_grad_rw ? 1 : 0, (int32_t)flags);
    OptT ws;
    try {
      if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, opts(x, at::kByte));
    } catch (const c10::OutOfMemoryError&) {
      if (!sliceable) throw;
      gx.reset();
      for (int64_t c = k / 2;; c /= 2) {
        try {
          return {by_slices(c), grad_w, grad_rw};
        } catch (const c10::OutOfMemoryError&) {
          if (c <= 1) throw;
        }
      }
    }
    check(cvmm_bwd_x(ptr(g), dtype_id(g.scalar_type()), g.size(0), g.stride(0), ptr(kv),
                     dtype_id(kv.scalar_type()), (int32_t)E, d_in, d_out, kv.stride(0), kv.stride(1), kv.stride(2),
                     tptr<int32_t>(s32), tptr<int64_t>(si), tptr<int64_t>(oi), R, tptr<int64_t>(offsets),
                     tptr<int32_t>(route_pos), ptr(rwf), rwd, k, ptr(xr), dtype_id(xr.scalar_type()), xr.size(0),
                     xr.stride(0), od, ptr(gx), dtype_id(x.scalar_type()), gx_rows, d_in, ptr(grad_rw),
                     rw.has_value() ? dtype_id(rw->scalar_type()) : 0, (int32_t)flags, ptr(ws), ws_bytes,
                     (void*)stream),
          "cvmm_bwd_x");
    if (gx.has_value()) grad_x = gx->view(x.sizes());
  }
  return {grad_x, grad_w, grad_rw};
}

// ---------------------------------------------------------------------------
// CVMM as a C++ autograd function (cvmm.py:1521-1755): the forward above, and
// a backward node that runs the backward above on the autograd engine's
// device thread without Python.  A Python autograd.Function's node takes the
// GIL on that thread to run its backward and again to free its context,
// which stalls the caller's next step.
// ---------------------------------------------------------------------------
int64_t current_stream(const Tensor& like) {
  return (int64_t)(uintptr_t)c10::hip::getCurrentHIPStream(like.get_device()).stream();
}

Tensor opt_or_undef(const OptT& t) { return t.has_value() ? *t : Tensor(); }
OptT undef_or_opt(const Tensor& t) { return t.defined() ? OptT(t) : std::nullopt; }

struct CvmmFunction : public torch::autograd::Function<CvmmFunction> {
  // x, keys and reduction_weight (optional) are the differentiable inputs;
  // the rest is routing, the op-dtype weight copies and settings.
  static Tensor forward(torch::autograd::AutogradContext* ctx, const Tensor& x, const Tensor& keys, const OptT& rw,
                        const Tensor& sel, const Tensor& sel_index, const OptT& out_index, const Tensor& offsets,
                        const OptT& route_pos, const OptT& keys_op, bool keys_op_is_t, const OptT& keys_x,
                        bool keys_x_is_t, int64_t top_k, int64_t op_id, int64_t flags,
                        const std::vector<int64_t>& out_shape) {
    const bool need_x = x.requires_grad(), need_keys = keys.requires_grad();
    const bool need_rw = rw.has_value() && rw->requires_grad();
    ctx->saved_data["keys_x_is_t"] = keys_x_is_t;
    ctx->saved_data["top_k"] = top_k;
    ctx->saved_data["op_id"] = op_id;
    ctx->saved_data["flags"] = flags;
    ctx->saved_data["need"] = (int64_t)((need_x ? 1 : 0) | (need_keys ? 2 : 0) | (need_rw ? 4 : 0));
    // a weight gradient that needs the weight-scaled route rows the forward's
    // dense top-k sum makes keeps them (one pass over the route rows saved)
    Tensor scaled;
    Tensor out = cvmm_forward_impl(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index, offsets, route_pos,
                                   rw, op_id, -1, flags, current_stream(x), need_keys ? &scaled : nullptr);
    ctx->save_for_backward({x, keys, opt_or_undef(rw), sel, sel_index, opt_or_undef(out_index), offsets,
                            opt_or_undef(route_pos), need_x || need_rw ? opt_or_undef(keys_x) : Tensor(), scaled});
    // not a view in autograd's sense (its base is no input and is never seen)
    return at::_unsafe_view(out, out_shape);
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto v = ctx->get_saved_variables();
    const Tensor& x = v[0];
    const int64_t need = ctx->saved_data["need"].toInt();
    auto [gx, gw, grw] = cvmm_backward_impl(
        grads[0], x, v[1], undef_or_opt(v[8]), ctx->saved_data["keys_x_is_t"].toBool(), v[3], v[4],
        undef_or_opt(v[5]), v[6], undef_or_opt(v[7]), undef_or_opt(v[2]), ctx->saved_data["top_k"].toInt(),
        ctx->saved_data["op_id"].toInt(), (need & 1) != 0, (need & 2) != 0, (need & 4) != 0,
        ctx->saved_data["flags"].toInt(), current_stream(x), undef_or_opt(v[9]));
    // one entry per forward argument
    return {opt_or_undef(gx), opt_or_undef(gw), opt_or_undef(grw), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(),
            Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

// The Python-facing forward and backward (torch.compile's ops): no kept rows.
Tensor forward_py(const Tensor& x, const Tensor& keys, const OptT& keys_op, bool keys_op_is_t, const Tensor& sel,
                  const Tensor& sel_index, const OptT& out_index, const Tensor& offsets, const OptT& route_pos,
                  const OptT& rw, int64_t op_id, int64_t out_id, int64_t flags, int64_t stream) {
  return cvmm_forward_impl(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index, offsets, route_pos, rw, op_id,
                           out_id, flags, stream);
}

std::tuple<OptT, OptT, OptT> backward_py(const Tensor& grad_output, const Tensor& x, const Tensor& keys,
                                         const OptT& keys_x, bool keys_x_is_t, const Tensor& sel,
                                         const Tensor& sel_index, const OptT& out_index, const Tensor& offsets,
                                         const OptT& route_pos, const OptT& rw, int64_t top_k, int64_t op_id,
                                         bool need_grad_x, bool need_grad_keys, bool need_grad_rw, int64_t flags,
                                         int64_t stream) {
  return cvmm_backward_impl(grad_output, x, keys, keys_x, keys_x_is_t, sel, sel_index, out_index, offsets, route_pos,
                            rw, top_k, op_id, need_grad_x, need_grad_keys, need_grad_rw, flags, stream);
}

Tensor cvmm_apply(const Tensor& x, const Tensor& keys, const OptT& rw, const Tensor& sel, const Tensor& sel_index,
                  const OptT& out_index, const Tensor& offsets, const OptT& route_pos, const OptT& keys_op,
                  bool keys_op_is_t, const OptT& keys_x, bool keys_x_is_t, int64_t top_k, int64_t op_id,
                  int64_t flags, const std::vector<int64_t>& out_shape) {
  return CvmmFunction::apply(x, keys, rw, sel, sel_index, out_index, offsets, route_pos, keys_op, keys_op_is_t,
                             keys_x, keys_x_is_t, top_k, op_id, flags, out_shape);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Host glue of cvmm_codex_amd: one call per CVMM phase into libcvmm_hip.so";
  m.def("sort_routes", &sort_routes, py::arg("raw"), py::arg("n_experts"), py::arg("top_k"), py::arg("stream"),
        py::arg("counted_ws") = py::none());
  m.def("expert_offsets", &expert_offsets, py::arg("sorted"), py::arg("n_experts"), py::arg("stream"));
  m.def("copy_ids", &copy_ids, py::arg("sel"), py::arg("stream"));
  m.def("copy_ids_count", &copy_ids_count, py::arg("sel"), py::arg("n_experts"), py::arg("stream"));
  m.def("route_topk", &route_topk, py::arg("logits"), py::arg("top_k"), py::arg("renormalize"), py::arg("stream"));
  m.def("route_topk_backward", &route_topk_backward, py::arg("logits"), py::arg("sel"), py::arg("grad_weights"),
        py::arg("top_k"), py::arg("renormalize"), py::arg("stream"));
  m.def("sort_routes_cast", &sort_routes_cast, py::arg("raw"), py::arg("n_experts"), py::arg("top_k"),
        py::arg("keys"), py::arg("op_id"), py::arg("want_t"), py::arg("want_n"), py::arg("layout"),
        py::arg("stream"), py::arg("counted_ws") = py::none());
  m.def("cast_keys", &cast_keys, py::arg("keys"), py::arg("op_id"), py::arg("want_t"), py::arg("want_n"),
        py::arg("layout"), py::arg("stream"));
  m.def("forward", &forward_py);
  m.def("forward_gelu", &forward_gelu);
  m.def("gelu_backward", &gelu_backward, py::arg("grad"), py::arg("pre_act"), py::arg("stream"));
  m.def("backward", &backward_py);
  m.def("cvmm_apply", &cvmm_apply);
  // operand rules, exposed for tests
  m.def("storage_for", [](const Tensor& t, int64_t op_id) { return storage_for(t, dtype_of(op_id)); });
  m.def("keys_view", &keys_view);
}
