"""MI355X-native drop-in for the reference's ``cvmm.py`` (RobertCsordas/cvmm_codex).

Same public surface, argument meaning and error behaviour as the reference:
``CVMMSel`` (cvmm.py:12-21), ``cvmm_prepare_sel`` (:24-27),
``cvmm_prepare_sel2`` (:1786-1803), ``cvmm`` (:1759-1783), the autograd
Function ``CVMM`` (:1521-1755), ``get_dtype`` / ``dtype_to_type_id`` (:30-44),
``create_kernels`` and ``_cvmm_expert_offsets`` (:68-78), plus the module
attributes the reference tests patch (``cvmm_expert_offsets_call``,
``cvmm_lowmem_chunk_size``).  ``cvmm_route_topk`` and ``cvmm_gelu`` (no
counterpart in cvmm.py) fuse the router lines its callers write before
``cvmm`` and the GELU they apply to the up projection.

All arithmetic runs in the HIP kernels of ``libcvmm_hip.so`` (C ABI in
``include/cvmm_hip.h``), launched on torch's current stream; nothing here
synchronises with the host.  There is no CPU or PyTorch fallback: CPU operands
and a missing library raise.  (Selectors may be prepared from ids in host
memory, as the reference's pure-torch preparation allows; that makes only the
sorted index metadata.)

Selector sorting is deferred: ``cvmm_prepare_sel2`` takes the int32 copy of
the ids the reference takes (cvmm.py:1796), so later writes to the caller's
``sel`` do not change the routing, and the stable counting sort of that copy
runs when ``cvmm`` first sees the selector, because the sort needs the expert
count, which is ``keys.shape[0]`` and is not an argument of
``cvmm_prepare_sel2``.  Reading ``.sel`` / ``.sel_index`` / ``.out_index``
earlier forces the sort (with the expert count taken from the largest id, one
host sync).
"""
from __future__ import annotations

import os
import threading
from dataclasses import dataclass
from typing import Dict, NamedTuple, Optional, Tuple, Union

import torch

from . import _native as N
from . import compile_ops as _ops


def _compiling() -> bool:
    """Tracing under torch.compile: go through the custom ops (compile_ops)."""
    return torch.compiler.is_compiling()

__all__ = [
    "CVMMSel", "cvmm_prepare_sel", "cvmm_prepare_sel2", "cvmm", "CVMM", "get_dtype",
    "dtype_to_type_id", "create_kernels", "cvmm_expert_offsets", "cvmm_triton_call", "cvmm_route_topk",
    "cvmm_gelu",
]


def _env_on(name: str, default: str = "0") -> bool:
    return os.environ.get(name, default).lower() in ("1", "true", "yes", "on")


# Test hooks with the reference's names (cvmm.py:47-64).  ``cvmm_expert_offsets_call``
# is the native offsets function once create_kernels() ran; setting it to None makes
# _cvmm_expert_offsets use the closed-form torch expression (what the reference's
# test compares against, test_cvmm_correctness.py:73-86).
cvmm_expert_offsets_call = None
cvmm_use_triton_expert_offsets = not _env_on("CVMM_DISABLE_TRITON_EXPERT_OFFSETS")
# Top-k columns per slice of the low-memory grad-input (cvmm.py:62, :80-84,
# :1228-1338): a token-input unweighted top-k sum that goes through the
# [R, d_in] route buffer runs over slices of this many top-k columns, each
# with a buffer of T * chunk rows, summed in fp32 and rounded once (the bits
# of the one-call sum).  0 (the default): all at once, falling back to slices
# when that workspace does not fit in memory.  Read when cvmm() is called.
cvmm_lowmem_chunk_size = int(os.environ.get("CVMM_LOWMEM_CHUNK_SIZE", "0"))
# Sum the top-k terms (weighted forward combine, token-input grad_x) with fp32
# atomics into token rows instead of a route-ordered buffer + ordered row sum.
cvmm_atomic_reduce = _env_on("CVMM_ATOMIC_REDUCE")
# Run the backward's weight gradient on a second stream of the device,
# concurrently with the grad-input and its top-k sum (same kernels, same
# bits): CVMM_OVERLAP_BACKWARD=1.  Off by default: measured on MI355X it
# paid only for the FFN stack (3.72 -> 3.68 ms) and cost the smaller
# projections up to a quarter of their step.  Read when cvmm() is called.
cvmm_overlap_backward = _env_on("CVMM_OVERLAP_BACKWARD", "0")
# Print each new (x.shape, keys.shape) like the reference (cvmm.py:1778-1781);
# on by default as there, CVMM_LOG_SHAPES=0 (or setting this to False) silences it.
cvmm_log_shapes = _env_on("CVMM_LOG_SHAPES", "1")
# The forward primitive as a torch.library op, as the reference exposes
# torch.ops.mylib.cvmm_triton (cvmm.py:1458-1459).
cvmm_triton_call = torch.ops.cvmm_codex_amd.cvmm_triton


def _require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"cvmm_codex_amd: {what} must be a ROCm GPU tensor (there is no CPU fallback)")


# ----------------------------------------------------------------------------
# dtype helpers (cvmm.py:30-44)
# ----------------------------------------------------------------------------

def get_dtype() -> torch.dtype:
    """Op/output dtype: fp32 unless autocast is on (cvmm.py:30-33)."""
    if not torch.is_autocast_enabled("cuda"):
        return torch.float32
    return torch.get_autocast_dtype("cuda")


def dtype_to_type_id(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return 0
    elif dtype == torch.float16:
        return 1
    elif dtype == torch.bfloat16:
        return 2
    raise ValueError("Unknown dtype")


# ----------------------------------------------------------------------------
# native selector preparation
# ----------------------------------------------------------------------------

def _sort_routes(raw_flat: torch.Tensor, n_experts: int, top_k: int, counted_ws=None):
    """Stable counting sort on the device: (sorted int32, perm int64,
    perm // top_k int64, inclusive offsets int64[E]).  `raw_flat` holds int32
    or int64 ids (int64 read as their low 32 bits, like an int32 cast).  The
    inverse permutation (int32) is attached to perm as ``_cvmm_route_pos``: the
    forward/backward calls that receive this perm as their route index use it
    to gather each token's routes."""
    if _compiling():
        ssel, perm, tok, offsets, _ = _ops.sort_routes(raw_flat, n_experts, top_k)
        return ssel, perm, tok, offsets
    ssel, perm, tok, offsets, route_pos = N.host().sort_routes(raw_flat, n_experts, top_k,
                                                               N.stream_of(raw_flat.device), counted_ws)
    perm._cvmm_route_pos = route_pos
    return ssel, perm, tok, offsets


# Weight casts made together with a sort by cvmm(), for the CVMM.forward of
# the same call: (keys, keys._version, op dtype, layout, kt, kn).
_cast_done = threading.local()


class _CopyPlan(NamedTuple):
    """The op-dtype weight copies a call reads.  The routed GEMMs read their K
    dimension with unit stride: kt [E, d_out, d_in] for the forward, kn
    [E, d_in, d_out] for the grad-input.  A top-k sum taken as a dense GEMM
    (cvmm_topk_dense) reads the same orientation with the experts interleaved
    between the rows (kt as [d_out, E, d_in], kn as [d_in, E, d_out]: the
    GEMM's B^T rows).  Under torch.compile tracing the copies stay in the
    routed layouts and a dense sum reads the other copy as [E*K, N] rows
    (`fwd_t` / `bwd_t` say which copy each phase reads)."""
    want_t: bool
    want_n: bool
    layout: int  # N.CAST_*_INTERLEAVED bits
    fwd_t: bool
    bwd_t: bool


def _sort_routes_cast(raw_flat: torch.Tensor, n_experts: int, top_k: int, cast, counted_ws=None):
    """_sort_routes plus the step's weight cast in the same launches
    (`cast` = (keys, op dtype, _CopyPlan)); the copies are left for
    CVMM.forward."""
    keys, op, plan = cast
    (ssel, perm, tok, offsets, route_pos), kt, kn = N.host().sort_routes_cast(
        raw_flat, n_experts, top_k, keys, N.dtype_id(op), plan.want_t, plan.want_n, plan.layout,
        N.stream_of(raw_flat.device), counted_ws)
    perm._cvmm_route_pos = route_pos
    _cast_done.entry = (keys, keys._version, op, plan.layout, kt, kn)
    return ssel, perm, tok, offsets


def _take_cast(keys: torch.Tensor, op: torch.dtype, plan: _CopyPlan):
    """The weight copies cast with this call's sort, if they still match."""
    entry = getattr(_cast_done, "entry", None)
    _cast_done.entry = None
    if entry is None:
        return None
    k, version, eop, layout, kt, kn = entry
    if (k is not keys or version != keys._version or eop != op or layout != plan.layout
            or (plan.want_t and kt is None) or (plan.want_n and kn is None)):
        return None
    return kt, kn


@torch._dynamo.assume_constant_result
def _topk_dense(n_tokens: int, n_experts: int, K: int, N_: int, top_k: int, op_id: int) -> bool:
    """Whether the library takes this top-k sum as one dense GEMM
    (cvmm_topk_dense: shapes and a cost model; a constant for tracing)."""
    return bool(N.lib().cvmm_topk_dense(n_tokens, n_experts, K, N_, top_k, op_id))


def _plan_copies(keys: torch.Tensor, op: torch.dtype, n_routes: int, top_k: int, weighted: bool,
                 token_input: bool, need_grad_input: bool) -> _CopyPlan:
    """The copies of this call (_CopyPlan)."""
    E, d_in, d_out = keys.shape
    op_id = N.dtype_id(op)
    T = n_routes // top_k if top_k > 0 else 0
    fwd_dense = weighted and top_k >= 2 and not cvmm_atomic_reduce and _topk_dense(T, E, d_in, d_out, top_k, op_id)
    bwd_dense = (need_grad_input and not weighted and token_input and top_k >= 2 and not cvmm_atomic_reduce
                 and _topk_dense(T, E, d_out, d_in, top_k, op_id))
    if _compiling():
        fwd_t, bwd_t = not fwd_dense, bwd_dense
        return _CopyPlan(fwd_t or (need_grad_input and bwd_t), (not fwd_t) or (need_grad_input and not bwd_t),
                         0, fwd_t, bwd_t)
    return _eager_plan(d_in, d_out, fwd_dense, bwd_dense, need_grad_input)


def _eager_plan(d_in: int, d_out: int, fwd_dense: bool, bwd_dense: bool, need_grad_input: bool) -> _CopyPlan:
    """Eager copies: one copy where one product runs the long-K routed GEMM
    (K > 128), which reads the weights in either orientation, and the other
    product needs that copy's own orientation (the short-K kernel's, or a
    dense top-k sum's interleaved rows); else kt for the forward and kn for
    the grad-input."""
    layout = (N.CAST_T_INTERLEAVED if fwd_dense else 0) | (N.CAST_N_INTERLEAVED if bwd_dense else 0)
    if not need_grad_input:
        return _CopyPlan(True, False, layout, True, False)
    fwd_ring = d_in > 128 and not fwd_dense
    bwd_ring = d_out > 128 and not bwd_dense
    if fwd_ring:       # kn only: the forward reads it n-contiguous
        return _CopyPlan(False, True, layout, False, False)
    if bwd_ring:       # kt only: the grad-input reads it n-contiguous
        return _CopyPlan(True, False, layout, True, True)
    return _CopyPlan(True, True, layout, True, False)


def _copy_view(plan: _CopyPlan, kt, kn, fwd: bool):
    """(copy, is_t) for the host call of the forward (`fwd`) or the
    grad-input: an interleaved copy goes as its logical [E, d_in, d_out]
    view (is_t False); a routed-layout copy as it is."""
    is_t = plan.fwd_t if fwd else plan.bwd_t
    copy = kt if is_t else kn
    if copy is None:
        return None, is_t
    if is_t and plan.layout & N.CAST_T_INTERLEAVED:
        return copy.permute(1, 2, 0), False   # [d_out, E, d_in] -> [E, d_in, d_out]
    if not is_t and plan.layout & N.CAST_N_INTERLEAVED:
        return copy.permute(1, 0, 2), False   # [d_in, E, d_out] -> [E, d_in, d_out]
    return copy, is_t


def cvmm_expert_offsets(sorted_experts: torch.Tensor, n_experts: int) -> torch.Tensor:
    """Native offsets: out[e] = #{i : sorted[i] <= e} (cvmm.py:1108-1120)."""
    if _compiling():
        return _ops.expert_offsets(sorted_experts.reshape(-1).to(torch.int32), n_experts)
    return N.host().expert_offsets(sorted_experts, n_experts, N.stream_of(sorted_experts.device))


def _cvmm_expert_offsets(sorted_experts: torch.Tensor, n_experts: int) -> torch.Tensor:
    """cvmm.py:68-78."""
    if cvmm_use_triton_expert_offsets and cvmm_expert_offsets_call is not None and sorted_experts.is_cuda:
        return cvmm_expert_offsets_call(sorted_experts, n_experts)
    unique_experts, counts = torch.unique_consecutive(sorted_experts, return_counts=True)
    if unique_experts.numel() == n_experts:
        return counts.cumsum(0)
    expert_counts = torch.zeros((n_experts,), device=sorted_experts.device, dtype=counts.dtype)
    expert_counts[unique_experts.long()] = counts
    return expert_counts.cumsum(0)


def _offsets_for(sel: torch.Tensor, n_experts: int) -> torch.Tensor:
    """Per-expert offsets of a sorted selector, cached on the tensor object."""
    if _compiling():
        return cvmm_expert_offsets(sel, n_experts)
    cache: Optional[Dict[int, torch.Tensor]] = getattr(sel, "_cvmm_offsets", None)
    if cache is not None and n_experts in cache:
        return cache[n_experts]
    off = cvmm_expert_offsets(sel, n_experts)
    try:
        if cache is None:
            cache = {}
            sel._cvmm_offsets = cache
        cache[n_experts] = off
    except (AttributeError, RuntimeError):
        pass
    return off


# The expert count the last sort of a selection of (routes, top_k) used:
# cvmm_prepare_sel2 builds the sort's histogram for it together with the id
# copy (cvmm_copy_ids_count), and the sort skips that launch when cvmm()
# brings the same count.
_expert_guess: Dict[Tuple[int, int], int] = {}


class _Routing:
    """One recorded selection; sorted on the device on first use, per expert count.
    `counted` = (expert count, sort workspace holding the ids' histogram for it)."""

    def __init__(self, raw_flat: torch.Tensor, top_k: int, counted=None):
        self.raw = raw_flat
        self.k = top_k
        self.by_e: Dict[int, Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]] = {}
        self.first_e: Optional[int] = None
        self.counted = counted

    def get(self, n_experts: int, cast=None):
        hit = self.by_e.get(n_experts)
        if hit is None:
            ws = None
            if self.counted is not None:   # one use: the sort turns the counts into prefixes
                ws = self.counted[1] if self.counted[0] == n_experts else None
                self.counted = None
            if not _compiling():
                if len(_expert_guess) > 64:
                    _expert_guess.clear()
                _expert_guess[(self.raw.numel(), self.k)] = n_experts
            hit = (_sort_routes_cast(self.raw, n_experts, self.k, cast, ws) if cast is not None
                   else _sort_routes(self.raw, n_experts, self.k, ws))
            self.by_e[n_experts] = hit
            if self.first_e is None:
                self.first_e = n_experts
        return hit

    def default(self):
        if self.first_e is None:
            n = int(self.raw.max().item()) + 1 if self.raw.numel() else 1   # host sync
            self.get(max(n, 1))
        return self.by_e[self.first_e]


@dataclass(init=False)
class CVMMSel:
    """Selector metadata (cvmm.py:12-21): the same dataclass fields, constructor
    and clone(), so ``dataclasses.fields``/``replace``/``asdict`` work as on the
    reference's selector.

    Instances made by cvmm_prepare_sel2 hold a snapshot of the ids and sort it
    lazily: ``sel``/``sel_index``/``out_index`` resolve on first read (see the
    module docstring); instances built directly are plain records.
    """

    raw_sel: torch.Tensor
    sel: torch.Tensor
    sel_index: torch.Tensor
    out_index: Optional[torch.Tensor] = None
    reduction_weight: Optional[torch.Tensor] = None

    def __init__(self, raw_sel: torch.Tensor, sel: torch.Tensor, sel_index: torch.Tensor,
                 out_index: Optional[torch.Tensor] = None, reduction_weight: Optional[torch.Tensor] = None):
        # the fields' backing attributes (the fields are properties, below)
        self._raw_sel = raw_sel
        self._raw_src = None
        self._sel = sel
        self._sel_index = sel_index
        self._out_index = out_index
        self.reduction_weight = reduction_weight
        self._routing = None
        self._route_mode = False

    def clone(self) -> "CVMMSel":
        if self._pending():
            return CVMMSel._deferred(self._raw_shape_tensor(), self._routing, self._route_mode,
                                     self.reduction_weight)
        return CVMMSel(self.raw_sel, self.sel, self.sel_index, self.out_index, self.reduction_weight)

    @classmethod
    def _deferred(cls, raw_src: torch.Tensor, routing: "_Routing", route_mode: bool, w) -> "CVMMSel":
        """`raw_src`: the ids as given (any integer dtype); the int32 tensor
        the reference stores as raw_sel is made only if it is read."""
        s = cls(None, None, None, None, w)
        s._raw_src = raw_src
        s._routing = routing
        s._route_mode = route_mode
        return s

    def _raw_shape_tensor(self) -> torch.Tensor:
        """A tensor of raw_sel's shape without forcing the int32 copy (the
        autograd function only reads its shape)."""
        if self._raw_sel is None and self._raw_src is not None:
            return self._raw_src
        return self._raw_sel

    def _pending(self) -> bool:
        return self._routing is not None and self._sel is None

    def _resolve(self, n_experts: Optional[int] = None, cast=None) -> None:
        if not self._pending():
            return
        r = self._routing
        ssel, perm, tok, offsets = r.get(n_experts, cast) if n_experts is not None else r.default()
        sel = ssel.view(self._raw_shape_tensor().shape)
        if not _compiling():
            sel._cvmm_offsets = {e: v[3] for e, v in r.by_e.items()}
            sel._cvmm_i32 = ssel
        self._sel = sel
        if self._route_mode:
            self._sel_index, self._out_index = perm, None
        else:
            self._sel_index, self._out_index = tok, perm

    def __repr__(self) -> str:
        if self._pending():
            return (f"CVMMSel(raw_sel={tuple(self._raw_shape_tensor().shape)}, pending sort, "
                    f"route_input={self._route_mode})")
        return (f"CVMMSel(raw_sel={self.raw_sel!r}, sel={self._sel!r}, sel_index={self._sel_index!r}, "
                f"out_index={self._out_index!r}, reduction_weight={self.reduction_weight!r})")


# The dataclass fields above are served by properties: reading sel / sel_index
# / out_index of a deferred selector runs its sort, raw_sel is made on demand.
def _get_raw_sel(self):
    if self._raw_sel is None and self._raw_src is not None:
        src = self._raw_src
        self._raw_sel = src if src.dtype == torch.int32 else src.reshape(-1).to(torch.int32).view(src.shape)
    return self._raw_sel


def _set_raw_sel(self, v):
    self._raw_sel = v
    self._raw_src = None


def _resolved_field(name):
    attr = "_" + name

    def get(self):
        self._resolve()
        return getattr(self, attr)

    def set_(self, v):
        self._resolve()
        setattr(self, attr, v)

    return property(get, set_)


CVMMSel.raw_sel = property(_get_raw_sel, _set_raw_sel)
for _name in ("sel", "sel_index", "out_index"):
    setattr(CVMMSel, _name, _resolved_field(_name))
del _name


def _host_sel(sel: torch.Tensor):
    """A selection held in host memory, prepared with torch ops as the
    reference prepares every selection (cvmm.py:25-26, :1796-1797): the int32
    ids (a copy, so later writes to `sel` change nothing, as on the device),
    their stable sort and its permutation.  Only the metadata is made here;
    cvmm() itself takes GPU tensors."""
    fsel = sel.reshape(-1).to(torch.int32, copy=True)
    ssel, perm = fsel.sort(stable=True)
    return fsel.view(sel.shape), ssel.view(sel.shape), perm


def cvmm_prepare_sel(sel: torch.Tensor, n_experts: int) -> CVMMSel:
    """cvmm.py:24-27: sort the flattened ids; sel_index = sorting permutation."""
    if not sel.is_cuda:
        raw, ssel, perm = _host_sel(sel)
        return CVMMSel(raw, ssel, perm, None)
    ssel, perm, _, offsets = _Routing(sel.reshape(-1), 1).get(n_experts)
    s = ssel.view(sel.shape)
    s._cvmm_offsets = {n_experts: offsets}
    s._cvmm_i32 = ssel
    out = CVMMSel(None, s, perm, None)
    out._raw_src = sel
    return out


def cvmm_prepare_sel2(sel: Union[torch.Tensor, CVMMSel], w: Optional[torch.Tensor] = None,
                      route_input: bool = False) -> CVMMSel:
    """cvmm.py:1786-1803.  Token input: sel_index = perm // top_k, out_index = perm.
    Route input: sel_index = perm, out_index = None.  A CVMMSel argument is
    re-wrapped (route input takes the up-projection's out_index, :1788-1792)."""
    if isinstance(sel, CVMMSel):
        if sel._pending():
            # token-mode parent: out_index = perm; route-mode parent: sel_index = perm
            return CVMMSel._deferred(sel._raw_shape_tensor(), sel._routing, True if route_input else sel._route_mode,
                                     w)
        if route_input:
            route_index = sel.out_index if sel.out_index is not None else sel.sel_index
            out = CVMMSel(None, sel.sel, route_index, None, w)
        else:
            out = CVMMSel(None, sel.sel, sel.sel_index, sel.out_index, w)
        # raw_sel as the parent holds it: its int32 copy is made if it is read
        out._raw_sel, out._raw_src = sel._raw_sel, sel._raw_src
        return out

    n_per_batch = sel.shape[-1]
    if not sel.is_cuda:
        raw, ssel, perm = _host_sel(sel)
        if route_input:
            return CVMMSel(raw, ssel, perm, None, w)
        return CVMMSel(raw, ssel, perm // n_per_batch, perm, w)
    # the reference's `fsel = sel.flatten().to(torch.int32)` (cvmm.py:1796):
    # the routing is fixed here, whatever later happens to `sel`
    if _compiling():
        fsel = sel.reshape(-1)
        fsel = fsel.clone() if fsel.dtype == torch.int32 else fsel.to(torch.int32)
        routing = _Routing(fsel, n_per_batch)
        shaped = fsel.view(sel.shape)
    else:
        guess = _expert_guess.get((sel.numel(), n_per_batch))
        stream = N.stream_of_tensor(sel)
        if guess is not None:
            shaped, ws = N.host().copy_ids_count(sel, guess, stream)
            fsel = shaped.reshape(-1)
            routing = _Routing(fsel, n_per_batch, (guess, ws))
        else:
            shaped = N.host().copy_ids(sel, stream)
            fsel = shaped.reshape(-1)
            routing = _Routing(fsel, n_per_batch)
    out = CVMMSel._deferred(shaped, routing, route_input, w)
    out._raw_sel = shaped
    return out


# ----------------------------------------------------------------------------
# router
# ----------------------------------------------------------------------------

class _RouteTopK(torch.autograd.Function):
    """Eager path of cvmm_route_topk: the native router forward, its native
    backward for the weights' gradient (logits dtype)."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, top_k: int, renormalize: bool):
        w, sel, ssel, perm, tok, offsets, route_pos = N.host().route_topk(logits, top_k, renormalize,
                                                                         N.stream_of(logits.device))
        ctx.save_for_backward(logits, sel)
        ctx.top_k, ctx.renormalize = top_k, renormalize
        ctx.mark_non_differentiable(sel, ssel, perm, tok, offsets, route_pos)
        # no zero tensors for the six id outputs (autograd would fill one per
        # output before every backward): their gradients arrive as None
        ctx.set_materialize_grads(False)
        return w, sel, ssel, perm, tok, offsets, route_pos

    @staticmethod
    def backward(ctx, grad_w, *_):
        logits, sel = ctx.saved_tensors
        if grad_w is None:
            return None, None, None
        g = N.host().route_topk_backward(logits, sel, grad_w.contiguous(), ctx.top_k, ctx.renormalize,
                                         N.stream_of(logits.device))
        return g, None, None


def cvmm_route_topk(logits: torch.Tensor, k: int, renormalize: bool = True):
    """The router lines of the reference's MoE callers in one native call
    (benchmark_ffn_moe.py:91-97, benchmark_framework_moe.py:129-135):

        probs = torch.softmax(logits.float(), dim=-1)
        weights, sel = probs.topk(k, dim=-1)
        weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)   # renormalize
        sel_up = cvmm_prepare_sel2(sel)

    Returns ``(weights, sel, sel_up)``: fp32 weights ``[..., k]`` (gradient
    flows to ``logits``), int64 expert ids ``[..., k]`` in probability order
    (ties to the lower id) and the token-input selector, already sorted
    (``cvmm_prepare_sel2(sel_up, weights, route_input=True)`` gives the
    down-projection selector).  At most 1024 experts and k <= 64.
    """
    _require_device(logits, "logits")
    if logits.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        logits = logits.float()
    E = logits.shape[-1]
    if not (0 < k <= E):
        raise ValueError(f"cvmm_route_topk: k={k} outside 1..{E}")
    lead = logits.shape[:-1]
    if _compiling():
        w, sel, ssel, perm, tok, offsets, route_pos = _ops.route_topk(logits, k, renormalize)
    else:
        w, sel, ssel, perm, tok, offsets, route_pos = _RouteTopK.apply(logits, k, renormalize)
        perm._cvmm_route_pos = route_pos
    sel = sel.view(*lead, k)
    routing = _Routing(sel.reshape(-1), k)
    routing.by_e[E] = (ssel, perm, tok, offsets)
    routing.first_e = E
    return w.view(*lead, k), sel, CVMMSel._deferred(sel, routing, False, None)


def _gate_grad_chunks(n_tokens: int, d_in: int, n_experts: int) -> int:
    """Token chunks of the gate gradient's product: enough [E x D] output
    tiles to fill the GPU (a single [D x T] @ [T x E] product has D*E/8192
    tiles of 128 x 64: 32 at the FFN stack's 2048 x 128), each chunk at least
    1024 tokens; 1 when the tokens do not split evenly."""
    c = 1
    while c < 16 and (d_in * n_experts // 8192) * c * 2 <= 512 and n_tokens % (2 * c) == 0 \
            and n_tokens // (2 * c) >= 1024:
        c *= 2
    return c


class _GateLogits(torch.autograd.Function):
    """logits = x @ gate as autocast computes it (both operands in the op
    dtype, that dtype out; benchmark_ffn_moe.py:91), whose gate gradient
    x^T @ dlogits -- a long-K product with few output tiles -- runs over token
    chunks as one batched product with fp32 partials, summed in chunk order
    and rounded to the op dtype as the single product's output is."""

    @staticmethod
    def forward(ctx, x, gate, op):
        xb, gb = x.to(op), gate.to(op)
        ctx.save_for_backward(xb, gb)
        ctx.dtypes = (x.dtype, gate.dtype)
        return xb @ gb

    @staticmethod
    def backward(ctx, g):
        xb, gb = ctx.saved_tensors
        x_dtype, gate_dtype = ctx.dtypes
        D, E = gb.shape
        g2 = g.to(xb.dtype).reshape(-1, E).contiguous()
        x2 = xb.reshape(-1, D)
        dx = dgate = None
        if ctx.needs_input_grad[0]:
            dx = (g2 @ gb.t().contiguous()).to(x_dtype).view(xb.shape)
        if ctx.needs_input_grad[1]:
            T = x2.shape[0]
            c = _gate_grad_chunks(T, D, E)
            if c == 1:
                dgate = (x2.t() @ g2).to(gate_dtype)
            else:
                # x's chunks as the transposed left operand (no copy); the
                # right operand stays contiguous
                a = x2.contiguous().view(c, T // c, D).transpose(1, 2)   # [c, D, T / c]
                b = g2.view(c, T // c, E)                                  # [c, T / c, E]
                part = torch.bmm(a, b) if a.dtype == torch.float32 else \
                    torch.bmm(a, b, out_dtype=torch.float32)              # [c, D, E] fp32
                dgate = part.sum(0).to(xb.dtype).to(gate_dtype)
        return dx, dgate, None


def cvmm_gate_logits(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """The router's projection of the reference's MoE callers, ``logits = x @
    gate`` (benchmark_ffn_moe.py:91), in the autocast dtype where autocast is
    on (else the promoted dtype): the same forward, input gradient and rounding
    points, with the gate gradient taken over token chunks (one batched
    product instead of a single long-K one whose few output tiles leave most
    CUs idle).  x ``[..., D]``, gate ``[D, E]``; returns ``[..., E]``."""
    _require_device(x, "x")
    _require_device(gate, "gate")
    if gate.dim() != 2 or x.shape[-1] != gate.shape[0]:
        raise ValueError(f"cvmm_gate_logits: x {tuple(x.shape)} and gate {tuple(gate.shape)} do not multiply")
    if torch.is_autocast_enabled("cuda"):
        op = torch.get_autocast_dtype("cuda")
    else:
        op = torch.result_type(x, gate)
    with torch.autocast("cuda", enabled=False):
        return _GateLogits.apply(x, gate, op)


# ----------------------------------------------------------------------------
# launch helpers
# ----------------------------------------------------------------------------

def _storage_for(t: torch.Tensor, op: torch.dtype) -> torch.Tensor:
    """Kernels read fp32 or op-dtype storage; other float types are widened to
    fp32 (exact), which leaves the in-kernel rounding to the op dtype unchanged."""
    return N.host().storage_for(t, N.dtype_id(op))


def _keys_view(keys: torch.Tensor) -> torch.Tensor:
    """keys as they are when one of the two inner strides is 1, else contiguous."""
    return N.host().keys_view(keys)


def _route_pos(rp: Optional[torch.Tensor], n_routes: int) -> Optional[torch.Tensor]:
    """The sort's inverse permutation when `rp` is the perm it returned."""
    if _compiling():
        return None
    pos = getattr(rp, "_cvmm_route_pos", None) if rp is not None else None
    if pos is None or pos.numel() != n_routes or pos.dtype != torch.int32 or pos.device != rp.device:
        return None
    return pos


def _fast_path(op: torch.dtype, d_in: int, d_out: int) -> bool:
    """The DMA-staged kernels need 16-bit operands and widths divisible by 8."""
    return op in (torch.bfloat16, torch.float16) and d_in % 8 == 0 and d_out % 8 == 0


def _flags() -> int:
    """ABI flags in the low 32 bits; bits 32..47: the low-memory slice width."""
    f = N.FLAG_ATOMIC_REDUCE if cvmm_atomic_reduce else 0
    if cvmm_lowmem_chunk_size > 0:
        f |= min(int(cvmm_lowmem_chunk_size), 0xffff) << 32
    if cvmm_overlap_backward:
        f |= N.HOST_OVERLAP_BACKWARD
    return f


def _cast_keys(keys: torch.Tensor, op: torch.dtype, plan: _CopyPlan):
    """keys [E, d_in, d_out] -> the op-dtype copies kt (forward) and kn
    (grad-input) of `plan`, one pass."""
    _require_device(keys, "keys")
    if _compiling():
        kt, kn = _ops.cast_keys(keys, op)
        return kt, kn
    return N.host().cast_keys(keys, N.dtype_id(op), plan.want_t, plan.want_n, plan.layout,
                              N.stream_of(keys.device))


def _forward(x, sel_index, sel, keys, out_index, rw, op_dtype, keys_op=None, keys_op_is_t=True):
    """cvmm_triton (cvmm.py:814-867) + the weighted combine (:1543-1545).
    `keys_op`: an op-dtype weight copy (kt when `keys_op_is_t`, else kn)."""
    _require_device(sel, "sel")
    n_experts = keys.shape[0]
    R = sel.numel()
    if _compiling():
        out = _ops.forward(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index, _offsets_for(sel, n_experts),
                           rw, op_dtype, _flags())
    else:
        out = N.host().forward(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index,
                               _offsets_for(sel, n_experts),
                               _route_pos(out_index if out_index is not None else sel_index, R), rw,
                               N.dtype_id(op_dtype), -1, _flags(), N.stream_of(x.device))
    if rw is None:
        return out.view(*sel.shape, keys.shape[2])
    return out.view(*rw.shape[:-1], keys.shape[2])


def _backward(ctx, grad_output, x, keys, raw_sel, sel, sel_index, out_index, rw,
              need_grad_x, need_grad_keys, need_grad_rw, keys_x=None, keys_x_is_t=False):
    """CVMM.backward's products (cvmm.py:1552-1755).  `keys_x`: the
    grad-input's op-dtype weight copy (kt when `keys_x_is_t`, else kn)."""
    top_k = raw_sel.shape[-1] if raw_sel.ndim > 0 else 1
    R = sel.numel()
    if _compiling():
        g = _ops.backward(grad_output, x, keys, keys_x, keys_x_is_t, sel, sel_index, out_index,
                          _offsets_for(sel, keys.shape[0]), rw, top_k, ctx.op_type, bool(need_grad_x),
                          bool(need_grad_keys), bool(need_grad_rw), _flags())
        return _ops.grads_or_none(g, [bool(need_grad_x), bool(need_grad_keys), bool(need_grad_rw)])
    return N.host().backward(grad_output, x, keys, keys_x, keys_x_is_t, sel, sel_index, out_index,
                             _offsets_for(sel, keys.shape[0]),
                             _route_pos(out_index if out_index is not None else sel_index, R), rw, top_k,
                             N.dtype_id(ctx.op_type), bool(need_grad_x), bool(need_grad_keys), bool(need_grad_rw),
                             _flags(), N.stream_of(x.device))


def _copies_for_call(ctx, keys, op, n_routes, top_k, weighted, token_input, need_grad_input):
    """The forward's weight copy (copy, is_t) for CVMM(.Gelu).forward, the
    grad-input's kept on ctx: cast with the sort when cvmm() did that, else
    here."""
    plan = _plan_copies(keys, op, n_routes, top_k, weighted, token_input, need_grad_input)
    pre = None if _compiling() else _take_cast(keys, op, plan)
    kt, kn = pre if pre is not None else _cast_keys(keys, op, plan)
    ctx.keys_x, ctx.keys_x_is_t = _copy_view(plan, kt, kn, False) if need_grad_input else (None, False)
    return _copy_view(plan, kt, kn, True)


class CVMM(torch.autograd.Function):
    """cvmm.py:1521-1755: forward = routed GEMM (+ weighted top-k combine),
    backward = grad x / grad keys / grad reduction weight."""

    warned = False

    @staticmethod
    def forward(ctx, x: torch.Tensor, raw_sel: torch.Tensor, sel_index: torch.Tensor, sel: torch.Tensor,
                keys: torch.Tensor, out_index: Optional[torch.Tensor] = None,
                reduction_weight: Optional[torch.Tensor] = None):
        ctx.save_for_backward(x, keys, raw_sel, sel, sel_index, out_index, reduction_weight)
        out_type = get_dtype()
        keys_op, fwd_t = None, True
        ctx.keys_x, ctx.keys_x_is_t = None, False
        if _fast_path(out_type, keys.shape[1], keys.shape[2]):
            weighted = reduction_weight is not None
            k = reduction_weight.shape[-1] if weighted else (raw_sel.shape[-1] if raw_sel.ndim > 0 else 1)
            need = ctx.needs_input_grad[0] or ctx.needs_input_grad[6]
            keys_op, fwd_t = _copies_for_call(ctx, keys, out_type, sel.numel(), k, weighted, out_index is not None,
                                              need)
        res = _forward(x, sel_index, sel, keys, out_index, reduction_weight, out_type, keys_op, fwd_t)
        ctx.op_type = out_type
        ctx.keys_type = keys.dtype
        ctx.dtype = out_type
        return res

    @staticmethod
    def backward(ctx, grad_output):
        x, keys, raw_sel, sel, sel_index, out_index, reduction_weight = ctx.saved_tensors
        need_grad_x = ctx.needs_input_grad[0]
        need_grad_keys = ctx.needs_input_grad[4]
        need_grad_rw = ctx.needs_input_grad[6] and reduction_weight is not None
        grad_x, grad_w, grad_rw = _backward(ctx, grad_output, x, keys, raw_sel, sel, sel_index, out_index,
                                            reduction_weight, need_grad_x, need_grad_keys, need_grad_rw,
                                            keys_x=ctx.keys_x, keys_x_is_t=ctx.keys_x_is_t)
        ctx.keys_x = None
        return grad_x, None, None, None, grad_w, None, grad_rw


class CVMMGelu(torch.autograd.Function):
    """F.gelu(CVMM(...)) for unweighted selections: the forward GEMM writes
    gelu(h) and keeps h (its own output) for the backward, which applies the
    GELU derivative natively and then runs CVMM's backward."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, raw_sel: torch.Tensor, sel_index: torch.Tensor, sel: torch.Tensor,
                keys: torch.Tensor, out_index: Optional[torch.Tensor] = None):
        out_type = get_dtype()
        keys_t, is_t = None, True
        ctx.keys_x, ctx.keys_x_is_t = None, False
        if _fast_path(out_type, keys.shape[1], keys.shape[2]):
            k = raw_sel.shape[-1] if raw_sel.ndim > 0 else 1
            keys_t, is_t = _copies_for_call(ctx, keys, out_type, sel.numel(), k, False, out_index is not None,
                                            ctx.needs_input_grad[0])
        n_experts = keys.shape[0]
        R = sel.numel()
        y, h = N.host().forward_gelu(x, keys, keys_t, is_t, sel, sel_index, out_index, _offsets_for(sel, n_experts),
                                     _route_pos(out_index if out_index is not None else sel_index, R),
                                     N.dtype_id(out_type), _flags(), N.stream_of(x.device))
        ctx.save_for_backward(x, keys, raw_sel, sel, sel_index, out_index, h)
        ctx.op_type = out_type
        return y.view(*sel.shape, keys.shape[2])

    @staticmethod
    def backward(ctx, grad_output):
        x, keys, raw_sel, sel, sel_index, out_index, h = ctx.saved_tensors
        gh = N.host().gelu_backward(grad_output, h, N.stream_of(h.device))
        grad_x, grad_w, _ = _backward(ctx, gh.view(grad_output.shape), x, keys, raw_sel, sel, sel_index,
                                      out_index, None, ctx.needs_input_grad[0], ctx.needs_input_grad[4], False,
                                      keys_x=ctx.keys_x, keys_x_is_t=ctx.keys_x_is_t)
        ctx.keys_x = None
        return grad_x, None, None, None, grad_w, None


def cvmm_gelu(x: torch.Tensor, sel: Union[torch.Tensor, CVMMSel], keys: torch.Tensor) -> torch.Tensor:
    """``F.gelu(cvmm(x, sel, keys))`` -- the up projection of the reference's
    MoE callers (benchmark_ffn_moe.py:96) -- with the GELU in the forward
    GEMM's epilogue when that GEMM is the long-K kernel (d_in > 128, 16-bit
    op): the pre-activation is written once, for the backward, instead of
    being read back by a separate GELU pass.  Same results as the
    composition; a weighted selection (or torch.compile tracing) runs the
    composition itself."""
    if not isinstance(sel, CVMMSel):
        sel = cvmm_prepare_sel(sel, keys.shape[0])
    if sel.reduction_weight is not None or _compiling():
        return torch.nn.functional.gelu(cvmm(x, sel, keys))
    create_kernels()
    cast = None
    op = get_dtype()
    if sel._pending() and keys.is_cuda and _fast_path(op, keys.shape[1], keys.shape[2]):
        raw = sel._raw_shape_tensor()
        plan = _plan_copies(keys, op, raw.numel(), raw.shape[-1] if raw.ndim else 1, False,
                            not sel._route_mode, torch.is_grad_enabled() and x.requires_grad)
        cast = (keys, op, plan)
    sel._resolve(keys.shape[0], cast)
    return CVMMGelu.apply(x, sel._raw_shape_tensor(), sel.sel_index, sel.sel, keys, sel.out_index)


known_shapes = set()


def create_kernels() -> None:
    """Load libcvmm_hip.so and the host glue (idempotent); raises if either is missing."""
    global cvmm_expert_offsets_call
    N.host()
    if cvmm_expert_offsets_call is None:
        cvmm_expert_offsets_call = cvmm_expert_offsets


def cvmm(x: torch.Tensor, sel: Union[torch.Tensor, CVMMSel], keys: torch.Tensor) -> torch.Tensor:
    """cvmm.py:1759-1783."""
    if not _compiling():
        return _cvmm_eager(x, sel, keys)
    if not isinstance(sel, CVMMSel):
        sel = cvmm_prepare_sel(sel, keys.shape[0])
    sel._resolve(keys.shape[0])
    _log_shape(x, keys)
    return CVMM.apply(x, sel._raw_shape_tensor(), sel.sel_index, sel.sel, keys, sel.out_index,
                      sel.reduction_weight)


def _log_shape(x: torch.Tensor, keys: torch.Tensor) -> None:
    if cvmm_log_shapes:
        sh = (x.shape, keys.shape)
        if sh not in known_shapes:
            print("New shape:", sh)
            known_shapes.add(sh)


def _cvmm_eager(x: torch.Tensor, sel: Union[torch.Tensor, CVMMSel], keys: torch.Tensor) -> torch.Tensor:
    """cvmm() outside torch.compile tracing: CVMM.apply as one C++ autograd
    function (the host glue's ``cvmm_apply``) with the same forward and
    backward host calls as CVMM.forward / CVMM.backward; its backward node
    runs in the autograd engine without Python (no GIL taken on the engine's
    device thread).  A selection still to be sorted is sorted in the launches
    that also cast this step's weights."""
    if N._host is None:
        create_kernels()
    if not isinstance(sel, CVMMSel):
        sel = cvmm_prepare_sel(sel, keys.shape[0])
    E, d_in, d_out = keys.shape
    op = get_dtype()
    rw = sel.reduction_weight
    weighted = rw is not None
    raw = sel._raw_shape_tensor()
    top_k = raw.shape[-1] if raw.ndim > 0 else 1
    pending = sel._pending()
    plan = None
    if keys.is_cuda and _fast_path(op, d_in, d_out):
        # the eager branch of _plan_copies
        need = torch.is_grad_enabled() and (x.requires_grad or (weighted and rw.requires_grad))
        token_input = (not sel._route_mode) if pending else sel._out_index is not None
        k = rw.shape[-1] if weighted else top_k
        op_id = _DTYPE_IDS[op]
        T = raw.numel() // k if k > 0 else 0
        fwd_dense = weighted and k >= 2 and not cvmm_atomic_reduce and _topk_dense(T, E, d_in, d_out, k, op_id)
        bwd_dense = (need and not weighted and token_input and k >= 2 and not cvmm_atomic_reduce
                     and _topk_dense(T, E, d_out, d_in, k, op_id))
        plan = _eager_plan(d_in, d_out, fwd_dense, bwd_dense, need)
    if pending:
        sel._resolve(E, (keys, op, plan) if plan is not None else None)
    _log_shape(x, keys)
    s, sel_index, out_index = sel._sel, sel._sel_index, sel._out_index
    keys_op = keys_x = None
    fwd_t, keys_x_is_t = True, False
    if plan is not None:
        pre = _take_cast(keys, op, plan)
        kt, kn = pre if pre is not None else _cast_keys(keys, op, plan)
        if need:
            keys_x, keys_x_is_t = _copy_view(plan, kt, kn, False)
        keys_op, fwd_t = _copy_view(plan, kt, kn, True)
    if not s.is_cuda:
        _require_device(s, "sel")
    shape = [*rw.shape[:-1], d_out] if weighted else [*s.shape, d_out]
    rp = out_index if out_index is not None else sel_index
    pos = getattr(rp, "_cvmm_route_pos", None)
    if pos is not None and pos.numel() != s.numel():
        pos = None
    return N._host.cvmm_apply(x, keys, rw, s, sel_index, out_index, _offsets_for(s, E), pos, keys_op, fwd_t,
                              keys_x, keys_x_is_t, top_k, _DTYPE_IDS[op], _flags(), shape)


_DTYPE_IDS = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
