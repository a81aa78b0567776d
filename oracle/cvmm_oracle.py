"""CPU oracle for CVMM -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, what the reference's CVMM path computes
(RobertCsordas/cvmm_codex, ``cvmm.py``).  It is the checker the HIP path is
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
``cvmm_codex_amd`` never does, and has no CPU fallback.

Numerics: every matmul is carried out in ``compute`` precision (float64 for the
parity checks, float32 for the CPU baseline timing).  The reference rounds to
the autocast dtype at fixed points (operands cast in-register to the op dtype,
per-route results stored in the output dtype, ...); ``op``/``out`` name those
dtypes and :func:`rnd` applies the same round-to-nearest-even at the same
points.  ``op=None`` disables every rounding point (exact mathematics), which is
what the golden fixtures pin.

Pinning (how each function is checked, see ``tests/test_oracle.py``):
  * prepare_sel / prepare_sel2 / expert_offsets: against brute-force Python
    sorting, ``numpy.bincount`` cumulative sums and the reference test's own
    ``unique_consecutive`` fallback (test_cvmm_correctness.py:73-86), and the
    reused-selector identity (test_cvmm_correctness.py:121-137).
  * forward / backward: against golden fixtures whose expected values come
    from the reference's *einsum* definition (test_cvmm_correctness.py:7-15)
    differentiated by torch autograd in float64 -- an independent formulation
    (materialised ``keys[sel]`` instead of sort/gather/matmul) -- plus
    pure-Python triple loops on tiny inputs, top-1 == dense per-token GEMM,
    E == 1 == plain GEMM, and empty experts => zero weight gradient.
  * rounding emulation (bf16/f16): against torch's own dtype conversions.
  * gelu / gelu_backward (the GELU the reference's callers apply to the up
    projection, benchmark_ffn_moe.py:96): against torch's F.gelu and its
    autograd in float64, and the derivative against central differences.
No function here is "parity unpinned".
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

__all__ = [
    "Sel", "rnd", "prepare_sel", "prepare_sel2", "expert_offsets",
    "forward", "backward", "bf16_bits_to_f32", "f32_to_bf16_bits", "gelu", "gelu_backward",
]


# ----------------------------------------------------------------------------
# dtype helpers
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round-to-nearest-even, NaN -> quiet NaN."""
    a32 = np.ascontiguousarray(a, dtype=np.float32)
    u = a32.view(np.uint32)
    # uint32 arithmetic: only NaN bit patterns can wrap, and those are replaced
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a32)
    if nan.any():
        r = r.copy()
        r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rnd(a: np.ndarray, dtype: Optional[str], compute=np.float64) -> np.ndarray:
    """Round ``a`` to storage dtype ``dtype`` and return it in ``compute``.

    ``dtype`` is one of None (no rounding), "float64", "float32", "bfloat16",
    "float16".  Values are first rounded to float32 (the reference accumulates
    and converts from float32 registers), then to the 16-bit type with RNE.
    """
    if dtype is None or dtype == "float64":
        return np.asarray(a, dtype=compute)
    a32 = np.asarray(a, dtype=np.float32)
    if dtype == "float32":
        out = a32
    elif dtype == "bfloat16":
        out = bf16_bits_to_f32(f32_to_bf16_bits(a32))
    elif dtype == "float16":
        with np.errstate(over="ignore"):
            out = a32.astype(np.float16).astype(np.float32)
    else:
        raise ValueError(f"unknown dtype {dtype!r}")
    return out.astype(compute, copy=False)


# ----------------------------------------------------------------------------
# selector metadata (cvmm.py:12-27, cvmm.py:1786-1803, cvmm.py:68-78)
# ----------------------------------------------------------------------------

@dataclass
class Sel:
    """Numpy mirror of ``CVMMSel`` (cvmm.py:12-21)."""
    raw_sel: np.ndarray
    sel: np.ndarray
    sel_index: np.ndarray
    out_index: Optional[np.ndarray] = None
    reduction_weight: Optional[np.ndarray] = None


def _stable_sort(fsel: np.ndarray):
    # cvmm.py:1797 calls ``fsel.sort()``; tie order there is unspecified, the
    # canonical (and our HIP) order is the stable one.
    perm = np.argsort(fsel, kind="stable").astype(np.int64)
    return fsel[perm], perm


def prepare_sel(sel: np.ndarray, n_experts: int) -> Sel:
    """cvmm.py:24-27: flatten -> int32 -> sort; sel_index = permutation."""
    fsel = np.asarray(sel).reshape(-1).astype(np.int32)
    ssel, perm = _stable_sort(fsel)
    shape = np.asarray(sel).shape
    return Sel(fsel.reshape(shape), ssel.reshape(shape), perm, None)


def prepare_sel2(sel, w: Optional[np.ndarray] = None, route_input: bool = False) -> Sel:
    """cvmm.py:1786-1803 (including the reuse branch at :1788-1792)."""
    if isinstance(sel, Sel):
        if route_input:
            route_index = sel.out_index if sel.out_index is not None else sel.sel_index
            return Sel(sel.raw_sel, sel.sel, route_index, None, w)
        return Sel(sel.raw_sel, sel.sel, sel.sel_index, sel.out_index, w)
    sel = np.asarray(sel)
    k = sel.shape[-1]
    fsel = sel.reshape(-1).astype(np.int32)
    ssel, perm = _stable_sort(fsel)
    if route_input:
        return Sel(fsel.reshape(sel.shape), ssel.reshape(sel.shape), perm, None, w)
    return Sel(fsel.reshape(sel.shape), ssel.reshape(sel.shape), perm // k, perm, w)


def expert_offsets(sorted_sel: np.ndarray, n_experts: int) -> np.ndarray:
    """cvmm.py:315-335 / :1108-1120: offsets[e] = #{i : sorted[i] <= e} (int64).

    Restated as the upper-bound binary search the reference kernel performs.
    """
    s = np.asarray(sorted_sel).reshape(-1)
    return np.searchsorted(s, np.arange(n_experts), side="right").astype(np.int64)


# ----------------------------------------------------------------------------
# forward (cvmm.py:1524-1550 + cvmm_kernel cvmm.py:101-243)
# ----------------------------------------------------------------------------

def _route_rows(meta: Sel):
    """Per sorted route: the route position (output row / weight index)."""
    return meta.out_index if meta.out_index is not None else meta.sel_index


def _grouped(meta: Sel, n_experts: int):
    """Yield (expert, slice of sorted positions) for every non-empty expert."""
    ssel = np.asarray(meta.sel).reshape(-1)
    offs = expert_offsets(ssel, n_experts)
    start = 0
    for e in range(n_experts):
        end = int(offs[e])
        if end > start:
            yield e, slice(start, end)
        start = end


def forward(x, meta: Sel, keys, op: Optional[str] = None, out: Optional[str] = None,
            compute=np.float64) -> np.ndarray:
    """Forward of ``CVMM`` (cvmm.py:1524-1550).

    y[rp(i)] = rnd_out( rnd_op(x[sel_index[i]]) @ rnd_op(keys[sel[i]]) ) for every
    expert-sorted route i, where rp = out_index (token input) or sel_index
    (route input) -- the kernel's store at cvmm.py:224-243.  With a reduction
    weight the per-route results are combined per token:
    out = rnd_out( rnd_out(w)[..., None, :] @ y ) (cvmm.py:1543-1545).
    """
    n_experts, din, dout = keys.shape
    xf = np.asarray(x).reshape(-1, din)
    xr = rnd(xf, op, compute)
    kr = rnd(keys, op, compute)
    R = meta.sel.size
    y = np.zeros((R, dout), dtype=compute)
    rp = _route_rows(meta)
    for e, sl in _grouped(meta, n_experts):
        y[rp[sl]] = xr[meta.sel_index[sl]] @ kr[e]
    y = rnd(y, out, compute).reshape(*meta.sel.shape, dout)
    if meta.reduction_weight is None:
        return y
    w = rnd(meta.reduction_weight, out, compute)
    yk = y.reshape(*meta.reduction_weight.shape, dout)
    res = (w[..., None, :] @ yk)[..., 0, :]
    return rnd(res, out, compute)


# ----------------------------------------------------------------------------
# backward (cvmm.py:1552-1755 and the kernels it dispatches to)
# ----------------------------------------------------------------------------

def backward(x, meta: Sel, keys, grad_out, op: Optional[str] = None,
             x_dtype: Optional[str] = None, keys_dtype: Optional[str] = None,
             w_dtype: Optional[str] = None, compute=np.float64,
             need_x: bool = True, need_w: bool = True):
    """Gradients (grad_x, grad_keys, grad_reduction_weight) of ``CVMM``.

    Which kernel the reference uses depends on the selector layout
    (cvmm.py:1571-1753); the rounding points per path are:

    * token input, unweighted, top_k > 1 (grouped path, cvmm.py:1141-1225):
      dW[e] = sum_i rnd_op(x[tok_i])^T rnd_op(dY[rp_i]) (fp32 -> keys dtype);
      per-route dX_r = rnd_x(rnd_op(dY_r) @ rnd_op(W_e)^T), summed over top-k
      (torch ``.sum`` in the x dtype, cvmm.py:1223).
    * unweighted, route input or top_k == 1 (kernel3 + generic path,
      cvmm.py:1654-1667, :1727-1753): dX[rp] = rnd_x(dY[rp] @ W_e^T).
    * weighted, route input (cvmm.py:1341-1433, kernels :541-604, :1008-1105):
      G_r = rnd_op(rnd_op(dY[tok]) * rnd_op(w_r)); dW[e] = sum rnd_op(x_r)^T G_r;
      g_r = rnd_op(dY[tok] @ W_e^T); dX_r = rnd_x(rnd_op(g_r * rnd_op(w_r)));
      dgate_r = <g_r, x_r> in fp32.
    * weighted, token input (generic path, cvmm.py:1687-1753):
      g_r = rnd_op(dY[tok] @ W_e^T); dX[t] = rnd_op(sum_k rnd_op(w_k) g_k);
      dgate_r = <g_r, x[tok]> in fp32; dW as in the weighted route-input case.
    """
    n_experts, din, dout = keys.shape
    xf = np.asarray(x).reshape(-1, din)
    xr = rnd(xf, op, compute)
    kr = rnd(keys, op, compute)
    R = meta.sel.size
    rp = _route_rows(meta)
    top_k = meta.raw_sel.shape[-1] if meta.raw_sel.ndim > 0 else 1
    rw = meta.reduction_weight
    weighted = rw is not None
    token_input = meta.out_index is not None
    go = np.asarray(grad_out)
    gy = rnd(go.reshape(-1, dout), op, compute)       # dY rows in op dtype

    # -- grad W -------------------------------------------------------------
    dW = np.zeros((n_experts, din, dout), dtype=compute) if need_w else None
    if weighted:
        wf = rnd(np.asarray(rw).reshape(-1), op, compute)
        kdim = rw.shape[-1]
    for e, sl in (_grouped(meta, n_experts) if need_w else ()):
        xs = xr[meta.sel_index[sl]]
        if weighted:
            r = rp[sl]
            g = rnd(gy[r // kdim] * wf[r][:, None], op, compute)
        else:
            g = gy[rp[sl]]
        dW[e] = xs.T @ g
    acc32 = None if op is None else "float32"           # fp32 accumulator buffer
    if need_w:
        dW = rnd(rnd(dW, acc32, compute), keys_dtype, compute)
    if not need_x:
        return None, dW, None

    # -- grad x / grad reduction weight ---------------------------------------
    krT = np.swapaxes(kr, 1, 2)
    dgate = None
    if not weighted:
        per_route = np.zeros((R, din), dtype=compute)
        for e, sl in _grouped(meta, n_experts):
            per_route[rp[sl]] = gy[rp[sl]] @ krT[e]
        per_route = rnd(per_route, x_dtype, compute)
        if token_input and top_k > 1:
            dx = rnd(per_route.reshape(-1, top_k, din).sum(1), x_dtype, compute)
        else:
            dx = per_route
        return dx.reshape(np.asarray(x).shape), dW, None

    kdim = rw.shape[-1]
    g = np.zeros((R, din), dtype=compute)
    for e, sl in _grouped(meta, n_experts):
        g[rp[sl]] = gy[rp[sl] // kdim] @ krT[e]
    g = rnd(g, op, compute)
    wr = rnd(np.asarray(rw).reshape(-1), op, compute)
    x_plain = np.asarray(xf, dtype=compute)          # dgate uses x as stored
    if not token_input:
        dx = rnd(rnd(g * wr[:, None], op, compute), x_dtype, compute)
        dgate = (g * x_plain).sum(-1)
    else:
        gk = g.reshape(-1, kdim, din)
        dx = rnd((wr.reshape(-1, kdim)[:, :, None] * gk).sum(1), op, compute)
        dx = rnd(dx, x_dtype, compute)
        dgate = (gk * x_plain[:, None, :]).sum(-1).reshape(-1)
    dgate = rnd(rnd(dgate, acc32, compute), w_dtype, compute)
    return dx.reshape(np.asarray(x).shape), dW, dgate.reshape(rw.shape)


# ----------------------------------------------------------------------------
# GELU of the up projection (benchmark_ffn_moe.py:96: F.gelu(cvmm(...)))
# ----------------------------------------------------------------------------

def gelu(h: np.ndarray, out: Optional[str] = None, compute=np.float64) -> np.ndarray:
    """rnd_out(0.5 h (1 + erf(h / sqrt 2))): F.gelu (erf form) of the stored
    up-projection values, computed in float and rounded to their dtype."""
    from scipy.special import erf
    x = np.asarray(h, dtype=compute)
    return rnd(0.5 * x * (1.0 + erf(x / np.sqrt(2.0))), out, compute)


def gelu_backward(grad: np.ndarray, h: np.ndarray, out: Optional[str] = None, compute=np.float64) -> np.ndarray:
    """rnd_out(grad * gelu'(h)), gelu'(x) = 0.5 (1 + erf(x / sqrt 2)) +
    x exp(-x^2 / 2) / sqrt(2 pi)."""
    from scipy.special import erf
    x = np.asarray(h, dtype=compute)
    d = 0.5 * (1.0 + erf(x / np.sqrt(2.0))) + x * np.exp(-0.5 * x * x) / np.sqrt(2.0 * np.pi)
    return rnd(np.asarray(grad, dtype=compute) * d, out, compute)
