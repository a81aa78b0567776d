"""CPU oracle for the router -- TEST INFRASTRUCTURE ONLY.

Restates, in numpy, the router lines the reference's MoE callers run before
``cvmm`` (benchmark_ffn_moe.py:91-97, benchmark_framework_moe.py:129-135):

    probs = torch.softmax(logits.float(), dim=-1)
    weights, sel = probs.topk(k, dim=-1)
    weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)
    sel_up = cvmm_prepare_sel2(sel)

and their gradient with respect to the logits.  Only ``tests/`` may import it;
the product package never does.

Numerics: ``compute`` precision (float64 by default).  The top-k order is
probability descending with ties to the lower expert id (a stable sort of
-probs).  The sorted selector comes from ``cvmm_oracle.prepare_sel2``.

Pinning (``tests/test_oracle.py``): the forward against torch's own CPU
``softmax`` / ``topk`` / ``sum`` / ``clamp_min`` on the same logits (library
routines), the backward against torch autograd through those lines, the
renormalised weights against the closed form (rows sum to 1), and the sorted
selector against ``prepare_sel2`` of torch's ids.  No function here is
"parity unpinned".
"""
from __future__ import annotations

import numpy as np

from .cvmm_oracle import prepare_sel2

__all__ = ["softmax", "route_topk", "route_topk_backward"]


def softmax(logits: np.ndarray, compute=np.float64) -> np.ndarray:
    """torch.softmax(logits.float(), -1) (benchmark_ffn_moe.py:92)."""
    l = np.asarray(logits, dtype=compute)
    e = np.exp(l - l.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def route_topk(logits: np.ndarray, k: int, renormalize: bool = True, compute=np.float64):
    """(weights [..., k], sel [..., k] int64, Sel of prepare_sel2(sel)):
    benchmark_ffn_moe.py:92-95."""
    p = softmax(logits, compute)
    order = np.argsort(-p, axis=-1, kind="stable")[..., :k]          # :93, ties to the lower id
    w = np.take_along_axis(p, order, axis=-1)
    if renormalize:                                                  # :94
        w = w / np.maximum(w.sum(axis=-1, keepdims=True), 1e-20)
    sel = order.astype(np.int64)
    return w, sel, prepare_sel2(sel)                                 # :95


def route_topk_backward(logits: np.ndarray, sel: np.ndarray, grad_w: np.ndarray, renormalize: bool = True,
                        compute=np.float64) -> np.ndarray:
    """d loss / d logits for the lines above, given d loss / d weights:
    g = d loss / d probs is non-zero at the chosen experts (topk's backward
    scatters), with renormalised weights w = p_sel / S:
    g_sel = (dw - sum(dw * w)) / S (S clamped at 1e-20: a constant there);
    then the softmax backward d l = p * (g - sum(g * p))."""
    p = softmax(logits, compute)
    ps = np.take_along_axis(p, sel, axis=-1)
    dw = np.asarray(grad_w, dtype=compute)
    if renormalize:
        S = ps.sum(axis=-1, keepdims=True)
        Sc = np.maximum(S, 1e-20)
        w = ps / Sc
        gs = np.where(S < 1e-20, dw / Sc, (dw - (dw * w).sum(axis=-1, keepdims=True)) / Sc)
    else:
        gs = dw
    g = np.zeros_like(p)
    np.put_along_axis(g, sel, gs, axis=-1)
    return p * (g - (g * p).sum(axis=-1, keepdims=True))
