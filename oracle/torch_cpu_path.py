"""PyTorch CPU CVMM path -- TEST INFRASTRUCTURE ONLY (the CPU baseline).

The reference's CVMM computation restated with torch CPU ops in float32 (no
rounding points): stable sort of the routes by expert, per-expert offsets,
then per expert a row gather + ``matmul`` for the forward
(cvmm.py:1524-1550, weighted combine :1543-1545), the grad-input and the
weight gradient, and the reduction-weight gradient (cvmm.py:1552-1755).  This
is what BASELINE.json calls "the reference's PyTorch CPU CVMM path (gather +
per-expert matmul)"; ``bench.py``'s ``cpu_baseline`` leg times it on the host
cores.  It is a checker/baseline only: the product package never imports it.

Pinned in ``tests/test_oracle.py`` against the golden fixtures (the
reference test's einsum definition in float64) on every golden case: token
and route input, weighted, top-1, odd widths, missing experts.  Device
agnostic: the full-size GPU parity tests run it in float32 on the GPU as a
whole-problem reference.
"""
from __future__ import annotations

from typing import Optional

import torch


class Routes:
    """Selector metadata (cvmm.py:1786-1803): stable sort of the flattened ids."""

    def __init__(self, sel: torch.Tensor, n_experts: int, route_input: bool):
        self.shape = tuple(sel.shape)
        fsel = sel.reshape(-1).to(torch.int64)
        self.k = sel.shape[-1]
        self.ssel, self.perm = torch.sort(fsel, stable=True)
        self.route_input = route_input
        # x row per sorted route; route position (output row) per sorted route
        self.x_row = self.perm if route_input else self.perm // self.k
        self.rp = self.perm
        counts = torch.bincount(self.ssel, minlength=n_experts).cpu()
        self.offsets = counts.cumsum(0)
        self.bounds = [(e, int(s), int(t)) for e, (s, t) in enumerate(
            zip(torch.cat([torch.zeros(1, dtype=torch.int64), self.offsets[:-1]]).tolist(), self.offsets.tolist()))
            if t > s]


def forward(x: torch.Tensor, r: Routes, keys: torch.Tensor, w: Optional[torch.Tensor]) -> torch.Tensor:
    """y[rp] = x[x_row] @ keys[e] per expert; weighted: out[t] = sum_j w[t, j] y[t, j]."""
    din, dout = keys.shape[1], keys.shape[2]
    xf = x.reshape(-1, din)
    R = r.ssel.numel()
    y = torch.empty(R, dout, dtype=x.dtype, device=x.device)
    for e, s, t in r.bounds:
        y[r.rp[s:t]] = xf[r.x_row[s:t]] @ keys[e]
    if w is None:
        return y.view(*r.shape, dout)
    return (w.reshape(-1, 1, r.k) @ y.view(-1, r.k, dout)).view(*r.shape[:-1], dout)


def backward(x: torch.Tensor, r: Routes, keys: torch.Tensor, w: Optional[torch.Tensor], gy: torch.Tensor):
    """(grad_x, grad_keys, grad_w): per-expert gathers and matmuls."""
    E, din, dout = keys.shape
    xf = x.reshape(-1, din)
    R = r.ssel.numel()
    g = gy.reshape(-1, dout)
    # dY row of every route: its own row (unweighted) or its token's row scaled by w
    if w is None:
        g_route = g
    else:
        g_route = g.repeat_interleave(r.k, 0) * w.reshape(-1, 1)
    dW = torch.zeros(E, din, dout, dtype=x.dtype, device=x.device)
    per_route = torch.empty(R, din, dtype=x.dtype, device=x.device)
    g_plain = g if w is None else g.repeat_interleave(r.k, 0)
    for e, s, t in r.bounds:
        rows = r.rp[s:t]
        dW[e] = xf[r.x_row[s:t]].T @ g_route[rows]
        per_route[rows] = g_plain[rows] @ keys[e].T
    dw = None
    if w is not None:
        xr = xf if r.route_input else xf.repeat_interleave(r.k, 0)
        dw = (per_route * xr).sum(-1).view(w.shape)
        per_route = per_route * w.reshape(-1, 1)
    if r.route_input:
        dx = per_route
    else:
        dx = per_route.view(-1, r.k, din).sum(1)
    return dx.view(x.shape), dW, dw


def step(x, sel, keys, w, gy, route_input: bool):
    """One selector preparation + forward + backward (what bench.py times)."""
    r = Routes(sel, keys.shape[0], route_input)
    out = forward(x, r, keys, w)
    grads = backward(x, r, keys, w, gy)
    return out, grads
