"""Parity at the full BASELINE.json sizes of C4 (SwitchHead V/O) and C5 (MoE
FFN stack with Zipf-skewed routing), checked on samples.

A full-size oracle run is out of reach for numpy (C4 is 412 GFLOP per step,
C5 1.6 TFLOP), but every quantity the path produces depends on few inputs:
an output row, an input-gradient row and a routing-weight gradient depend
only on their own token's routes, and an expert's weight gradient only on the
routes sent to it.  So the full-size GPU run is compared, element for element,
with oracle runs on sub-problems: a random sample of tokens (all their routes)
and a few experts (all their routes, posed as a one-route-per-row problem with
the same rounding points), the hottest expert of the skewed C5 routing among
them.  Tolerance: max|a - b| / max|b| <= 2e-2 (bf16 autocast), as for the
other configs.

Every token and every expert is covered as well: the torch restatement of
the path (oracle/torch_cpu_path.py, pinned to the golden fixtures) runs in
float32 on the GPU over the whole problem (no rounding points: at 2e-2 the
bf16 roundings are far inside the bound), and every output row, every input
gradient and every expert's weight gradient (each expert on its own scale)
must agree with it.  This is what would catch a scheduling mistake in a tile
or an expert that the samples miss (the token-major tile order and the
coarse weight-gradient tiles only run at these sizes).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cvmm_codex_amd as C
import workloads as W
from oracle import cvmm_oracle as O
from oracle import torch_cpu_path as P
from tests.gpu_util import norm_rel

pytestmark = pytest.mark.gpu

TOL = 2e-2
BF = "bfloat16"


def _np(t):
    return t.detach().float().cpu().numpy()


def _check(name, got, exp):
    err = norm_rel(got, exp)
    assert err <= TOL, f"{name}: max|a-b|/max|b| = {err:.3e}"
    return err


def _token_oracle(x, sel, w, keys, gy, route_input, tokens):
    """Oracle forward / input-side backward on the routes of `tokens`.
    x: [T, d_in] (token input) or [T, k, d_in] (route input), sel [T, k],
    w [T, k] or None, gy [T, k, d_out] (unweighted) or [T, d_out] (weighted)."""
    xs = x[tokens]
    used, local = np.unique(sel[tokens], return_inverse=True)   # only the experts these routes use
    keys = keys[used]
    meta = O.prepare_sel2(local.reshape(sel[tokens].shape), None if w is None else w[tokens],
                          route_input=route_input)
    out = O.forward(xs, meta, keys, BF, BF)
    gys = O.rnd(gy[tokens], BF)
    dx, _, dg = O.backward(xs, meta, keys, gys, BF, x_dtype=BF, keys_dtype="float32",
                           w_dtype=None if w is None else "float32", need_w=False)
    return out, dx, dg


def _expert_oracle(e, x_rows, gy_rows, w_rows, keys):
    """Oracle weight gradient of expert `e` from its routes only, posed as a
    route-input problem with one route per row (the rounding points of the
    grouped and weighted kernels are per route)."""
    n = x_rows.shape[0]
    if n == 0:
        return np.zeros(keys.shape[1:], dtype=np.float64)
    sel = np.zeros((n, 1), dtype=np.int64)              # expert e as the only (local) expert 0
    w = None if w_rows is None else w_rows.reshape(n, 1)
    meta = O.prepare_sel2(sel, w, route_input=True)
    gy = O.rnd(gy_rows.reshape(n, 1, -1) if w is None else gy_rows.reshape(n, -1), BF)
    _, dW, _ = O.backward(x_rows.reshape(n, 1, -1), meta, keys[e:e + 1], gy, BF, x_dtype=BF,
                          keys_dtype="float32", w_dtype=None if w is None else "float32", need_x=False)
    return dW[0]


def _run_projection(p: W.Projection):
    dev = torch.device("cuda")
    x = p.x.to(dev).requires_grad_(True)
    keys = p.keys.to(dev).requires_grad_(True)
    w = None if p.weights is None else p.weights.to(dev).requires_grad_(True)
    s = C.cvmm_prepare_sel2(p.sel.to(dev), w, route_input=p.route_input)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(x, s, keys)
    y.backward(p.grad_out.to(dev).to(y.dtype))
    torch.cuda.synchronize()
    return y, x.grad, keys.grad, None if w is None else w.grad


def _f32(t):
    return None if t is None else t.detach().to(device="cuda", dtype=torch.float32).contiguous()


def _full_check(tag, x, sel, keys, w, gy, route_input, got):
    """All of (out, x_grad, keys_grad, weights_grad) against the torch path in
    float32 on the GPU; keys_grad expert by expert."""
    with torch.no_grad():
        out, (dx, dw, dg) = P.step(_f32(x), sel.cuda(), _f32(keys), _f32(w), _f32(gy), route_input)
    y, gx, gk, gw = got
    errs = {"out": _check(f"{tag}.out", _np(y), _np(out)),
            "x_grad": _check(f"{tag}.x_grad", _np(gx), _np(dx))}
    if dg is not None:
        errs["weights_grad"] = _check(f"{tag}.weights_grad", _np(gw), _np(dg))
    counts = torch.bincount(sel.reshape(-1).cuda(), minlength=keys.shape[0])
    worst = 0.0
    for e in range(keys.shape[0]):
        if counts[e] == 0:
            assert torch.count_nonzero(gk[e]) == 0, f"{tag}.keys_grad[{e}] of an empty expert"
            continue
        a, b = gk[e].float(), dw[e]
        err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
        assert err <= TOL, f"{tag}.keys_grad[{e}] ({int(counts[e])} routes): {err:.3e}"
        worst = max(worst, err)
    errs["keys_grad_worst_expert"] = worst
    del out, dx, dw, dg
    torch.cuda.empty_cache()
    return errs


@pytest.mark.parametrize("dense", [0, 1], ids=["default", "route_buffer"])
@pytest.mark.parametrize("name", ["switch_v_2048", "switch_o_2048_weighted"])
def test_c4_full_size_every_token_and_expert(name, dense):
    """dense=0: the default path (the top-k sums as the dense expert-slot
    GEMM); dense=1: CVMM_TUNE_DENSE_TOPK=1, the hand-written route-buffer
    path (routed GEMM into [R, N] rows, then the ordered top-k row sum)."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    p = W.PROJECTIONS[name]()
    try:
        assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, dense) == 0
        got = _run_projection(p)
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    _full_check(name, p.x, p.sel, p.keys, p.weights, p.grad_out, p.route_input, got)


@pytest.mark.parametrize("name", ["switch_v_2048", "switch_o_2048_weighted"])
def test_c4_full_size_sampled(name):
    p = W.PROJECTIONS[name]()
    y, gx, gk, gw = _run_projection(p)
    k = p.sel.shape[-1]
    d_in, d_out = p.keys.shape[1], p.keys.shape[2]
    sel = p.sel.reshape(-1, k).numpy()
    T = sel.shape[0]
    x = _np(p.x).reshape(T, k, d_in) if p.route_input else _np(p.x).reshape(T, d_in)
    w = None if p.weights is None else _np(p.weights).reshape(T, k)
    gy = _np(p.grad_out).reshape(T, d_out) if w is not None else _np(p.grad_out).reshape(T, k, d_out)
    keys = _np(p.keys)
    rng = np.random.default_rng(17)
    tokens = np.sort(rng.choice(T, size=48, replace=False))
    out, dx, dg = _token_oracle(x, sel, w, keys, gy, p.route_input, tokens)
    _check("out", _np(y).reshape(T, *out.shape[1:])[tokens], out)
    _check("x_grad", _np(gx).reshape(T, *dx.shape[1:])[tokens], dx)
    if w is not None:
        _check("weights_grad", _np(gw).reshape(T, k)[tokens], dg)
    gkn = _np(gk)
    counts = np.bincount(sel.reshape(-1), minlength=keys.shape[0])
    for e in (int(counts.argmax()), int(counts.argmin()), 77):
        t_idx, j_idx = np.nonzero(sel == e)
        xr = x[t_idx, j_idx] if p.route_input else x[t_idx]
        gr = gy[t_idx] if w is not None else gy[t_idx, j_idx]
        wr = None if w is None else w[t_idx, j_idx]
        _check(f"keys_grad[{e}]", gkn[e], _expert_oracle(e, xr, gr, wr, keys))


def test_c5_ffn_stack_full_size_sampled():
    dev = torch.device("cuda")
    s = W.c5_ffn_stack().to(dev)
    B, Tn, D = s.x.shape
    E, _, H = s.w_up.shape
    k = s.k
    x = s.x.clone().requires_grad_(True)
    w_up = s.w_up.clone().requires_grad_(True)
    w_down = s.w_down.clone().requires_grad_(True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        # router on a detached x, so x.grad is the up projection's input gradient
        logits = x.detach() @ s.gate + s.bias
        probs = torch.softmax(logits.float(), dim=-1)
        weights, sel = probs.topk(k, dim=-1)
        weights = (weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)).detach().requires_grad_(True)
        sel_up = C.cvmm_prepare_sel2(sel)
        h_pre = C.cvmm(x, sel_up, w_up)
        h_pre.retain_grad()
        hidden = F.gelu(h_pre)
        hidden.retain_grad()
        sel_down = C.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        y = C.cvmm(hidden.view(B, Tn, k, H), sel_down, w_down)
    y.backward(s.grad_out.to(y.dtype))
    torch.cuda.synchronize()

    T = B * Tn
    seln = sel.reshape(T, k).cpu().numpy()
    counts = np.bincount(seln.reshape(-1), minlength=E)
    assert counts.max() > 10 * counts.mean()            # Zipf-skewed loads, as configured
    xn = _np(x).reshape(T, D)
    wn = _np(weights).reshape(T, k)
    hn = _np(hidden).reshape(T, k, H)
    gy = _np(s.grad_out).reshape(T, D)
    g_h = _np(h_pre.grad).reshape(T, k, H)             # grad into the up projection's output
    wu, wd = _np(w_up), _np(w_down)
    rng = np.random.default_rng(5)
    tokens = np.sort(rng.choice(T, size=32, replace=False))

    # up projection (token input, unweighted)
    out, dx, _ = _token_oracle(xn, seln, None, wu, g_h, False, tokens)
    _check("up.out", _np(h_pre).reshape(T, k, H)[tokens], out)
    _check("up.x_grad", _np(x.grad).reshape(T, D)[tokens], dx)
    # down projection (route input, weighted by the gate)
    out, dx, dg = _token_oracle(hn, seln, wn, wd, gy, True, tokens)
    _check("down.out", _np(y).reshape(T, D)[tokens], out)
    _check("down.x_grad", _np(hidden.grad).reshape(T, k, H)[tokens], dx)
    _check("down.weights_grad", _np(weights.grad).reshape(T, k)[tokens], dg)
    # weight gradients of the hottest, a cold and a middle expert
    gup, gdn = _np(w_up.grad), _np(w_down.grad)
    for e in (int(counts.argmax()), int(np.argsort(counts)[E // 2]), int(counts.argmin())):
        t_idx, j_idx = np.nonzero(seln == e)
        _check(f"w_up.grad[{e}]", gup[e], _expert_oracle(e, xn[t_idx], g_h[t_idx, j_idx], None, wu))
        _check(f"w_down.grad[{e}]", gdn[e],
               _expert_oracle(e, hn[t_idx, j_idx], gy[t_idx], wn[t_idx, j_idx], wd))

    # every token and every expert of both projections
    _full_check("up", x, sel.cpu(), w_up, None, h_pre.grad, False, (h_pre, x.grad, w_up.grad, None))
    _full_check("down", hidden.view(B, Tn, k, H), sel.cpu(), w_down, weights, s.grad_out, True,
                (y, hidden.grad, w_down.grad, weights.grad))


def test_c5_fused_stack_full_size_every_token_and_expert():
    """The path the C5 bench line times, workloads.ffn_forward_fused (the
    router projection cvmm_gate_logits, the native router cvmm_route_topk and
    the up projection with its GELU in the GEMM epilogue, cvmm_gelu), at full
    size.  The router's choice is checked
    to be a top-k of the softmax in probability order; then, with that
    routing, the whole stack is restated in float32 on the GPU (the torch
    path of oracle/torch_cpu_path.py, torch autograd for the gradients,
    router included) and every output row, x and gate gradient, and every
    expert's weight gradients must agree."""
    dev = torch.device("cuda")
    s = W.c5_ffn_stack().to(dev)
    B, Tn, D = s.x.shape
    E, _, H = s.w_up.shape
    k, T = s.k, B * Tn
    x = s.x.clone().requires_grad_(True)
    gate = s.gate.clone().requires_grad_(True)
    w_up = s.w_up.clone().requires_grad_(True)
    w_down = s.w_down.clone().requires_grad_(True)
    y = W.ffn_forward_fused(s, C, x, gate, w_up, w_down)
    y.backward(s.grad_out.to(y.dtype))
    torch.cuda.synchronize()

    # the routing the fused router chose: the same launch on the same logits
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = s.x @ s.gate + s.bias
        w_got, sel, _ = C.cvmm_route_topk(logits, k, True)
    sel = sel.reshape(T, k)
    probs = torch.softmax(logits.float(), dim=-1).reshape(T, E)
    assert float((probs.gather(1, sel) - probs.topk(k, dim=-1).values).abs().max()) <= 1e-6
    counts = torch.bincount(sel.reshape(-1), minlength=E)
    assert counts.max() > 10 * counts.float().mean()          # Zipf-skewed loads, as configured

    # float32 restatement with that routing
    xf = s.x.float().reshape(T, D).clone().requires_grad_(True)
    gf = s.gate.float().clone().requires_grad_(True)
    wuf = s.w_up.float().clone().requires_grad_(True)
    wdf = s.w_down.float().clone().requires_grad_(True)
    pw = torch.softmax(xf @ gf + s.bias.float(), dim=-1).gather(1, sel)
    wr = pw / pw.sum(-1, keepdim=True).clamp_min(1e-20)
    hidden = F.gelu(P.forward(xf, P.Routes(sel, E, False), wuf, None))
    yr = P.forward(hidden, P.Routes(sel, E, True), wdf, wr)
    yr.backward(s.grad_out.float().reshape(T, D))
    torch.cuda.synchronize()

    _check("weights", _np(w_got).reshape(T, k), _np(wr))
    _check("out", _np(y).reshape(T, D), _np(yr))
    _check("x_grad", _np(x.grad).reshape(T, D), _np(xf.grad))
    _check("gate_grad", _np(gate.grad), _np(gf.grad))
    for name, got, exp in (("w_up.grad", w_up.grad, wuf.grad), ("w_down.grad", w_down.grad, wdf.grad)):
        for e in range(E):
            if counts[e] == 0:
                assert torch.count_nonzero(got[e]) == 0, f"{name}[{e}] of an empty expert"
                continue
            a, b = got[e].float(), exp[e]
            err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
            assert err <= TOL, f"{name}[{e}] ({int(counts[e])} routes): {err:.3e}"
