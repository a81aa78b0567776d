"""Router (cvmm_route_topk) on the GPU against the CPU oracle and against the
reference callers' own router lines.

``cvmm_route_topk`` replaces benchmark_ffn_moe.py:92-95 (softmax of the
float logits, top-k, renormalisation, cvmm_prepare_sel2).  Checked here:
  * expert ids equal to the oracle's (probability order, ties to the lower
    id); a row may differ only where two probabilities are within fp32
    rounding of each other (the oracle is float64);
  * weights within 1e-5 of max|weight| (fp32 softmax against float64);
  * the sorted selector bit-exact against the oracle's prepare_sel2 of the
    kernel's own ids (stable sort, offsets, inverse permutation);
  * the logits' gradient against the oracle's closed form (1e-5 of max in
    fp32, 2e-2 in bf16/f16, which the gradient is written in);
  * two runs bit-identical;
  * the FFN stack of benchmark_ffn_moe.py:89-98 with the fused router against
    the same stack with torch's router lines (bf16 autocast, 2e-2).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cvmm_codex_amd as C
from oracle import cvmm_oracle as O
from oracle import router_oracle as RO
from tests.gpu_util import compare, norm_rel, to_np

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
CASES = [  # T, E, k, renormalize, logits dtype
    (16384, 128, 8, True, "bf16"),     # the FFN stack's router (BASELINE C5 shape)
    (1000, 64, 2, False, "f32"),
    (777, 1000, 8, True, "f32"),
    (513, 40, 40, True, "f16"),        # k = E
    (300, 256, 64, True, "bf16"),      # k at its limit
    (5, 3, 1, False, "f32"),
    (1, 100, 7, True, "f32"),
]


def _random_cases(n=16, seed=77):
    """Seeded draws within the router's limits (1..1024 experts, top-k up
    to 64 and at most the expert count)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.integers(1, 1025))
        k = int(rng.integers(1, min(E, 64) + 1))
        out.append((int(rng.integers(1, 5000)), E, k, bool(rng.integers(0, 2)), str(rng.choice(list(DT)))))
    return out


CASES = CASES + _random_cases()


def _logits(T, E, dt, seed):
    g = torch.Generator().manual_seed(seed)
    # a Zipf-like bias makes some experts hot, as in the C5 routing
    bias = 1.5 * torch.log1p(torch.arange(E, 0, -1, dtype=torch.float32))
    return (torch.randn(T, E, generator=g) * 2 + bias).to(DT[dt])


def _check_ids(sel, exp_sel, probs):
    bad = np.nonzero((sel != exp_sel).any(-1))[0]
    for t in bad:  # only near-ties may reorder
        a = probs[t][sel[t]]
        b = probs[t][exp_sel[t]]
        assert np.abs(np.sort(a) - np.sort(b)).max() <= 1e-5 * probs[t].max(), f"token {t}: {sel[t]} vs {exp_sel[t]}"
    assert len(bad) <= max(2, sel.shape[0] // 1000), f"{len(bad)} rows differ"


@pytest.mark.parametrize("T,E,k,renorm,dt", CASES)
def test_router_matches_oracle(T, E, k, renorm, dt):
    logits = _logits(T, E, dt, T + E + k)
    w, sel, sel_up = C.cvmm_route_topk(logits.cuda(), k, renorm)
    torch.cuda.synchronize()
    ln = logits.float().numpy()
    ew, esel, _ = RO.route_topk(ln, k, renorm)
    probs = RO.softmax(ln)
    gsel = sel.cpu().numpy()
    _check_ids(gsel, esel, probs)
    assert w.dtype == torch.float32 and sel.dtype == torch.int64
    assert tuple(w.shape) == (T, k) and tuple(sel.shape) == (T, k)
    # weights: against the oracle's values for the kernel's own ids
    p_sel = np.take_along_axis(probs, gsel, -1)
    ref_w = p_sel / np.maximum(p_sel.sum(-1, keepdims=True), 1e-20) if renorm else p_sel
    assert norm_rel(w.cpu().numpy(), ref_w) <= 1e-5
    # the sorted selector, bit-exact
    meta = O.prepare_sel2(gsel)
    np.testing.assert_array_equal(sel_up.sel.cpu().numpy().reshape(-1), meta.sel.reshape(-1))
    np.testing.assert_array_equal(sel_up.sel_index.cpu().numpy(), meta.sel_index)
    np.testing.assert_array_equal(sel_up.out_index.cpu().numpy(), meta.out_index)
    off = C.api._offsets_for(sel_up.sel, E).cpu().numpy()
    np.testing.assert_array_equal(off, O.expert_offsets(meta.sel.reshape(-1), E))
    pos = sel_up.out_index._cvmm_route_pos.cpu().numpy()
    np.testing.assert_array_equal(pos[meta.out_index], np.arange(T * k))


@pytest.mark.parametrize("T,E,k,renorm,dt", CASES)
def test_router_backward_matches_oracle(T, E, k, renorm, dt):
    logits = _logits(T, E, dt, 7 * T + E).cuda().requires_grad_(True)
    w, sel, _ = C.cvmm_route_topk(logits, k, renorm)
    g = torch.Generator().manual_seed(T + 3)
    gw = torch.randn(T, k, generator=g)
    w.backward(gw.cuda())
    torch.cuda.synchronize()
    assert logits.grad.dtype == logits.dtype
    exp = RO.route_topk_backward(logits.detach().float().cpu().numpy(), sel.cpu().numpy(), gw.numpy(), renorm)
    tol = 1e-5 if dt == "f32" else 2e-2
    assert norm_rel(to_np(logits.grad), exp) <= tol


def test_router_is_deterministic():
    logits = _logits(4096, 128, "bf16", 3).cuda()
    outs = []
    for _ in range(2):
        l = logits.clone().requires_grad_(True)
        w, sel, s = C.cvmm_route_topk(l, 8, True)
        w.backward(torch.ones_like(w))
        outs.append((w.detach(), sel, s.sel, s.sel_index, s.out_index, l.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def _ffn(x, gate, w_up, w_down, k, fused):
    """benchmark_ffn_moe.py:89-98, with the router lines or cvmm_route_topk."""
    B, T, D = x.shape
    H = w_up.shape[2]
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = x @ gate
        if fused:
            weights, _, sel_up = C.cvmm_route_topk(logits, k, True)
        else:
            probs = torch.softmax(logits.float(), dim=-1)
            weights, sel = probs.topk(k, dim=-1)
            weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)
            sel_up = C.cvmm_prepare_sel2(sel)
        hidden = F.gelu(C.cvmm(x, sel_up, w_up))
        sel_down = C.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        return C.cvmm(hidden.view(B, T, k, H), sel_down, w_down)


def test_ffn_stack_with_fused_router_matches_torch_router():
    g = torch.Generator().manual_seed(11)
    B, T, D, H, E, k = 2, 512, 256, 128, 32, 4
    x0 = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    gate0 = torch.randn(D, E, generator=g) / D ** 0.5
    up0 = torch.randn(E, D, H, generator=g) / D ** 0.5
    down0 = torch.randn(E, H, D, generator=g) / H ** 0.5
    gy = torch.randn(B, T, D, generator=g)
    res = {}
    for fused in (False, True):
        x = x0.cuda().requires_grad_(True)
        gate = gate0.cuda().requires_grad_(True)
        up = up0.cuda().requires_grad_(True)
        down = down0.cuda().requires_grad_(True)
        out = _ffn(x, gate, up, down, k, fused)
        out.backward(gy.cuda().to(out.dtype))
        torch.cuda.synchronize()
        res[fused] = {"out": out.detach(), "x_grad": x.grad, "gate_grad": gate.grad, "up_grad": up.grad,
                      "down_grad": down.grad}
    exp = {n: to_np(v) for n, v in res[False].items()}
    compare(res[True], exp, 2e-2, names=tuple(exp))


@pytest.mark.parametrize("T,D,E,amp", [
    (16384, 2048, 128, True),    # the FFN stack's router projection: 16 token chunks
    (4096, 512, 64, True),       # 4 chunks
    (1000, 64, 16, True),        # one product (too few tokens to split)
    (2048, 256, 32, False),      # fp32, no autocast
])
def test_gate_logits_against_the_torch_projection(T, D, E, amp):
    """cvmm_gate_logits(x, gate) is the callers' ``x @ gate``
    (benchmark_ffn_moe.py:91) under autocast: the same logits bit for bit,
    the same input gradient, and the gate gradient -- summed over token
    chunks in fp32 -- within the op dtype's rounding of torch's, and against
    float64."""
    g = torch.Generator().manual_seed(T + D + E)
    xd = torch.randn(T, D, generator=g).to(torch.bfloat16 if amp else torch.float32).cuda()
    gate = (torch.randn(D, E, generator=g) / D ** 0.5).cuda()
    dl = torch.randn(T, E, generator=g).cuda()
    outs = []
    for fn in (lambda a, b: a @ b, C.cvmm_gate_logits):
        x = xd.clone().requires_grad_(True)
        gt = gate.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
            y = fn(x, gt)
        y.backward(dl.to(y.dtype))
        torch.cuda.synchronize()
        outs.append((y.detach(), x.grad, gt.grad))
    (y0, dx0, dg0), (y1, dx1, dg1) = outs
    assert y1.dtype == y0.dtype and dg1.dtype == dg0.dtype and dx1.dtype == dx0.dtype
    assert torch.equal(y1, y0)
    tol = 2e-2 if amp else 1e-4
    assert norm_rel(to_np(dx1), to_np(dx0)) <= tol
    assert norm_rel(to_np(dg1), to_np(dg0)) <= tol
    # float64 restatement of the gate gradient with the op-dtype operands
    xo = xd.double().cpu()
    dlo = dl.to(y0.dtype).double().cpu()
    assert norm_rel(to_np(dg1), (xo.t() @ dlo).numpy()) <= tol
