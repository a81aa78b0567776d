"""cvmm_gelu (F.gelu(cvmm(...)), the up projection of benchmark_ffn_moe.py:96)
on the GPU.

Checked against the composition F.gelu(cvmm(x, sel, keys)) run on the same
GPU, and against the CPU oracle (the projection, the GELU, its derivative and
the projection's backward, each at the reference's rounding points):
  * long-K shapes (d_in > 128), where the GELU runs in the forward GEMM's
    epilogue -- the forward then launches no separate GELU pass;
  * short-K shapes and fp32 (other GEMM kernels: a GELU pass after the GEMM);
  * route-input and token-input selections; a weighted selection falls back
    to the composition;
  * the FFN stack of benchmark_ffn_moe.py:89-98 with cvmm_route_topk and
    cvmm_gelu against the same stack written with torch's router lines and
    F.gelu.
Tolerance 2e-2 of max|b| under bf16 autocast (the rounding points agree; erf
evaluations may differ in the last float bit), 1e-4 in fp32.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cvmm_codex_amd as C
from cvmm_codex_amd import _native as N
from oracle import cvmm_oracle as O
from tests.gpu_util import compare, norm_rel, to_np

pytestmark = pytest.mark.gpu


def _launches(cls, fn):
    lib = N.lib()
    torch.cuda.synchronize()
    lib.cvmm_timing_enable(cls)
    try:
        res = fn()
        torch.cuda.synchronize()
    finally:
        lib.cvmm_timing_enable(0)
    ms, n = ctypes.c_double(), ctypes.c_int64()
    N.check(lib.cvmm_timing_result(cls, ctypes.byref(ms), ctypes.byref(n)), "cvmm_timing_result")
    return res, n.value


def _case(T, k, E, d_in, d_out, route_input, seed, x_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((T, k, d_in) if route_input else (T, d_in)), generator=g).to(x_dtype)
    keys = torch.randn(E, d_in, d_out, generator=g) / d_in ** 0.5
    sel = torch.randint(0, E, (T, k), generator=g)
    gy = torch.randn(T, k, d_out, generator=g)
    return x, keys, sel, gy


def _run(fn, x, keys, sel, gy, route_input, amp):
    xd = x.cuda().requires_grad_(True)
    kd = keys.cuda().requires_grad_(True)
    s = C.cvmm_prepare_sel2(sel.cuda(), route_input=route_input)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
        y = fn(xd, s, kd)
    y.backward(gy.cuda().to(y.dtype))
    torch.cuda.synchronize()
    return {"out": y.detach(), "x_grad": xd.grad, "keys_grad": kd.grad}


def _oracle(x, keys, sel, gy, route_input, amp):
    op = "bfloat16" if amp else "float32"
    xn, kn = to_np(x), to_np(keys)
    meta = O.prepare_sel2(sel.numpy(), None, route_input=route_input)
    h = O.forward(xn, meta, kn, op, op)
    y = O.gelu(h, op if amp else None)
    gh = O.gelu_backward(O.rnd(to_np(gy), op), h, op if amp else None)
    dx, dw, _ = O.backward(xn, meta, kn, gh, op, x_dtype="bfloat16" if x.dtype == torch.bfloat16 else "float32",
                           keys_dtype="float32")
    return {"out": y, "x_grad": dx, "keys_grad": dw}


@pytest.mark.parametrize("T,k,E,d_in,d_out,route_input,amp,fused", [
    (700, 4, 16, 512, 256, False, True, True),     # long K: GELU in the ring GEMM's epilogue
    (300, 2, 8, 1024, 64, True, True, True),       # long K, N <= 64 tiles, route input
    (500, 4, 16, 128, 512, False, True, False),    # short K: panel GEMM + GELU pass
    (257, 3, 7, 96, 80, False, True, False),       # odd widths: tiled GEMM + GELU pass
    (200, 2, 8, 256, 128, False, False, False),    # fp32: GELU pass
])
def test_cvmm_gelu_matches_composition_and_oracle(T, k, E, d_in, d_out, route_input, amp, fused):
    x, keys, sel, gy = _case(T, k, E, d_in, d_out, route_input, seed=T + d_in,
                             x_dtype=torch.bfloat16 if amp else torch.float32)
    got = _run(C.cvmm_gelu, x, keys, sel, gy, route_input, amp)
    ref = _run(lambda a, s, w: F.gelu(C.cvmm(a, s, w)), x, keys, sel, gy, route_input, amp)
    tol = 2e-2 if amp else 1e-4
    compare(got, {n: to_np(v) for n, v in ref.items()}, tol)
    compare(got, _oracle(x, keys, sel, gy, route_input, amp), tol)
    # the forward runs a separate GELU pass only where the GEMM has no epilogue for it
    xd = x.cuda()
    s = C.cvmm_prepare_sel2(sel.cuda(), route_input=route_input)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
        _, n = _launches(N.KC_COMBINE, lambda: C.cvmm_gelu(xd, s, keys.cuda()))
    assert n == (0 if fused else 1)


def _random_cases(n=16, seed=5):
    """Seeded draws: widths around the long-K switch (K > 128) and odd ones,
    route or token input, bf16 autocast or fp32."""
    import numpy as np
    rng = np.random.default_rng(seed)
    widths = (8, 24, 33, 64, 96, 128, 136, 200, 256, 384, 520, 1024)
    out = []
    while len(out) < n:
        T, k = int(rng.integers(1, 1000)), int(rng.integers(1, 9))
        E = int(rng.choice((1, 3, 8, 16, 64)))
        d_in, d_out = (int(rng.choice(widths)) for _ in range(2))
        if T * k * d_in * d_out > 2e8:
            continue
        out.append((T, k, E, d_in, d_out, bool(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("T,k,E,d_in,d_out,route_input,amp", _random_cases())
def test_cvmm_gelu_random_shapes(T, k, E, d_in, d_out, route_input, amp):
    x, keys, sel, gy = _case(T, k, E, d_in, d_out, route_input, seed=3 * T + d_out,
                             x_dtype=torch.bfloat16 if amp else torch.float32)
    got = _run(C.cvmm_gelu, x, keys, sel, gy, route_input, amp)
    ref = _run(lambda a, s, w: F.gelu(C.cvmm(a, s, w)), x, keys, sel, gy, route_input, amp)
    tol = 2e-2 if amp else 1e-4
    compare(got, {n: to_np(v) for n, v in ref.items()}, tol)
    compare(got, _oracle(x, keys, sel, gy, route_input, amp), tol)


def test_cvmm_gelu_weighted_selection_is_the_composition():
    x, keys, sel, _ = _case(100, 3, 8, 256, 64, True, seed=3)
    g = torch.Generator().manual_seed(4)
    w = torch.rand(100, 3, generator=g)
    s = C.cvmm_prepare_sel2(sel.cuda(), w.cuda(), route_input=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        a = C.cvmm_gelu(x.cuda(), s, keys.cuda())
        b = F.gelu(C.cvmm(x.cuda(), s, keys.cuda()))
    assert torch.equal(a, b)


def _ffn(x, gate, w_up, w_down, k, fused):
    """benchmark_ffn_moe.py:89-98 written with the library's fused pieces or
    with torch's router lines and F.gelu."""
    B, T, D = x.shape
    H = w_up.shape[2]
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = x @ gate
        if fused:
            weights, _, sel_up = C.cvmm_route_topk(logits, k, True)
            hidden = C.cvmm_gelu(x, sel_up, w_up)
        else:
            probs = torch.softmax(logits.float(), dim=-1)
            weights, sel = probs.topk(k, dim=-1)
            weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)
            sel_up = C.cvmm_prepare_sel2(sel)
            hidden = F.gelu(C.cvmm(x, sel_up, w_up))
        sel_down = C.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        return C.cvmm(hidden.view(B, T, k, H), sel_down, w_down)


def test_ffn_stack_fused_pieces_match_torch_composition():
    g = torch.Generator().manual_seed(12)
    B, T, D, H, E, k = 2, 512, 512, 256, 32, 4
    x0 = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    gate0 = torch.randn(D, E, generator=g) / D ** 0.5
    up0 = torch.randn(E, D, H, generator=g) / D ** 0.5
    down0 = torch.randn(E, H, D, generator=g) / H ** 0.5
    gy = torch.randn(B, T, D, generator=g)
    res = {}
    for fused in (False, True):
        ts = [t.cuda().requires_grad_(True) for t in (x0, gate0, up0, down0)]
        out = _ffn(*ts, k, fused)
        out.backward(gy.cuda().to(out.dtype))
        torch.cuda.synchronize()
        res[fused] = {"out": out.detach(), "x_grad": ts[0].grad, "gate_grad": ts[1].grad, "up_grad": ts[2].grad,
                      "down_grad": ts[3].grad}
    exp = {n: to_np(v) for n, v in res[False].items()}
    compare(res[True], exp, 2e-2, names=tuple(exp))
