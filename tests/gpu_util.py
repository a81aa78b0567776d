"""Helpers for the GPU parity tests: run the HIP path the way the reference
harness drives cvmm (benchmark_correctness_original.py:202-214) and compare
with the CPU oracle."""
from __future__ import annotations

import numpy as np
import torch

import cvmm_codex_amd.api as C
from oracle import cvmm_oracle as O

TORCH_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
NP_NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def to_np(t):
    if t is None:
        return None
    return t.detach().float().cpu().numpy()


def norm_rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max(initial=0.0) / max(np.abs(b).max(initial=0.0), 1e-30))


def run_hip(x, keys, sel, weights, grad_out, route_input, amp, amp_dtype=torch.bfloat16, prepare=None):
    """x/keys/sel/weights/grad_out: CPU tensors in their storage dtypes."""
    dev = torch.device("cuda")
    xd = x.to(dev).detach().requires_grad_(True)
    kd = keys.to(dev).detach().requires_grad_(True)
    sd = sel.to(dev)
    wd = None if weights is None else weights.to(dev).detach().requires_grad_(True)
    sel_obj = (prepare or C.cvmm_prepare_sel2)(sd, wd, route_input=route_input)
    with torch.autocast(device_type="cuda", dtype=amp_dtype, enabled=amp):
        out = C.cvmm(xd, sel_obj, kd)
    out.backward(grad_out.to(dev).to(out.dtype))
    torch.cuda.synchronize()
    return {"out": out.detach(), "x_grad": xd.grad, "keys_grad": kd.grad,
            "weights_grad": None if wd is None else wd.grad}


def run_oracle(x, keys, sel, weights, grad_out, route_input, amp, amp_dtype="bfloat16",
               compute=np.float64, need_x=True, need_w=True):
    op = amp_dtype if amp else "float32"
    xn, kn = to_np(x), to_np(keys)
    wn = to_np(weights)
    meta = O.prepare_sel2(sel.numpy(), wn, route_input=route_input)
    out = O.forward(xn, meta, kn, op, op, compute=compute) if need_x else None
    gy = O.rnd(to_np(grad_out), op, compute)
    dx, dw, dg = O.backward(xn, meta, kn, gy, op, x_dtype=NP_NAME[x.dtype], keys_dtype=NP_NAME[keys.dtype],
                            w_dtype=None if weights is None else NP_NAME[weights.dtype], compute=compute,
                            need_x=need_x, need_w=need_w)
    return {"out": out, "x_grad": dx, "keys_grad": dw, "weights_grad": dg}


def compare(got, exp, tol, names=("out", "x_grad", "keys_grad", "weights_grad")):
    errs = {}
    for n in names:
        if exp.get(n) is None:
            assert got.get(n) is None, n
            continue
        g = to_np(got[n])
        assert g.shape == tuple(exp[n].shape), (n, g.shape, exp[n].shape)
        assert np.isfinite(g).all(), n
        errs[n] = norm_rel(g, exp[n])
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"parity failed (tol {tol}): {errs}"
    return errs
