"""Generate the golden CVMM fixtures (tests/golden/cvmm_cases.npz).

Inputs follow the reference's CPU-seeded payload recipe
(benchmark_correctness_original.py:35-43 cases, :45 dtype modes, :98-133
``make_case_payload``, seed = 1234 + case index as at :306), so they are
reproducible without a GPU.

Expected values are NOT produced by ``oracle/``: they come from the reference
test's own einsum definition of CVMM (test_cvmm_correctness.py:7-15, which
materialises ``keys[sel]`` and reduces with broadcasting) evaluated in float64,
with gradients from torch autograd.  That independent formulation is what pins
the oracle's sort/gather/matmul restatement.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
from dataclasses import dataclass, asdict

import numpy as np
import torch


@dataclass(frozen=True)
class Case:
    name: str
    B: int
    T: int
    N: int        # input width  (Din)
    E: int        # output width (Dout)
    K: int        # top-k
    N_E: int      # number of experts
    weighted: bool = False
    route_input: bool = False


# benchmark_correctness_original.py:35-43
CASES = [
    Case("top1_unweighted_masks", 2, 7, 17, 9, 1, 13),
    Case("top3_unweighted", 3, 5, 19, 11, 3, 7),
    Case("weighted_combine", 2, 9, 23, 13, 4, 11, weighted=True),
    Case("weighted_route_input", 2, 8, 29, 17, 4, 9, weighted=True, route_input=True),
    Case("larger_top8_unweighted", 2, 16, 64, 32, 8, 16),
    Case("larger_top8_weighted_route_input", 2, 16, 32, 64, 8, 16, weighted=True, route_input=True),
    Case("many_missing_experts", 1, 5, 15, 10, 2, 32, weighted=True),
]

DTYPE_MODES = ("float32", "bf16_amp", "bf16_params")   # :45


def dtype_for(mode: str, name: str) -> torch.dtype:
    """benchmark_correctness_original.py:85-95."""
    if mode == "float32":
        return torch.float32
    if mode == "bf16_params":
        return torch.bfloat16
    return torch.bfloat16 if name == "x" else torch.float32


def make_payload(case: Case, mode: str, seed: int):
    """Same draw order and scales as make_case_payload (:107-133)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)

    def t(shape, name, scale):
        return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(dtype_for(mode, name))

    x_shape = (case.B, case.T, case.K, case.N) if case.route_input else (case.B, case.T, case.N)
    x = t(x_shape, "x", 0.4)
    keys = t((case.N_E, case.N, case.E), "keys", 0.3)
    sel = torch.randint(0, case.N_E, (case.B, case.T, case.K), generator=g, dtype=torch.int64)
    out_shape = (case.B, case.T, case.E) if case.weighted else (case.B, case.T, case.K, case.E)
    grad_out = t(out_shape, "x", 0.2)
    weights = t((case.B, case.T, case.K), "weights", 0.25) if case.weighted else None
    return x, keys, sel, weights, grad_out


def einsum_reference(x, sel, keys, weights=None):
    """test_cvmm_correctness.py:7-15, evaluated in float64."""
    selected = keys[sel]
    if x.shape[:-1] == sel.shape:
        out = (x.unsqueeze(-1) * selected).sum(dim=-2)
    else:
        out = (x.unsqueeze(-2).unsqueeze(-1) * selected).sum(dim=-2)
    if weights is not None:
        out = (weights.unsqueeze(-1) * out).sum(dim=-2)
    return out


def expected_fp64(x, keys, sel, weights, grad_out):
    xd = x.double().detach().requires_grad_(True)
    kd = keys.double().detach().requires_grad_(True)
    wd = None if weights is None else weights.double().detach().requires_grad_(True)
    out = einsum_reference(xd, sel, kd, wd)
    out.backward(grad_out.double())
    return out.detach(), xd.grad, kd.grad, (None if wd is None else wd.grad)


def to_np(t: torch.Tensor):
    """(array, dtype tag); bf16 is stored as its uint16 bit pattern."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16), "bfloat16"
    return t.numpy(), str(t.dtype).replace("torch.", "")


def main(path: str | None = None) -> str:
    path = path or os.path.join(os.path.dirname(os.path.abspath(__file__)), "cvmm_cases.npz")
    arrays = {}
    for mode in DTYPE_MODES:
        for idx, case in enumerate(CASES):
            x, keys, sel, weights, grad_out = make_payload(case, mode, 1234 + idx)
            out, gx, gk, gw = expected_fp64(x, keys, sel, weights, grad_out)
            p = f"{case.name}__{mode}__"
            for name, tns in (("x", x), ("keys", keys), ("grad_out", grad_out), ("weights", weights)):
                if tns is None:
                    continue
                arr, tag = to_np(tns)
                arrays[p + name] = arr
                arrays[p + name + "_dtype"] = np.array(tag)
            arrays[p + "sel"] = sel.numpy()
            arrays[p + "exp_out"] = out.numpy()
            arrays[p + "exp_x_grad"] = gx.numpy()
            arrays[p + "exp_keys_grad"] = gk.numpy()
            if gw is not None:
                arrays[p + "exp_weights_grad"] = gw.numpy()
    arrays["cases"] = np.array([repr(asdict(c)) for c in CASES])
    np.savez_compressed(path, **arrays)
    return path


if __name__ == "__main__":
    print("wrote", main())
