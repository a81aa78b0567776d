"""Reduce GEMM (top-k sums without the route-ordered buffer) on the GPU.

The weighted forward of a route-input projection (SwitchHead's output
projection, cvmm.py:1543-1545) and the input gradient of a token-input
projection (the top-k sum of cvmm.py:1223) are sums over each token's routes.
With routes from the stable sort and a fan-out at or above the threshold set
by CVMM_TUNE_REDUCE_MIN_TOPK (the reduce GEMM is off by default) the library
computes them with the reduce GEMM.  Every case below is checked:
  * that the reduce GEMM ran (its kernel class saw launches),
  * against the CPU oracle (max|a-b|/max|b| <= 2e-2 under bf16/fp16 autocast),
  * against the route-buffer path of the same call (reduce GEMM switched
    off): the two differ only in the fp32 summation order of a
    token's routes (expert order here, route order there), so each element
    may move by one rounding step of the output type: <= 8e-3 of max|b|;
    the outputs that do not go through a top-k sum are bit-identical,
  * for repeatability (two runs, bit-identical).
Shapes cover K = 64 and 128, widths of 64-column slices (and one that is not,
which keeps the route buffer), token counts that are not a multiple of the
256-token group, experts without routes, tokens that picked one expert more
than once (routes of one token in one stage, added one at a time), fp32
storage (converted in the gather, fp32 output) and fp16.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import cvmm_codex_amd.api as C
from cvmm_codex_amd import _native as N
from tests.gpu_util import compare, norm_rel, run_hip, run_oracle, to_np

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_PATHS = 8e-3
OFF = 0  # the built-in choice: route-buffer path


@pytest.fixture
def min_topk():
    lib = N.lib()

    def set_(v):
        N.check(lib.cvmm_tuning_set(N.TUNE_REDUCE_MIN_TOPK, v), "cvmm_tuning_set")

    yield set_
    set_(0)


def _reduce_launches(fn):
    lib = N.lib()
    torch.cuda.synchronize()
    lib.cvmm_timing_enable(N.KC_REDUCE)
    try:
        res = fn()
        torch.cuda.synchronize()
    finally:
        lib.cvmm_timing_enable(0)
    ms, n = ctypes.c_double(), ctypes.c_int64()
    N.check(lib.cvmm_timing_result(N.KC_REDUCE, ctypes.byref(ms), ctypes.byref(n)), "cvmm_timing_result")
    return res, n.value


def _case(T, k, E, d_in, d_out, route_input, weighted, seed, dup=False, x_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((T, k, d_in) if route_input else (T, d_in)), generator=g).to(x_dtype)
    keys = torch.randn(E, d_in, d_out, generator=g) / d_in ** 0.5
    # uneven expert loads (expert e drawn with probability ~ e + 1); the last
    # experts are never drawn: experts without routes
    p = torch.arange(1, E + 1, dtype=torch.float32)
    p[-3:] = 0
    sel = torch.multinomial(p.expand(T, E), k, replacement=dup, generator=g)
    w = torch.softmax(torch.randn(T, k, generator=g), -1) if weighted else None
    gy = torch.randn(*((T, d_out) if weighted else (T, k, d_out)), generator=g).to(torch.bfloat16)
    return x, keys, sel, w, gy


def _check(case, route_input, set_min, amp_dtype=torch.bfloat16, min_topk=None):
    x, keys, sel, w, gy = case
    reduced = "out" if w is not None and route_input else "x_grad"
    set_min(min_topk or 1)
    got, n = _reduce_launches(lambda: run_hip(x, keys, sel, w, gy, route_input, True, amp_dtype=amp_dtype))
    assert n >= 1, "the reduce GEMM did not run"
    again = run_hip(x, keys, sel, w, gy, route_input, True, amp_dtype=amp_dtype)
    set_min(OFF)
    buf, n_off = _reduce_launches(lambda: run_hip(x, keys, sel, w, gy, route_input, True, amp_dtype=amp_dtype))
    assert n_off == 0
    op = "float16" if amp_dtype == torch.float16 else "bfloat16"
    exp = run_oracle(x, keys, sel, w, gy, route_input, True, amp_dtype=op)
    errs = compare(got, exp, TOL)
    for name in ("out", "x_grad", "keys_grad", "weights_grad"):
        if got[name] is None:
            continue
        assert torch.equal(got[name], again[name]), f"{name} differs between two runs"
        if name == reduced:
            assert norm_rel(to_np(got[name]), to_np(buf[name])) <= TOL_PATHS, name
        else:
            assert torch.equal(got[name], buf[name]), f"{name} changed with the top-k sum's path"
    return errs


def test_weighted_route_input_forward_k64(min_topk):
    """SwitchHead output projection shape: top-64 over 256 experts, K = 64."""
    _check(_case(520, 64, 256, 64, 128, True, True, seed=1), True, min_topk)


def test_token_input_grad_k64(min_topk):
    """SwitchHead value projection shape: the top-64 token-gradient sum."""
    _check(_case(520, 64, 256, 192, 64, False, False, seed=2), False, min_topk)


def test_weighted_route_input_forward_k128(min_topk):
    _check(_case(300, 32, 64, 128, 128, True, True, seed=3), True, min_topk)


def test_token_input_grad_k128(min_topk):
    _check(_case(300, 32, 64, 192, 128, False, False, seed=4), False, min_topk)


@pytest.mark.parametrize("route_input", [True, False], ids=["weighted-forward", "token-grad"])
def test_tokens_that_pick_an_expert_twice(route_input, min_topk):
    """Drawn with replacement: 40 routes over 16 experts, so most tokens send
    several routes to one expert (they meet in one stage of the kernel)."""
    case = _case(290, 40, 16, 64 if route_input else 128, 128 if route_input else 64, route_input, route_input,
                 seed=5, dup=True)
    _check(case, route_input, min_topk)


@pytest.mark.parametrize("route_input", [True, False], ids=["weighted-forward", "token-grad"])
def test_fp32_storage(route_input, min_topk):
    """fp32 x: converted to bf16 by the gather; the token gradient is fp32."""
    case = _case(270, 32, 48, 64 if route_input else 128, 128 if route_input else 64, route_input, route_input,
                 seed=6, x_dtype=torch.float32)
    _check(case, route_input, min_topk)


def test_fp16_autocast(min_topk):
    case = _case(260, 32, 40, 64, 64, True, True, seed=7, x_dtype=torch.float16)
    _check(case, True, min_topk, amp_dtype=torch.float16)


def test_widths_off_the_kernel_take_the_buffer_path(min_topk):
    """N = 96 is not a multiple of the 64-column slice: the flagged call is the
    call without the flag (route buffer), with the same results."""
    x, keys, sel, w, gy = _case(300, 32, 40, 64, 96, True, True, seed=11)
    min_topk(1)
    got, n = _reduce_launches(lambda: run_hip(x, keys, sel, w, gy, True, True))
    assert n == 0
    compare(got, run_oracle(x, keys, sel, w, gy, True, True), TOL)


def test_top8_small_stages(min_topk):
    """The FFN down projection's top-8 weighted forward with the threshold at
    8: small per-expert segments (32-route stages), many partial stages."""
    _check(_case(700, 8, 16, 128, 256, True, True, seed=8), True, min_topk, min_topk=8)


def test_weighted_token_input_forward_and_grad(min_topk):
    """Token input with weights: the forward is a top-k sum of token rows and
    the weighted token gradient (with grad_rw) keeps the route buffer path."""
    x, keys, sel, w, gy = _case(330, 32, 48, 64, 64, False, True, seed=9)
    min_topk(1)
    got, n = _reduce_launches(lambda: run_hip(x, keys, sel, w, gy, False, True))
    assert n >= 1
    compare(got, run_oracle(x, keys, sel, w, gy, False, True), TOL)


def test_weighted_token_grad_without_rw_grad(min_topk):
    """A weighted token-input call whose reduction weights need no gradient:
    the token gradient is a weighted top-k sum through the reduce GEMM."""
    x, keys, sel, w, gy = _case(330, 32, 48, 64, 64, False, True, seed=10)
    dev = torch.device("cuda")

    def run():
        xd = x.to(dev).requires_grad_(True)
        kd = keys.to(dev).requires_grad_(True)
        s = C.cvmm_prepare_sel2(sel.to(dev), w.to(dev))
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = C.cvmm(xd, s, kd)
        y.backward(gy.to(dev).to(y.dtype))
        torch.cuda.synchronize()
        return {"out": y.detach(), "x_grad": xd.grad, "keys_grad": kd.grad, "weights_grad": None}

    min_topk(1)
    (got, n) = _reduce_launches(run)
    assert n >= 2  # forward and token gradient
    exp = run_oracle(x, keys, sel, w, gy, False, True, need_w=True)
    exp["weights_grad"] = None
    compare(got, exp, TOL)
