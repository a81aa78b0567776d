"""Run the CPU oracle on a golden fixture the way the reference test harness
drives CVMM (benchmark_correctness_original.py:202-214)."""
from __future__ import annotations

import numpy as np

from oracle import cvmm_oracle as O
from tests.golden_data import Fixture, mode_dtypes


def run(fx: Fixture, exact: bool = False, compute=np.float64, oracle=O):
    """Returns dict(out, x_grad, keys_grad, weights_grad) from the oracle.

    ``exact``: no rounding points at all (pure float64 mathematics), which is
    what the golden expected values are.
    """
    op, out = (None, None) if exact else mode_dtypes(fx.mode)
    x_dt = None if exact else fx.x_dtype
    k_dt = None if exact else fx.keys_dtype
    w_dt = None if exact else fx.weights_dtype
    meta = oracle.prepare_sel2(fx.sel, fx.weights, route_input=fx.case["route_input"])
    y = oracle.forward(fx.x, meta, fx.keys, op, out, compute=compute)
    gy = oracle.rnd(fx.grad_out, out, compute)          # grad_out.to(out.dtype)
    dx, dw, dg = oracle.backward(fx.x, meta, fx.keys, gy, op, x_dtype=x_dt, keys_dtype=k_dt,
                                 w_dtype=w_dt, compute=compute)
    return {"out": y, "x_grad": dx, "keys_grad": dw, "weights_grad": dg}


def expected(fx: Fixture):
    return {"out": fx.exp_out, "x_grad": fx.exp_x_grad, "keys_grad": fx.exp_keys_grad,
            "weights_grad": fx.exp_weights_grad}
