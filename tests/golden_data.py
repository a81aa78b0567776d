"""Loader for the committed golden fixtures (tests/golden/cvmm_cases.npz)."""
from __future__ import annotations

import ast
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np

from oracle.cvmm_oracle import bf16_bits_to_f32

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cvmm_cases.npz")
MODES = ("float32", "bf16_amp", "bf16_params")

# benchmark_correctness_original.py:47-66, as (atol, rtol)
TOLERANCES = {
    "float32": {"out": (2e-4, 2e-4), "x_grad": (5e-4, 5e-4), "keys_grad": (2e-3, 2e-3), "weights_grad": (2e-3, 2e-3)},
    "bf16_amp": {"out": (1.5e-1, 6e-2), "x_grad": (2.5e-1, 8e-2), "keys_grad": (3.5e-1, 8e-2), "weights_grad": (3.5e-1, 8e-2)},
    "bf16_params": {"out": (2.0e-1, 8e-2), "x_grad": (3.0e-1, 1e-1), "keys_grad": (3.5e-1, 1e-1), "weights_grad": (3.5e-1, 1e-1)},
}

# The north-star parity bound, as max|a-b| / max|b| per tensor.
NORM_REL = {"float32": 1e-4, "bf16_amp": 2e-2, "bf16_params": 2e-2}


@dataclass
class Fixture:
    case: dict
    mode: str
    x: np.ndarray
    x_dtype: str
    keys: np.ndarray
    keys_dtype: str
    sel: np.ndarray
    weights: Optional[np.ndarray]
    weights_dtype: Optional[str]
    grad_out: np.ndarray
    grad_dtype: str
    exp_out: np.ndarray
    exp_x_grad: np.ndarray
    exp_keys_grad: np.ndarray
    exp_weights_grad: Optional[np.ndarray]

    @property
    def name(self):
        return f"{self.case['name']}[{self.mode}]"


_cache = None


def _load():
    global _cache
    if _cache is None:
        _cache = dict(np.load(PATH, allow_pickle=False))
    return _cache


def _arr(d, key):
    a = d[key]
    tag = str(d[key + "_dtype"])
    if tag == "bfloat16":
        return bf16_bits_to_f32(a), tag
    return a.astype(np.float32), tag


def cases():
    d = _load()
    return [ast.literal_eval(s) for s in d["cases"]]


def fixtures():
    d = _load()
    out = []
    for mode in MODES:
        for case in cases():
            p = f"{case['name']}__{mode}__"
            x, xdt = _arr(d, p + "x")
            keys, kdt = _arr(d, p + "keys")
            go, gdt = _arr(d, p + "grad_out")
            if (p + "weights") in d:
                w, wdt = _arr(d, p + "weights")
                ewg = d[p + "exp_weights_grad"]
            else:
                w, wdt, ewg = None, None, None
            out.append(Fixture(case, mode, x, xdt, keys, kdt, d[p + "sel"], w, wdt, go, gdt,
                               d[p + "exp_out"], d[p + "exp_x_grad"], d[p + "exp_keys_grad"], ewg))
    return out


def norm_rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = max(np.abs(b).max(initial=0.0), 1e-30)
    return float(np.abs(a - b).max(initial=0.0) / denom)


def mode_dtypes(mode: str):
    """(op dtype, out dtype) of the reference for a dtype mode: autocast bf16
    unless float32 (benchmark_correctness_original.py:98-99, cvmm.py:30-33)."""
    if mode == "float32":
        return "float32", "float32"
    return "bfloat16", "bfloat16"
