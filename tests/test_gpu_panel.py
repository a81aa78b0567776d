"""Small-K routed GEMM (the panel kernel: K <= 128, N % 64 == 0) on the GPU.

The kernel streams each workgroup's n-tiles through a three-buffer LDS ring
with exact wait counts, so its results must not depend on how many n-tiles a
workgroup walks: every run below is checked against the CPU oracle and the
runs with different tiles-per-workgroup settings must agree bit for bit.
Shapes cover both inner-dimension variants (K <= 64 and K <= 128, including
K not a multiple of 32), both n-tile widths (N % 128 == 0 and N % 64 == 0),
partial m-tiles, fp32 outputs and the forward and grad-input products.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cvmm_codex_amd import _native as N
from tests.gpu_util import compare, run_hip, run_oracle, to_np

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2


@pytest.fixture
def tiles_per_wg():
    lib = N.lib()

    def set_(v):
        N.check(lib.cvmm_tuning_set(N.TUNE_PANEL_TILES_PER_WG, v), "cvmm_tuning_set")

    yield set_
    set_(0)


def _case(d_in, d_out, E, tokens, top_k, seed, x_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, d_in, generator=g).to(x_dtype)
    keys = torch.randn(E, d_in, d_out, generator=g) / d_in ** 0.5
    # uneven expert loads: expert e drawn with probability ~ (e + 1)
    p = torch.arange(1, E + 1, dtype=torch.float32)
    sel = torch.multinomial(p.expand(tokens, E), top_k, replacement=False, generator=g)
    gy = torch.randn(tokens, top_k, d_out, generator=g).to(torch.bfloat16)
    return x, keys, sel, gy


# (d_in, d_out): which products take the panel kernel
#   (128, 1024): forward K=128 N=1024          (KP 128, BN 64)
#   (1024, 128): grad-input K=128 N=1024        (KP 128, BN 64)
#   (64, 256):   forward K=64 N=256             (KP 64, BN 128)
#   (256, 64):   grad-input K=64 N=256          (KP 64, BN 128)
#   (40, 192):   forward K=40 N=192             (KP 64, BN 64, zero k chunks)
#   (192, 96):   grad-input K=96 N=192          (KP 128, BN 64, zero k chunks)
SHAPES = [(128, 1024), (1024, 128), (64, 256), (256, 64), (40, 192), (192, 96)]


@pytest.mark.parametrize("d_in,d_out", SHAPES)
def test_panel_matches_oracle_for_every_tiles_per_wg(d_in, d_out, tiles_per_wg):
    x, keys, sel, gy = _case(d_in, d_out, E=5, tokens=700, top_k=2, seed=d_in * 7 + d_out)
    exp = run_oracle(x, keys, sel, None, gy, False, True, need_w=False)
    first = None
    for tpw in (0, 1, 2, 3, 4, 5, 7):
        tiles_per_wg(tpw)
        got = run_hip(x, keys, sel, None, gy, False, True)
        compare(got, exp, TOL_BF16, names=("out", "x_grad"))
        cur = (to_np(got["out"]), to_np(got["x_grad"]))
        if first is None:
            first = cur
        else:
            assert np.array_equal(first[0], cur[0]), f"forward differs at tiles_per_wg={tpw}"
            assert np.array_equal(first[1], cur[1]), f"grad-input differs at tiles_per_wg={tpw}"


def test_panel_fp32_route_buffer(tiles_per_wg):
    # fp32 x under autocast: the grad-input route buffer is fp32 (16-byte stores)
    x, keys, sel, gy = _case(512, 128, E=4, tokens=600, top_k=3, seed=11, x_dtype=torch.float32)
    exp = run_oracle(x, keys, sel, None, gy, False, True, need_w=False)
    outs = []
    for tpw in (0, 1, 3):
        tiles_per_wg(tpw)
        got = run_hip(x, keys, sel, None, gy, False, True)
        compare(got, exp, TOL_BF16, names=("out", "x_grad"))
        outs.append(to_np(got["x_grad"]))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_panel_route_input_weighted_forward(tiles_per_wg):
    # ff_down shape: route-major x, weighted combine; the forward product
    # (K = 128, N = 512) writes the route-ordered buffer the combine reads
    g = torch.Generator().manual_seed(5)
    tokens, top_k, E, d_in, d_out = 300, 4, 6, 128, 512
    x = torch.randn(tokens, top_k, d_in, generator=g).to(torch.bfloat16)
    keys = torch.randn(E, d_in, d_out, generator=g) / d_in ** 0.5
    sel = torch.randint(0, E, (tokens, top_k), generator=g)
    w = torch.softmax(torch.randn(tokens, top_k, generator=g), -1)
    gy = torch.randn(tokens, d_out, generator=g).to(torch.bfloat16)
    exp = run_oracle(x, keys, sel, w, gy, True, True, need_w=False)
    outs = []
    for tpw in (0, 2, 5):
        tiles_per_wg(tpw)
        got = run_hip(x, keys, sel, w, gy, True, True)
        compare(got, exp, TOL_BF16, names=("out", "x_grad", "weights_grad"))
        outs.append(to_np(got["out"]))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
