"""Drop-in behaviour of the selector and of unusual inputs, on the GPU:

* cvmm_prepare_sel2 fixes the routing when it is called, as the reference's
  `fsel = sel.flatten().to(int32); fsel.sort()` does (cvmm.py:1796-1797):
  writing to `sel` afterwards changes nothing;
* CVMMSel is a dataclass (cvmm.py:12-21): dataclasses.replace gives a
  selector cvmm() accepts;
* routes whose expert id is outside [0, E) get zero rows wherever the op
  writes one row per route (no uninitialised memory);
* the counting sort is bit-exact up to the largest expert count the ABI
  accepts (32767), where its scatter takes 128 KB of LDS.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

import cvmm_codex_amd.api as C
from oracle import cvmm_oracle as O
from tests import gpu_util as U

pytestmark = pytest.mark.gpu


def _case(seed, B=2, T=96, D=128, H=64, E=8, K=4, weighted=False, route_input=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((B, T, K, D) if route_input else (B, T, D)), generator=g).to(torch.bfloat16)
    keys = torch.randn(E, D, H, generator=g) / D ** 0.5
    sel = torch.randint(0, E, (B, T, K), generator=g)
    w = torch.rand(B, T, K, generator=g) if weighted else None
    go = torch.randn(*((B, T, H) if weighted else (B, T, K, H)), generator=g).to(torch.bfloat16)
    return x, keys, sel, w, go


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True)])
def test_writes_to_sel_after_prepare_do_not_change_the_routing(dtype, weighted, route_input):
    """Prepare, then overwrite `sel` in place before cvmm: the result is the
    one of the selection as it was at prepare time (oracle on the original)."""
    x, keys, sel, w, go = _case(11, weighted=weighted, route_input=route_input)
    sel = sel.to(dtype)

    def prepare_then_clobber(sd, wd, route_input):
        s = C.cvmm_prepare_sel2(sd, wd, route_input=route_input)
        sd.copy_((sd + 3) % keys.shape[0])     # a different routing, same storage
        return s

    got = U.run_hip(x, keys, sel, w, go, route_input, True, prepare=prepare_then_clobber)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    U.compare(got, exp, 2e-2)


def test_clobbered_sel_changes_nothing_when_read_early():
    """Reading .sel before cvmm (which sorts then, taking E from the largest
    id) still sees the prepare-time ids."""
    _, _, sel, _, _ = _case(12)
    sd = sel.cuda()
    s = C.cvmm_prepare_sel2(sd)
    sd.zero_()
    m = O.prepare_sel2(sel.numpy())
    assert np.array_equal(s.sel.cpu().numpy(), m.sel)
    assert np.array_equal(s.out_index.cpu().numpy(), m.out_index)
    assert np.array_equal(s.raw_sel.cpu().numpy(), m.raw_sel)


def test_dataclass_replace_gives_a_working_selector():
    x, keys, sel, w, go = _case(13, weighted=True, route_input=False)
    s = C.cvmm_prepare_sel2(sel.cuda())
    wd = w.cuda().requires_grad_(True)
    s2 = dataclasses.replace(s, reduction_weight=wd)          # forces the sort (E from the largest id)
    xd = x.cuda().requires_grad_(True)
    kd = keys.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(xd, s2, kd)
    y.backward(go.cuda().to(y.dtype))
    got = {"out": y.detach(), "x_grad": xd.grad, "keys_grad": kd.grad, "weights_grad": wd.grad}
    U.compare(got, U.run_oracle(x, keys, sel, w, go, False, True), 2e-2)


# ---------------------------------------------------------------------------
# out-of-range expert ids: their per-route rows are zero
# ---------------------------------------------------------------------------

def _with_bad_ids(sel, E, seed):
    g = torch.Generator().manual_seed(seed)
    bad = torch.rand(sel.shape, generator=g) < 0.15
    s = sel.clone()
    s[bad] = torch.where(torch.rand(sel.shape, generator=g) < 0.5, -2, E + 5)[bad]
    return s, bad


@pytest.mark.parametrize("route_input,amp,D,H", [(False, True, 256, 64), (True, True, 128, 64),
                                                 (False, False, 64, 48), (True, False, 40, 24),
                                                 (False, True, 96, 40)])
def test_unweighted_rows_of_invalid_routes_are_zero(route_input, amp, D, H):
    """Forward rows (one per route) and, for route input, grad-input rows of
    invalid routes are exactly zero; every other value matches the oracle
    run with those routes sent to expert 0 with a zero gradient row.  Covers
    the DMA kernels (16-bit, widths % 8), the general kernel (fp32, odd
    widths) and the per-route fp32 path."""
    E = 8
    x, keys, sel, _, go = _case(21, D=D, H=H, E=E, route_input=route_input)
    if not amp:
        x = x.float()
    sel_bad, bad = _with_bad_ids(sel, E, 22)
    # torch.empty garbage first: the caching allocator hands the same blocks back
    junk = [torch.full((1 << 20,), float("nan"), device="cuda") for _ in range(4)]
    del junk
    got = U.run_hip(x, keys, sel_bad, None, go, route_input, amp)
    badf = bad.reshape(-1).numpy()
    out = U.to_np(got["out"]).reshape(-1, H)
    assert np.all(out[badf] == 0)
    sel_ok = sel.clone()
    sel_ok[bad] = 0
    go_ok = go.clone()
    go_ok[bad] = 0
    exp = U.run_oracle(x, keys, sel_ok, None, go_ok, route_input, amp)
    tol = 2e-2 if amp else 1e-4
    assert U.norm_rel(out[~badf], exp["out"].reshape(-1, H)[~badf]) <= tol
    if route_input:
        gx = U.to_np(got["x_grad"]).reshape(-1, D)
        assert np.all(gx[badf] == 0)
        assert U.norm_rel(gx[~badf], exp["x_grad"].reshape(-1, D)[~badf]) <= tol
    else:
        assert U.norm_rel(U.to_np(got["x_grad"]), exp["x_grad"]) <= tol
    assert U.norm_rel(U.to_np(got["keys_grad"]), exp["keys_grad"]) <= tol


def test_weighted_route_input_grad_rows_of_invalid_routes_are_zero():
    E = 8
    x, keys, sel, w, go = _case(23, D=128, H=192, E=E, weighted=True, route_input=True)
    sel_bad, bad = _with_bad_ids(sel, E, 24)
    junk = [torch.full((1 << 20,), float("nan"), device="cuda") for _ in range(4)]
    del junk
    got = U.run_hip(x, keys, sel_bad, w, go, True, True)
    badf = bad.reshape(-1).numpy()
    gx = U.to_np(got["x_grad"]).reshape(-1, 128)
    assert np.all(gx[badf] == 0)
    assert np.all(U.to_np(got["weights_grad"]).reshape(-1)[badf] == 0)
    w_ok = w.clone()
    w_ok[bad] = 0
    sel_ok = sel.clone()
    sel_ok[bad] = 0
    exp = U.run_oracle(x, keys, sel_ok, w_ok, go, True, True)
    assert U.norm_rel(U.to_np(got["out"]), exp["out"]) <= 2e-2
    assert U.norm_rel(gx[~badf], exp["x_grad"].reshape(-1, 128)[~badf]) <= 2e-2


def test_gelu_rows_of_invalid_routes_are_zero():
    """cvmm_gelu (the long-K GELU epilogue and the separate GELU pass) keeps
    gelu(0) = 0 rows for invalid routes."""
    E = 8
    for D, H in ((256, 128), (64, 64)):
        x, keys, sel, _, _ = _case(25, D=D, H=H, E=E)
        sel_bad, bad = _with_bad_ids(sel, E, 26)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = C.cvmm_gelu(x.cuda(), C.cvmm_prepare_sel2(sel_bad.cuda()), keys.cuda())
        yn = U.to_np(y).reshape(-1, H)
        assert np.all(yn[bad.reshape(-1).numpy()] == 0), (D, H)


# ---------------------------------------------------------------------------
# the sort at the largest expert counts
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("E,R", [(8191, 3000), (8192, 3000), (20000, 5000), (32767, 4000), (32767, 70000)])
def test_sort_many_experts_bit_exact(E, R):
    """Above 8191 experts the scatter keeps only its bucket positions in LDS
    (up to 128 KB at 32767); ids, permutation, token index, offsets and the
    inverse permutation stay bit-exact, invalid ids included."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    g = torch.Generator().manual_seed(E + R)
    sel = torch.randint(-2, E + 2, (R,), generator=g)
    raw = sel.cuda()
    k = 2
    ssel = torch.empty(R, dtype=torch.int32, device="cuda")
    perm = torch.empty(R, dtype=torch.int64, device="cuda")
    tok = torch.empty(R, dtype=torch.int64, device="cuda")
    off = torch.empty(E, dtype=torch.int64, device="cuda")
    pos = torch.full((R,), -1, dtype=torch.int32, device="cuda")
    nin = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_b = lib.cvmm_sort_workspace_bytes(R, E)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    N.check(lib.cvmm_sort_routes(N.ptr(raw), 1, R, E, k, N.ptr(ssel), N.ptr(perm), N.ptr(tok), N.ptr(off),
                                 N.ptr(pos), N.ptr(nin), N.ptr(ws), ws_b, N.stream_of(raw.device)), "sort")
    s = sel.numpy()
    valid = (s >= 0) & (s < E)
    exp_perm = np.argsort(np.where(valid, s, E), kind="stable")
    assert int(nin.item()) == int((~valid).sum())
    assert np.array_equal(perm.cpu().numpy(), exp_perm)
    assert np.array_equal(tok.cpu().numpy(), exp_perm // k)
    assert np.array_equal(ssel.cpu().numpy(), s[exp_perm].astype(np.int32))
    inv = np.empty_like(exp_perm)
    inv[exp_perm] = np.arange(R)
    assert np.array_equal(pos.cpu().numpy(), inv)
    assert np.array_equal(off.cpu().numpy(), np.cumsum(np.bincount(s[valid], minlength=E)))


def test_sort_many_experts_through_the_api():
    """cvmm over 20000 experts (top-2): the selector and the products match
    the oracle."""
    E, D, H = 20000, 64, 32
    g = torch.Generator().manual_seed(31)
    x = torch.randn(1, 300, D, generator=g).to(torch.bfloat16)
    keys = torch.randn(E, D, H, generator=g) / 8
    sel = torch.randint(0, E, (1, 300, 2), generator=g)
    go = torch.randn(1, 300, 2, H, generator=g).to(torch.bfloat16)
    got = U.run_hip(x, keys, sel, None, go, False, True)
    U.compare(got, U.run_oracle(x, keys, sel, None, go, False, True), 2e-2)


@pytest.mark.parametrize("dtype,n,offset", [(torch.int64, 65536, 0), (torch.int64, 1001, 1), (torch.int32, 4099, 0),
                                            (torch.int32, 77, 3), (torch.int64, 3, 0)])
def test_copy_ids_is_the_int32_conversion(dtype, n, offset):
    """cvmm_copy_ids (the ids copy cvmm_prepare_sel2 takes) equals torch's
    int32 conversion, int64 ids >= 2^31 wrapping as there; aligned (vector)
    and misaligned (element) views."""
    from cvmm_codex_amd import _native as N
    g = torch.Generator().manual_seed(n + offset)
    base = torch.randint(-(2 ** 40), 2 ** 40, (n + offset,), generator=g, dtype=torch.int64).to(dtype).cuda()
    sel = base[offset:]
    out = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    N.check(N.lib().cvmm_copy_ids(N.ptr(sel), 1 if dtype == torch.int64 else 0, n, N.ptr(out),
                                  N.stream_of(sel.device)), "cvmm_copy_ids")
    assert torch.equal(out.cpu(), sel.cpu().to(torch.int32))
