"""GPU parity of the HIP CVMM path against the CPU oracle and the golden
fixtures.  Tolerances: max|a-b|/max|b| <= 1e-4 in fp32 mode and <= 2e-2 in
bf16-AMP mode, plus the reference harness's own
elementwise (atol, rtol) table against the exact fp64 fixtures
(benchmark_correctness_original.py:47-66)."""
import itertools

import numpy as np
import pytest
import torch

import cvmm_codex_amd.api as C
from oracle import cvmm_oracle as O
from tests import golden_data as G
from tests import gpu_util as U

pytestmark = pytest.mark.gpu

FIXTURES = G.fixtures()


def _fixture_tensors(fx):
    dt = U.TORCH_DT
    x = torch.from_numpy(fx.x).to(dt[fx.x_dtype])
    keys = torch.from_numpy(fx.keys).to(dt[fx.keys_dtype])
    sel = torch.from_numpy(fx.sel)
    w = None if fx.weights is None else torch.from_numpy(fx.weights).to(dt[fx.weights_dtype])
    go = torch.from_numpy(fx.grad_out).to(dt[fx.grad_dtype])
    return x, keys, sel, w, go


@pytest.fixture(params=[False, True], ids=["ordered-reduce", "atomic-reduce"])
def reduce_mode(request, monkeypatch):
    monkeypatch.setattr(C, "cvmm_atomic_reduce", request.param)
    return request.param


@pytest.mark.parametrize("fx", FIXTURES, ids=lambda f: f.name)
def test_golden_cases(fx, reduce_mode):
    """The reference harness's 7 edge cases x 3 dtype modes."""
    x, keys, sel, w, go = _fixture_tensors(fx)
    amp = fx.mode != "float32"
    got = U.run_hip(x, keys, sel, w, go, fx.case["route_input"], amp)
    # 1) against the oracle with the reference's rounding points
    exp = U.run_oracle(x, keys, sel, w, go, fx.case["route_input"], amp)
    U.compare(got, exp, G.NORM_REL[fx.mode])
    # 2) against the exact fp64 einsum definition with the harness tolerances
    gold = {"out": fx.exp_out, "x_grad": fx.exp_x_grad, "keys_grad": fx.exp_keys_grad,
            "weights_grad": fx.exp_weights_grad}
    for name, ref in gold.items():
        if ref is None:
            continue
        atol, rtol = G.TOLERANCES[fx.mode][name]
        np.testing.assert_allclose(U.to_np(got[name]), ref, atol=atol, rtol=rtol, err_msg=name)


# ---------------------------------------------------------------------------
# the reference's own GPU tests (test_cvmm_correctness.py), with CPU-seeded data
# ---------------------------------------------------------------------------

def _einsum_reference(x, sel, keys, weights=None):
    """test_cvmm_correctness.py:7-15 (fp32 there; fp64 here)."""
    selected = keys[sel].double()
    if x.shape[:-1] == sel.shape:
        out = (x.double().unsqueeze(-1) * selected).sum(dim=-2)
    else:
        out = (x.double().unsqueeze(-2).unsqueeze(-1) * selected).sum(dim=-2)
    if weights is not None:
        out = (weights.unsqueeze(-1).double() * out).sum(dim=-2)
    return out


def _assert_close_like_reference(got, exact, oracle_val, rtol, atol):
    """Elementwise: |got - exact| <= atol + rtol*|exact| (the reference test's
    bound) + |oracle - exact| (what the reference's own bf16 rounding points
    cost at this element) + one bf16 ulp of |exact| (a different final
    rounding).  The reference test draws its inputs from the device RNG, so
    its fixed tolerance is only known to hold for its own draws."""
    got = np.asarray(U.to_np(got), dtype=np.float64)
    exact = np.asarray(exact, dtype=np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    bound = atol + rtol * np.abs(exact) + np.abs(np.asarray(oracle_val, dtype=np.float64) - exact) + ulp
    excess = np.abs(got - exact) - bound
    assert (excess <= 0).all(), f"max excess {excess.max():.3g}"


def _check_case(weighted, route_input=False):
    """test_cvmm_correctness.py:18-58, same shapes and tolerances."""
    g = torch.Generator().manual_seed(1234 + int(weighted) + 17 * int(route_input))
    b, t, d, out_d, n_experts, top_k = 3, 5, 16, 11, 7, 3
    x_shape = (b, t, top_k, d) if route_input else (b, t, d)
    x = torch.randn(*x_shape, generator=g).to(torch.bfloat16)
    keys = torch.randn(n_experts, d, out_d, generator=g)
    sel = torch.randint(0, n_experts, (b, t, top_k), generator=g)
    weights = torch.randn(b, t, top_k, generator=g) if weighted else None
    out_shape = (b, t, out_d) if weighted else (b, t, top_k, out_d)
    grad = torch.randn(*out_shape, generator=g).to(torch.bfloat16)
    got = U.run_hip(x, keys, sel, weights, grad, route_input, True)
    orc = U.run_oracle(x, keys, sel, weights, grad, route_input, True)
    U.compare(got, orc, 2e-2)

    xr = x.double().requires_grad_(True)
    kr = keys.double().requires_grad_(True)
    wr = None if weights is None else weights.double().requires_grad_(True)
    exp = _einsum_reference(xr, sel, kr, wr)
    exp.backward(grad.double())
    rtol, atol = (5e-2, 1e-1) if route_input else (2e-2, 2e-2)
    _assert_close_like_reference(got["out"], exp.detach().numpy(), orc["out"], rtol, atol)
    grad_rtol, grad_atol = (6e-2, 1e-1) if route_input else (3e-2, 3e-2)
    pairs = [("x_grad", xr.grad), ("keys_grad", kr.grad)]
    if weighted:
        pairs.append(("weights_grad", wr.grad))
    for name, e in pairs:
        _assert_close_like_reference(got[name], e.numpy(), orc[name], grad_rtol, grad_atol)


def test_unweighted():
    _check_case(False)


def test_weighted():
    _check_case(True)


def test_weighted_route_input():
    _check_case(True, route_input=True)


@pytest.mark.parametrize("n_experts,total_routes", list(itertools.product((1, 7, 64, 512), (1, 13, 1000))))
def test_expert_offsets_kernel(n_experts, total_routes, monkeypatch):
    """test_cvmm_correctness.py:73-86: native offsets == the torch closed form."""
    C.create_kernels()
    g = torch.Generator().manual_seed(n_experts * 7 + total_routes)
    sel = torch.randint(0, n_experts, (total_routes,), generator=g, dtype=torch.int32).sort().values
    fast = C._cvmm_expert_offsets(sel.cuda(), n_experts)
    monkeypatch.setattr(C, "cvmm_expert_offsets_call", None)
    ref = C._cvmm_expert_offsets(sel.cuda(), n_experts)
    assert torch.equal(fast.cpu(), ref.cpu())
    assert np.array_equal(fast.cpu().numpy(), O.expert_offsets(sel.numpy(), n_experts))


def test_top32_lowmem_unweighted(monkeypatch):
    """test_cvmm_correctness.py:89-118 (top-32 over 64 experts)."""
    monkeypatch.setattr(C, "cvmm_lowmem_chunk_size", 0)
    g = torch.Generator().manual_seed(2026)
    b, t, d, out_d, n_experts, top_k = 2, 5, 32, 16, 64, 32
    x = torch.randn(b, t, d, generator=g).to(torch.bfloat16)
    keys = torch.randn(n_experts, d, out_d, generator=g)
    sel = torch.randint(0, n_experts, (b, t, top_k), generator=g)
    grad = torch.randn(b, t, top_k, out_d, generator=g)
    got = U.run_hip(x, keys, sel, None, grad.to(torch.bfloat16), False, True)
    xr = x.double().requires_grad_(True)
    kr = keys.double().requires_grad_(True)
    exp = _einsum_reference(xr, sel, kr)
    exp.backward(grad.to(torch.bfloat16).double())
    torch.testing.assert_close(got["out"].float().cpu(), exp.float(), rtol=5e-2, atol=1e-1)
    torch.testing.assert_close(got["x_grad"].float().cpu(), xr.grad.float(), rtol=3e-1, atol=6e-1)
    torch.testing.assert_close(got["keys_grad"].float().cpu(), kr.grad.float(), rtol=1e-1, atol=1e-1)
    # and the tighter oracle bound
    exp2 = U.run_oracle(x, keys, sel, None, grad.to(torch.bfloat16), False, True)
    U.compare(got, exp2, 2e-2)


def test_weighted_route_input_reused_selector():
    """test_cvmm_correctness.py:121-137: bit-identical outputs."""
    g = torch.Generator().manual_seed(1251)
    b, t, d, out_d, n_experts, top_k = 3, 5, 16, 11, 7, 3
    x = torch.randn(b, t, top_k, d, generator=g).to(torch.bfloat16).cuda()
    keys = torch.randn(n_experts, d, out_d, generator=g).cuda()
    sel = torch.randint(0, n_experts, (b, t, top_k), generator=g).cuda()
    weights = torch.randn(b, t, top_k, generator=g).cuda()
    base = C.cvmm_prepare_sel2(sel)
    reused = C.cvmm_prepare_sel2(base, weights, route_input=True)
    fresh = C.cvmm_prepare_sel2(sel, weights, route_input=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        a = C.cvmm(x, reused, keys)
        e = C.cvmm(x, fresh, keys)
    assert torch.equal(a, e)
    # the same with an already-resolved parent selector
    base2 = C.cvmm_prepare_sel2(sel)
    _ = base2.sel_index
    reused2 = C.cvmm_prepare_sel2(base2, weights, route_input=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        a2 = C.cvmm(x, reused2, keys)
    assert torch.equal(a2, e)


# ---------------------------------------------------------------------------
# selector preparation: bit-exact against the stable sort
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,E,dtype", [
    ((1,), 1, torch.int64), ((13,), 7, torch.int64), ((3, 5, 3), 7, torch.int32),
    ((16, 512, 8), 64, torch.int64), ((8, 1024, 64), 256, torch.int64), ((2, 7, 1), 13, torch.int32),
    ((4, 4096, 8), 512, torch.int64), ((1, 5, 2), 32, torch.int64), ((64, 1000, 2), 2000, torch.int64),
    # >= 2^18 routes: the scatter orders each chunk in LDS first
    ((4, 65536, 1), 1, torch.int64), ((3, 30000, 4), 7, torch.int32), ((2, 40000, 4), 2047, torch.int64),
    ((2, 40000, 4), 2048, torch.int64),
])
def test_sort_routes_bit_exact(shape, E, dtype):
    g = torch.Generator().manual_seed(sum(shape) * 31 + E)
    sel = torch.randint(0, E, shape, generator=g, dtype=dtype)
    k = shape[-1]
    s = C.cvmm_prepare_sel2(sel.cuda())
    C.create_kernels()
    s._resolve(E)
    m = O.prepare_sel2(sel.numpy())
    assert s.raw_sel.dtype == torch.int32 and tuple(s.raw_sel.shape) == shape
    assert np.array_equal(s.raw_sel.cpu().numpy(), m.raw_sel)
    assert np.array_equal(s.sel.cpu().numpy(), m.sel)
    assert np.array_equal(s.out_index.cpu().numpy(), m.out_index)
    assert np.array_equal(s.sel_index.cpu().numpy(), m.sel_index)
    off = C._offsets_for(s.sel, E)
    assert np.array_equal(off.cpu().numpy(), O.expert_offsets(m.sel, E))
    r = C.cvmm_prepare_sel2(sel.cuda(), route_input=True)
    r._resolve(E)
    assert r.out_index is None and np.array_equal(r.sel_index.cpu().numpy(), m.out_index)
    p = C.cvmm_prepare_sel(sel.cuda(), E)
    assert p.out_index is None and np.array_equal(p.sel_index.cpu().numpy(), m.out_index)
    assert np.array_equal(p.sel.cpu().numpy(), m.sel)


def test_sort_int64_ids_wrap_like_int32_cast():
    """int64 ids are sorted as their int32 conversion (cvmm.py:1797 casts the
    flattened selection to int32 before sorting): 2**32 + 3 is expert 3."""
    g = torch.Generator().manual_seed(77)
    E = 9
    sel = torch.randint(0, E, (5, 40, 4), generator=g, dtype=torch.int64)
    big = sel.clone()
    big[::2] += 2 ** 32
    big[1::3] -= 2 ** 33
    s = C.cvmm_prepare_sel2(big.cuda())
    C.create_kernels()
    s._resolve(E)
    m = O.prepare_sel2(sel.numpy())
    assert np.array_equal(s.raw_sel.cpu().numpy(), m.raw_sel)
    assert np.array_equal(s.sel.cpu().numpy(), m.sel)
    assert np.array_equal(s.out_index.cpu().numpy(), m.out_index)
    assert np.array_equal(s.sel_index.cpu().numpy(), m.sel_index)


@pytest.mark.parametrize("R,E,k,d_in,d_out,fused", [
    (65536, 64, 8, 1024, 128, True), (4000, 16, 4, 128, 192, True), (3000, 7, 3, 64, 64, True),
    (777, 300, 1, 256, 64, True), (4000, 16, 4, 96, 128, False), (5000, 5, 2, 192, 384, True),
    (524288, 256, 64, 2048, 64, True),   # SwitchHead size: the column-scan scatter beside the cast
])
@pytest.mark.parametrize("layout", [0, 3])
def test_sort_and_cast_in_one_call_match_the_separate_calls(R, E, k, d_in, d_out, fused, layout):
    """cvmm_sort_routes_cast_keys (scatter and weight cast in one launch where
    the vectorised cast applies, else the two calls) gives the bits of
    cvmm_sort_routes + cvmm_cast_keys; out-of-range ids included.  Both copy
    layouts: routed ([E, d_out, d_in], [E, d_in, d_out]) and expert-interleaved
    ([d_out, E, d_in], [d_in, E, d_out]), each against torch's own cast."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    g = torch.Generator().manual_seed(R + E)
    raw = torch.randint(-1, E + 1, (R,), generator=g).cuda()
    keys = torch.randn(E, d_in, d_out, generator=g).cuda()
    st = N.stream_of(raw.device)
    ws_b = lib.cvmm_sort_workspace_bytes(R, E)

    def outputs():
        return dict(ssel=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                    perm=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                    tok=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                    off=torch.full((E,), -7, dtype=torch.int64, device="cuda"),
                    pos=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                    nin=torch.full((1,), -7, dtype=torch.int32, device="cuda"),
                    kt=torch.zeros(*((d_out, E, d_in) if layout & 1 else (E, d_out, d_in)),
                                   dtype=torch.bfloat16, device="cuda"),
                    kn=torch.zeros(*((d_in, E, d_out) if layout & 2 else (E, d_in, d_out)),
                                   dtype=torch.bfloat16, device="cuda"),
                    ws=torch.empty(ws_b, dtype=torch.uint8, device="cuda"))

    a, b = outputs(), outputs()
    sort_args = lambda o: (N.ptr(raw), 1, R, E, k, N.ptr(o["ssel"]), N.ptr(o["perm"]), N.ptr(o["tok"]),
                           N.ptr(o["off"]), N.ptr(o["pos"]), N.ptr(o["nin"]), N.ptr(o["ws"]), ws_b)
    key_args = (N.ptr(keys), N.F32)
    N.check(lib.cvmm_sort_routes(*sort_args(a), st), "sort")
    N.check(lib.cvmm_cast_keys(*key_args, E, d_in, d_out, *keys.stride(), N.BF16, N.ptr(a["kt"]), N.ptr(a["kn"]),
                               layout, st), "cast")
    N.check(lib.cvmm_sort_routes_cast_keys(*sort_args(b), *key_args, d_in, d_out, *keys.stride(), N.BF16,
                                           N.ptr(b["kt"]), N.ptr(b["kn"]), layout, st), "sort+cast")
    for n in ("ssel", "perm", "tok", "off", "pos", "nin", "kt", "kn"):
        assert torch.equal(a[n], b[n]), n
    kb = keys.to(torch.bfloat16)
    assert torch.equal(b["kn"], kb.permute(1, 0, 2) if layout & 2 else kb)
    assert torch.equal(b["kt"], kb.permute(2, 0, 1) if layout & 1 else kb.transpose(1, 2))
    assert fused == (d_in % 64 == 0 and d_out % 64 == 0)


@pytest.mark.parametrize("R,E,k,d_in,d_out,is64", [
    (65536, 64, 8, 1024, 128, True), (4000, 16, 4, 128, 192, False), (777, 300, 1, 256, 64, True),
    (4000, 16, 4, 96, 128, True),        # cast not fusable: separate cast launch
    (524288, 256, 64, 2048, 64, True),   # column-scan scatter
    (3000, 9000, 2, 64, 64, False),      # many-bucket scatter
])
def test_sort_with_counts_from_the_id_copy(R, E, k, d_in, d_out, is64):
    """cvmm_copy_ids_count (the id copy plus the sort's histogram) followed by
    cvmm_sort_routes_cast_keys_ex with CVMM_FLAG_COUNTS_READY gives the bits
    of cvmm_copy_ids + cvmm_sort_routes + cvmm_cast_keys, out-of-range ids
    included; keys NULL gives the sort alone."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    g = torch.Generator().manual_seed(R + E + 1)
    raw = torch.randint(-1, E + 1, (R,), generator=g).cuda()
    if not is64:
        raw = raw.to(torch.int32)
    keys = torch.randn(E, d_in, d_out, generator=g).cuda() if E * d_in * d_out <= 1 << 26 else None
    st = N.stream_of(raw.device)
    ws_b = lib.cvmm_sort_workspace_bytes(R, E)

    def outputs():
        o = dict(ids=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                 ssel=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                 perm=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                 tok=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                 off=torch.full((E,), -7, dtype=torch.int64, device="cuda"),
                 pos=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                 nin=torch.full((1,), -7, dtype=torch.int32, device="cuda"),
                 ws=torch.full((ws_b,), 0xA5, dtype=torch.uint8, device="cuda"))
        if keys is not None:
            o["kt"] = torch.zeros(E, d_out, d_in, dtype=torch.bfloat16, device="cuda")
            o["kn"] = torch.zeros(E, d_in, d_out, dtype=torch.bfloat16, device="cuda")
        return o

    a, b = outputs(), outputs()
    sort_args = lambda o: (N.ptr(o["ids"]), 0, R, E, k, N.ptr(o["ssel"]), N.ptr(o["perm"]), N.ptr(o["tok"]),
                           N.ptr(o["off"]), N.ptr(o["pos"]), N.ptr(o["nin"]), N.ptr(o["ws"]), ws_b)
    N.check(lib.cvmm_copy_ids(N.ptr(raw), int(is64), R, N.ptr(a["ids"]), st), "copy")
    N.check(lib.cvmm_sort_routes(*sort_args(a), st), "sort")
    N.check(lib.cvmm_copy_ids_count(N.ptr(raw), int(is64), R, E, N.ptr(b["ids"]), N.ptr(b["ws"]), ws_b, st),
            "copy+count")
    if keys is not None:
        N.check(lib.cvmm_cast_keys(N.ptr(keys), N.F32, E, d_in, d_out, *keys.stride(), N.BF16, N.ptr(a["kt"]),
                                   N.ptr(a["kn"]), 0, st), "cast")
        N.check(lib.cvmm_sort_routes_cast_keys_ex(*sort_args(b), N.ptr(keys), N.F32, d_in, d_out, *keys.stride(),
                                                  N.BF16, N.ptr(b["kt"]), N.ptr(b["kn"]), 0, N.FLAG_COUNTS_READY,
                                                  st), "sort+cast, counted")
    else:
        N.check(lib.cvmm_sort_routes_cast_keys_ex(*sort_args(b), None, 0, 0, 0, 0, 0, 0, 0, None, None, 0,
                                                  N.FLAG_COUNTS_READY, st), "sort, counted")
    torch.cuda.synchronize()
    for n in ("ids", "ssel", "perm", "tok", "off", "pos", "nin") + (("kt", "kn") if keys is not None else ()):
        assert torch.equal(a[n], b[n]), n


def test_counted_sort_ignores_counts_of_another_chunk():
    """A count matrix made by cvmm_copy_ids_count for one sort chunk is not
    trusted once the sort-chunk knob has changed (the sort counts again), nor
    a second time (the sort turned it into prefixes): both flagged sorts give
    the bits of a plain sort under the new chunk."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    R, E, k = 30000, 64, 4
    g = torch.Generator().manual_seed(77)
    raw = torch.randint(0, E, (R,), generator=g).to(torch.int32).cuda()
    st = N.stream_of(raw.device)
    ws_b = lib.cvmm_sort_workspace_bytes(R, E)

    def outputs():
        return dict(ids=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                    ssel=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                    perm=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                    tok=torch.full((R,), -7, dtype=torch.int64, device="cuda"),
                    off=torch.full((E,), -7, dtype=torch.int64, device="cuda"),
                    pos=torch.full((R,), -7, dtype=torch.int32, device="cuda"),
                    nin=torch.full((1,), -7, dtype=torch.int32, device="cuda"),
                    ws=torch.full((ws_b,), 0xA5, dtype=torch.uint8, device="cuda"))

    sort_args = lambda o: (N.ptr(o["ids"]), 0, R, E, k, N.ptr(o["ssel"]), N.ptr(o["perm"]), N.ptr(o["tok"]),
                           N.ptr(o["off"]), N.ptr(o["pos"]), N.ptr(o["nin"]), N.ptr(o["ws"]), ws_b)
    a, b = outputs(), outputs()
    try:
        N.check(lib.cvmm_copy_ids_count(N.ptr(raw), 0, R, E, N.ptr(b["ids"]), N.ptr(b["ws"]), ws_b, st), "count")
        # default chunk here: 1024 routes; larger chunks need less workspace,
        # so the stale counts would pass the size check
        assert lib.cvmm_tuning_set(N.TUNE_SORT_CHUNK, 2048) == 0
        N.check(lib.cvmm_copy_ids(N.ptr(raw), 0, R, N.ptr(a["ids"]), st), "copy")
        N.check(lib.cvmm_sort_routes(*sort_args(a), st), "plain sort")
        for _ in range(2):
            N.check(lib.cvmm_sort_routes_cast_keys_ex(*sort_args(b), None, 0, 0, 0, 0, 0, 0, 0, None, None, 0,
                                                      N.FLAG_COUNTS_READY, st), "flagged sort")
            torch.cuda.synchronize()
            for n in ("ids", "ssel", "perm", "tok", "off", "pos", "nin"):
                assert torch.equal(a[n], b[n]), n
    finally:
        lib.cvmm_tuning_set(N.TUNE_SORT_CHUNK, 0)


def test_prepared_selection_sorts_with_the_expected_expert_count():
    """cvmm_prepare_sel2 counts the ids for the expert count the last sort of
    a same-sized selection used, and cvmm() sorts without the histogram launch
    when its keys bring that count; another count sorts from scratch.  Three
    calls (no expectation yet, the expected count, a different count) each
    match the oracle."""
    x, keys, sel, w, go = _rand_case(71, 2, 96, 64, 80, 8, 4, False, False)
    key = (sel.numel(), sel.shape[-1])
    C._expert_guess.pop(key, None)
    for E in (8, 8, 12):
        keys_e = keys if E == 8 else (torch.randn(E, 64, 80, generator=torch.Generator().manual_seed(E)) / 8)
        got = U.run_hip(x, keys_e, sel, w, go, False, True)
        exp = U.run_oracle(x, keys_e, sel, w, go, False, True)
        U.compare(got, exp, 2e-2)
        assert C._expert_guess[key] == E


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True), (True, False)])
def test_invalid_ids_contribute_nothing(weighted, route_input):
    """Routes whose expert id is outside [0, E) sort last and no GEMM writes
    their rows; the top-k sums (the token gradient of a token-input
    selection, the weighted forward) leave them out instead of reading
    unwritten rows.  Checked against the oracle with those routes sent to
    expert 0 with a zero grad row (token input) or a zero routing weight
    (weighted), which contribute exact zeros; outputs that belong to an
    invalid route itself (its forward row, its route-input gradient row) have
    no defined value and are left out; its weight gradient is zero (the GEMM's
    surplus workgroups write its partials, which are not pre-filled)."""
    x, keys, sel, w, go = _rand_case(51, 2, 256, 128, 192, 8, 4, weighted, route_input)
    g = torch.Generator().manual_seed(52)
    bad = torch.rand(sel.shape, generator=g) < 0.1
    sel_bad = sel.clone()
    sel_bad[bad] = torch.where(torch.rand(sel.shape, generator=g) < 0.5, -1, 8 + 3)[bad]
    got = U.run_hip(x, keys, sel_bad, w, go, route_input, True)
    sel_ok = sel.clone()
    sel_ok[bad] = 0
    if weighted:
        w_ok = w.clone()
        w_ok[bad] = 0
        exp = U.run_oracle(x, keys, sel_ok, w_ok, go, route_input, True)
        keep = ~bad.reshape(-1).numpy()
        if route_input:  # per-route input rows: only the valid routes' are defined
            got["x_grad"] = got["x_grad"].reshape(-1, x.shape[-1])[torch.from_numpy(keep).cuda()]
            exp["x_grad"] = exp["x_grad"].reshape(-1, x.shape[-1])[keep]
        assert torch.all(got["weights_grad"].reshape(-1)[torch.from_numpy(~keep).cuda()] == 0)
        got["weights_grad"] = got["weights_grad"].reshape(-1)[torch.from_numpy(keep).cuda()]
        exp["weights_grad"] = exp["weights_grad"].reshape(-1)[keep]
        U.compare(got, exp, 2e-2)
    else:
        go_ok = go.clone()
        go_ok[bad] = 0
        exp = U.run_oracle(x, keys, sel_ok, None, go_ok, route_input, True)
        got["out"] = exp["out"] = None
        U.compare(got, exp, 2e-2, names=("x_grad", "keys_grad"))


@pytest.mark.parametrize("D,H,amp,ring_tile", [(128, 256, True, 1), (1024, 320, True, 1), (1024, 320, True, 2),
                                               (512, 320, True, 3), (64, 256, True, 0), (256, 64, True, 0),
                                               (48, 96, True, 0), (96, 80, False, 0)])
def test_weight_grad_partials_need_no_filled_workspace(D, H, amp, ring_tile):
    """Through the C ABI, weighted route-input grad-input with grad_rw: the
    per-(route, n tile) partials are written by the GEMM itself (covered
    routes by their tile, routes with out-of-range expert ids as zeros by the
    surplus workgroups), so a workspace of 0xFF bytes (NaN as fp32) gives the
    same bits as a zeroed one.  Shapes: the long-K ring kernel (128- and
    160-row tiles, its 256 x 256 tile with two partials per n tile, and its
    256 x 64 tile for N <= 64), the short-K tiled
    kernel (128 x 128 and 256 x 64) and the general kernel (fp32 op)."""
    from cvmm_codex_amd import _native as N
    E, K, T = 8, 4, 192
    dt = torch.bfloat16 if amp else torch.float32
    x, keys, sel, w, go = _rand_case(61 + D + H, 2, T, D, H, E, K, True, True,
                                     x_dt=dt, k_dt=torch.float32)
    g = torch.Generator().manual_seed(62)
    bad = torch.rand(sel.shape, generator=g) < 0.1
    sel_bad = sel.clone()
    sel_bad[bad] = torch.where(torch.rand(sel.shape, generator=g) < 0.5, -1, E + 3)[bad]
    s = C.cvmm_prepare_sel2(sel_bad.cuda(), w.cuda(), route_input=True)
    s._resolve(E)
    lib = N.lib()
    st = N.stream_of(torch.device("cuda"))
    op = N.BF16 if amp else N.F32
    kv = keys.cuda().to(dt)                                  # [E, d_in, d_out]
    gd = go.cuda().to(dt).reshape(-1, H).contiguous()
    xd = x.cuda().reshape(-1, D).contiguous()
    rw = w.cuda().reshape(-1).contiguous()
    R = sel.numel()
    offs = C._offsets_for(s.sel, E)
    rp = s.out_index if s.out_index is not None else s.sel_index
    rpos = C._route_pos(rp, R)
    ws_b = lib.cvmm_bwd_x_workspace_bytes(R, E, D, H, R, 1, 1, 1 if s.out_index is not None else 0, K,
                                          N.dtype_id(dt), op, 1, 0)

    def call(fill):
        ws = torch.full((max(ws_b, 1),), fill, dtype=torch.uint8, device="cuda")
        gx = torch.empty(R, D, dtype=dt, device="cuda")
        grw = torch.empty(R, dtype=torch.float32, device="cuda")
        N.check(lib.cvmm_bwd_x(N.ptr(gd), N.dtype_id(dt), gd.shape[0], gd.stride(0), N.ptr(kv), N.dtype_id(dt), E,
                               D, H, *kv.stride(), N.ptr(s.sel), N.ptr(s.sel_index), N.ptr(s.out_index), R,
                               N.ptr(offs), N.ptr(rpos), N.ptr(rw), N.F32, K, N.ptr(xd), N.dtype_id(dt), R, D, op,
                               N.ptr(gx), N.dtype_id(dt), R, D, N.ptr(grw), N.F32, 0, N.ptr(ws), ws_b, st),
                "cvmm_bwd_x")
        torch.cuda.synchronize()
        return gx, grw

    assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, ring_tile) == 0
    try:
        gx0, grw0 = call(0)
        gx1, grw1 = call(0xFF)
    finally:
        lib.cvmm_tuning_set(N.TUNE_RING_TILE, 0)
    assert torch.equal(grw0, grw1) and torch.equal(gx0, gx1)
    assert torch.isfinite(grw1).all()
    badc = bad.reshape(-1).cuda()
    assert torch.all(grw1[badc] == 0)
    sel_ok = sel.clone()
    sel_ok[bad] = 0
    w_ok = w.clone()
    w_ok[bad] = 0
    exp = U.run_oracle(x, keys, sel_ok, w_ok, go, True, amp)
    keep = ~bad.reshape(-1).numpy()
    err = U.norm_rel(U.to_np(grw1)[keep], exp["weights_grad"].reshape(-1)[keep])
    assert err <= (2e-2 if amp else 1e-4), err


@pytest.mark.parametrize("R,E", [(4000, 16), (524288, 256), (262144, 1000)])
def test_sort_invalid_ids_go_last(R, E):
    """Ids outside [0, E) are counted, sorted stably after all valid routes and
    never read by the GEMMs.  The larger cases (SwitchHead's 524288 routes
    over 256 experts; 1000 experts) have count matrices large enough for the
    one-pass column scan."""
    g = torch.Generator().manual_seed(5)
    sel = torch.randint(-3, E + 4, (R,), generator=g)
    raw = sel.to(torch.int32).cuda()
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    ssel = torch.empty(R, dtype=torch.int32, device="cuda")
    perm = torch.empty(R, dtype=torch.int64, device="cuda")
    off = torch.empty(E, dtype=torch.int64, device="cuda")
    nin = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.full((R,), -1, dtype=torch.int32, device="cuda")
    ws_b = lib.cvmm_sort_workspace_bytes(R, E)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    N.check(lib.cvmm_sort_routes(N.ptr(raw), 0, R, E, 1, N.ptr(ssel), N.ptr(perm), None, N.ptr(off), N.ptr(pos),
                                 N.ptr(nin), N.ptr(ws), ws_b, N.stream_of(raw.device)), "sort")
    s = sel.numpy()
    valid = (s >= 0) & (s < E)
    key = np.where(valid, s, E)
    exp_perm = np.argsort(key, kind="stable")
    assert int(nin.item()) == int((~valid).sum())
    assert np.array_equal(perm.cpu().numpy(), exp_perm)
    inv = np.empty_like(exp_perm)
    inv[exp_perm] = np.arange(R)
    assert np.array_equal(pos.cpu().numpy(), inv)
    assert np.array_equal(ssel.cpu().numpy(), s[exp_perm].astype(np.int32))
    assert np.array_equal(off.cpu().numpy(), np.cumsum(np.bincount(s[valid], minlength=E)))


# ---------------------------------------------------------------------------
# more paths
# ---------------------------------------------------------------------------

def _rand_case(seed, B, T, D, H, E, K, weighted=False, route_input=False, x_dt=torch.bfloat16,
               k_dt=torch.float32, skew=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((B, T, K, D) if route_input else (B, T, D)), generator=g).to(x_dt)
    keys = (torch.randn(E, D, H, generator=g) / D ** 0.5).to(k_dt)
    if skew is None:
        sel = torch.randint(0, E, (B, T, K), generator=g)
    else:  # expert 0 takes `skew` of all routes
        sel = torch.randint(1, E, (B, T, K), generator=g)
        hot = torch.rand(B, T, K, generator=g) < skew
        sel[hot] = 0
    w = torch.rand(B, T, K, generator=g) if weighted else None
    go = torch.randn(*((B, T, H) if weighted else (B, T, K, H)), generator=g).to(
        x_dt if x_dt != torch.float32 else torch.bfloat16)
    return x, keys, sel, w, go


@pytest.fixture
def small_wgrad_chunks():
    """Weight-gradient chunks of 1024 routes, so that the hot expert of these
    cases (~6000 routes) is split into several chunks."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 1024) == 0
    yield
    lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 0)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True), (True, False), (False, True)])
def test_hot_expert_split_reduction(weighted, route_input, reduce_mode, small_wgrad_chunks):
    """One expert holds ~70% of the routes: its weight gradient is split into
    several route chunks reduced in a fixed order."""
    x, keys, sel, w, go = _rand_case(11, 4, 512, 128, 96, 8, 4, weighted, route_input, skew=0.7)
    got = U.run_hip(x, keys, sel, w, go, route_input, True)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    U.compare(got, exp, 2e-2)


def test_hot_expert_unsplit_and_split_agree():
    """The same hot-expert case under the built-in chunk (not split at ~6000
    routes) and under 1024-route chunks (split, partials summed in chunk
    order): both against the oracle, and within a few fp32 roundings of each
    other."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    x, keys, sel, w, go = _rand_case(13, 4, 512, 128, 96, 8, 4, True, True, skew=0.7)
    one = U.run_hip(x, keys, sel, w, go, True, True)
    try:
        assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 1024) == 0
        split = U.run_hip(x, keys, sel, w, go, True, True)
    finally:
        lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 0)
    exp = U.run_oracle(x, keys, sel, w, go, True, True)
    U.compare(one, exp, 2e-2)
    U.compare(split, exp, 2e-2)
    assert U.norm_rel(U.to_np(one["keys_grad"]), U.to_np(split["keys_grad"])) <= 1e-5


def test_weight_grad_is_deterministic(small_wgrad_chunks):
    x, keys, sel, w, go = _rand_case(12, 4, 512, 128, 96, 8, 4, True, True, skew=0.7)
    a = U.run_hip(x, keys, sel, w, go, True, True)
    b = U.run_hip(x, keys, sel, w, go, True, True)
    for n in ("out", "x_grad", "keys_grad", "weights_grad"):
        assert torch.equal(a[n], b[n]), n


@pytest.mark.parametrize("weighted,route_input,D,H,amp", [
    (False, False, 128, 96, torch.bfloat16), (True, True, 128, 96, torch.bfloat16),
    (False, False, 512, 384, torch.bfloat16), (True, True, 384, 512, torch.bfloat16),
    (True, False, 512, 256, torch.float16),
])
def test_weight_grad_order_and_tile_do_not_change_bits(weighted, route_input, D, H, amp, small_wgrad_chunks):
    """Every workgroup order and dW tile of the weight-gradient kernel sums
    each element over the same 32-route slices and the same split chunks in
    the same order: identical bits, hot expert (split into chunks) included.
    Widths cover partial coarse tiles (128 x 96 under a 256 x 256 tile) and
    full ones; one case runs the fp16 kernels."""
    from cvmm_codex_amd import _native as N
    x, keys, sel, w, go = _rand_case(31, 4, 512, D, H, 8, 4, weighted, route_input, skew=0.7,
                                     x_dt=amp)
    lib = N.lib()
    ref = None
    try:
        for order in (1, 2, 3):
            for tile in (1, 2, 3, 4, 5):
                assert lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, order) == 0
                assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, tile) == 0
                got = U.run_hip(x, keys, sel, w, go, route_input, True, amp_dtype=amp)
                if ref is None:
                    ref = got
                else:
                    assert torch.equal(ref["keys_grad"], got["keys_grad"]), (order, tile)
    finally:
        lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, 0)
        lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 0)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True,
                       amp_dtype="float16" if amp == torch.float16 else "bfloat16")
    U.compare(ref, exp, 2e-2)


def test_weight_grad_built_in_coarse_tile_matches_base_bits():
    """1024 x 1024 dW over 64 experts and 65536 routes: the built-in choice is
    the 256 x 256 tile (grid >= 4 workgroups per CU); its bits equal the
    128 x 128 tile's, which the oracle tests pin."""
    from cvmm_codex_amd import _native as N
    x, keys, sel, w, go = _rand_case(41, 2, 4096, 1024, 1024, 64, 8, False, False, skew=0.3)
    lib = N.lib()
    try:
        auto = U.run_hip(x, keys, sel, w, go, False, True)
        assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 1) == 0
        base = U.run_hip(x, keys, sel, w, go, False, True)
    finally:
        lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 0)
    assert torch.equal(auto["keys_grad"], base["keys_grad"])
    assert torch.isfinite(auto["keys_grad"]).all() and auto["keys_grad"].abs().max() > 0


@pytest.mark.parametrize("weighted,route_input,skew", [(False, False, None), (True, True, 0.7), (True, False, 0.0)])
def test_gemm_order_does_not_change_bits(weighted, route_input, skew):
    """Expert-major and token-major m-tile orders of the routed GEMMs compute
    every tile the same way: identical bits for every output."""
    from cvmm_codex_amd import _native as N
    x, keys, sel, w, go = _rand_case(33, 4, 512, 256, 192, 24, 6, weighted, route_input, skew=skew)
    lib = N.lib()
    try:
        assert lib.cvmm_tuning_set(N.TUNE_GEMM_ORDER, 1) == 0
        a = U.run_hip(x, keys, sel, w, go, route_input, True)
        assert lib.cvmm_tuning_set(N.TUNE_GEMM_ORDER, 2) == 0
        b = U.run_hip(x, keys, sel, w, go, route_input, True)
    finally:
        lib.cvmm_tuning_set(N.TUNE_GEMM_ORDER, 0)
    for n in ("out", "x_grad", "keys_grad", "weights_grad"):
        if a[n] is None:
            assert b[n] is None
        else:
            assert torch.equal(a[n], b[n]), n
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    U.compare(b, exp, 2e-2)


@pytest.mark.parametrize("weighted,route_input,D,H,skew", [
    (False, False, 256, 128, None),   # long-K forward, one n tile
    (True, True, 128, 256, 0.7),      # long-K weighted grad-input with the routing-weight gradient, hot expert
    (False, False, 384, 256, None),   # long-K forward, two n tiles
    (True, False, 256, 384, 0.0),     # both products long-K
    (False, True, 512, 512, 0.5),     # both products 256 x 256 where chosen, hot expert
    (True, False, 256, 512, 0.5),     # 256 x 256 grad-input with the routing-weight gradient
])
def test_long_k_tile_height_does_not_change_bits(weighted, route_input, D, H, skew):
    """128- and 160-row m-tiles of the long-K routed GEMM, and its eight-wave
    256 x 256 tiles (where N is a multiple of 256; with the routing-weight
    gradient one partial per 128-column half), run every row's k slices in
    the same order: identical bits, and the oracle's values."""
    from cvmm_codex_amd import _native as N
    x, keys, sel, w, go = _rand_case(35, 4, 384, D, H, 12, 6, weighted, route_input, skew=skew)
    lib = N.lib()
    runs = []
    try:
        for t in (1, 2, 3):
            assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, t) == 0
            runs.append(U.run_hip(x, keys, sel, w, go, route_input, True))
    finally:
        lib.cvmm_tuning_set(N.TUNE_RING_TILE, 0)
    a = runs[0]
    for t, b in zip((2, 3), runs[1:]):
        for n in ("out", "x_grad", "keys_grad", "weights_grad"):
            if a[n] is None:
                assert b[n] is None
            else:
                assert torch.equal(a[n], b[n]), (t, n)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    for b in runs[1:]:
        U.compare(b, exp, 2e-2)


@pytest.mark.parametrize("op", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,H,weighted,route_input,tile", [
    (1024, 128, False, False, 2),   # forward 160 x 128 (ff_up); grad-input: short K
    (256, 128, False, False, 1),    # forward 128 x 128
    (512, 64, False, False, 0),     # forward 256 x 64 with fragment read-ahead
    (128, 1024, True, True, 2),     # grad-input 160 x 128 with the routing-weight gradient (ff_down)
    (64, 512, True, True, 0),       # grad-input 256 x 64 + routing-weight gradient (SwitchHead O)
    (512, 256, False, False, 1),    # both products long-K
    (200, 96, True, False, 0),      # d_in % 64 != 0: the last k slice part-filled
    (512, 256, False, False, 3),    # both products 256 x 256, eight waves
    (256, 512, False, True, 3),     # both 256 x 256, route input
    (200, 512, True, False, 3),     # weighted forward 256 x 256 with a part-filled last k slice
    (512, 256, True, True, 3),      # grad-input 256 x 256 + routing-weight gradient
])
def test_long_k_reads_either_weight_orientation(D, H, weighted, route_input, tile, op):
    """The long-K routed GEMM reads the weights k-contiguous ([n][k] rows: the
    copy in its own orientation) or n-contiguous ([k][n] rows: the other
    orientation's copy, through transposed LDS reads).  Both give the same
    bits, for the forward and for the input gradient (with the routing-weight
    gradient when weighted), at every tile shape, and the oracle's values."""
    from cvmm_codex_amd import _native as N

    class Ctx:
        op_type = op

    lib = N.lib()
    E, K = 8, 4
    x, keys, sel, w, go = _rand_case(91 + D + H, 2, 160, D, H, E, K, weighted, route_input, x_dt=op)
    s = C.cvmm_prepare_sel2(sel.cuda(), w.cuda() if weighted else None, route_input=route_input)
    s._resolve(E)
    xd, kd, gd = x.cuda(), keys.cuda(), go.cuda()
    wd = w.cuda() if weighted else None
    kt = kd.transpose(1, 2).contiguous().to(op)   # [E, d_out, d_in]: k-contiguous forward rows
    kn = kd.to(op)                                 # [E, d_in, d_out]: k-contiguous grad-input rows
    outs = {}
    try:
        assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, tile) == 0
        assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 1) == 0   # the routed GEMMs, not a dense top-k sum
        for name, (k_fwd, fwd_t, k_bwd, bwd_t) in {"own": (kt, True, kn, False),
                                                   "other": (kn, False, kt, True)}.items():
            y = C._forward(xd, s.sel_index, s.sel, kd, s.out_index, wd, op, k_fwd, fwd_t)
            gx, _, grw = C._backward(Ctx, gd, xd, kd, s.raw_sel, s.sel, s.sel_index, s.out_index, wd, True, False,
                                     weighted, keys_x=k_bwd, keys_x_is_t=bwd_t)
            torch.cuda.synchronize()
            outs[name] = (y, gx, grw)
    finally:
        lib.cvmm_tuning_set(N.TUNE_RING_TILE, 0)
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    # bits compared where the product is long-K (the short-K one falls back
    # to the general kernel for the other orientation: checked on values)
    for a, b, what, long_k in zip(outs["own"], outs["other"], ("out", "x_grad", "weights_grad"),
                                  (D > 128, H > 128, H > 128)):
        if a is None:
            assert b is None
        elif long_k:
            assert torch.equal(a, b), what
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True,
                       amp_dtype="bfloat16" if op == torch.bfloat16 else "float16")
    y, gx, grw = outs["other"]
    assert U.norm_rel(U.to_np(y), exp["out"].reshape(y.shape)) <= 2e-2
    assert U.norm_rel(U.to_np(gx).reshape(exp["x_grad"].shape), exp["x_grad"]) <= 2e-2
    if weighted:
        assert U.norm_rel(U.to_np(grw).reshape(exp["weights_grad"].shape), exp["weights_grad"]) <= 2e-2


@pytest.mark.parametrize("H", [128, 512])
def test_long_k_gelu_epilogue_tile_height_does_not_change_bits(H):
    """The GELU epilogue of the long-K forward at every tile shape (256 x 256
    where H is a multiple of 256)."""
    from cvmm_codex_amd import _native as N
    import cvmm_codex_amd.api as C
    x, keys, sel, _, go = _rand_case(36, 4, 384, 256, H, 12, 6)
    lib = N.lib()
    outs = []
    try:
        for t in (1, 2, 3):
            assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, t) == 0
            xd, kd = x.cuda().requires_grad_(True), keys.cuda().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = C.cvmm_gelu(xd, C.cvmm_prepare_sel2(sel.cuda()), kd)
            y.backward(go.cuda().to(y.dtype))
            torch.cuda.synchronize()
            outs.append((y.detach(), xd.grad, kd.grad))
    finally:
        lib.cvmm_tuning_set(N.TUNE_RING_TILE, 0)
    for other in outs[1:]:
        for u, v in zip(outs[0], other):
            assert torch.equal(u, v)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True), (True, False)])
def test_route_positions_from_sort_or_computed(weighted, route_input):
    """The route-ordered rows are gathered per token through the sort's
    inverse permutation; a selector built by hand (indices without it) makes
    the call compute the inverse itself.  Both give the same bits."""
    x, keys, sel, w, go = _rand_case(21, 3, 200, 128, 256, 7, 4, weighted, route_input)
    a = U.run_hip(x, keys, sel, w, go, route_input, True)

    def manual(sel_d, w_d, route_input):
        s = C.cvmm_prepare_sel2(sel_d, w_d, route_input=route_input)
        s._resolve(keys.shape[0])
        return C.CVMMSel(s.raw_sel, s.sel, s.sel_index.clone(),
                         None if s.out_index is None else s.out_index.clone(), s.reduction_weight)

    b = U.run_hip(x, keys, sel, w, go, route_input, True, prepare=manual)
    for n in ("out", "x_grad", "keys_grad", "weights_grad"):
        if a[n] is None:
            assert b[n] is None
        else:
            assert torch.equal(a[n], b[n]), n


def test_fp16_autocast():
    x, keys, sel, w, go = _rand_case(13, 2, 64, 96, 80, 6, 2, x_dt=torch.float16)
    got = U.run_hip(x, keys, sel, w, go.to(torch.float16), False, True, amp_dtype=torch.float16)
    exp = U.run_oracle(x, keys, sel, w, go.to(torch.float16), False, True, amp_dtype="float16")
    U.compare(got, exp, 2e-2)


@pytest.mark.parametrize("route_input,D,amp", [(True, 256, torch.float16), (False, 256, torch.float16),
                                               (True, 200, torch.bfloat16), (True, 40, torch.bfloat16)])
def test_weighted_long_k_routing_weight_grad(route_input, D, amp):
    """The long-K kernels with the weighted epilogue and the routing-weight
    gradient (d_out = 320 > 128 on the input gradient): fp16, a last n tile
    of 72 columns (d_in = 200) and a single narrow tile (d_in = 40)."""
    x, keys, sel, w, go = _rand_case(15, 2, 256, D, 320, 8, 4, True, route_input, x_dt=amp)
    op = "float16" if amp == torch.float16 else "bfloat16"
    got = U.run_hip(x, keys, sel, w, go.to(amp), route_input, True, amp_dtype=amp)
    exp = U.run_oracle(x, keys, sel, w, go.to(amp), route_input, True, amp_dtype=op)
    U.compare(got, exp, 2e-2)


@pytest.mark.parametrize("route_input", [True, False])
def test_routing_weight_grad_with_misaligned_x_rows(route_input):
    """x as a view one element into rows of 257: neither its address nor its
    row stride is 8-byte aligned.  The forward and the weight gradient take
    the general kernels; the grad-input GEMM (aligned grad operand, d_out =
    320) with its routing-weight gradient takes the tiled kernel, which reads
    x element by element (the long-K kernel reads only 8-byte pieces)."""
    x, keys, sel, w, go = _rand_case(16, 2, 128, 256, 320, 8, 4, True, route_input)
    dev = torch.device("cuda")
    base = torch.zeros(*x.shape[:-1], x.shape[-1] + 1, dtype=x.dtype, device=dev)
    base[..., 1:] = x.to(dev)
    xd = base[..., 1:].requires_grad_(True)
    assert xd.data_ptr() % 8 != 0 and xd.stride(-2) == 257
    kd = keys.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    s = C.cvmm_prepare_sel2(sel.to(dev), wd, route_input=route_input)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(xd, s, kd)
    y.backward(go.to(dev).to(y.dtype))
    torch.cuda.synchronize()
    got = {"out": y.detach(), "x_grad": xd.grad, "keys_grad": kd.grad, "weights_grad": wd.grad}
    U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


@pytest.mark.parametrize("D,H,route_input", [(96, 80, False), (128, 320, True), (64, 256, True)])
def test_fp32_x_under_autocast(D, H, route_input):
    """fp32 activations with bf16 autocast: cast to bf16 inside the kernels.
    With route input and d_out > 128 the grad-input GEMM is long-K and its
    routing-weight gradient reads fp32 x rows (the tiled kernel's path)."""
    x, keys, sel, w, go = _rand_case(14, 2, 64, D, H, 6, 3, True, route_input, x_dt=torch.float32)
    got = U.run_hip(x, keys, sel, w, go, route_input, True)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    U.compare(got, exp, 2e-2)


def test_transposed_keys_view():
    """keys given as a transposed view (unit stride on d_in)."""
    x, keys, sel, w, go = _rand_case(15, 2, 64, 64, 96, 5, 2)
    kt = keys.transpose(1, 2).contiguous().transpose(1, 2)
    assert kt.stride(1) == 1
    got = U.run_hip(x, kt, sel, w, go, False, True)
    exp = U.run_oracle(x, keys, sel, w, go, False, True)
    U.compare(got, exp, 2e-2)


def test_stride0_grad_output():
    """``out.sum().backward()`` (the reference benchmark) passes an expanded grad."""
    x, keys, sel, _, _ = _rand_case(16, 2, 64, 64, 48, 5, 3)
    dev = torch.device("cuda")
    xd = x.to(dev).requires_grad_(True)
    kd = keys.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(xd, C.cvmm_prepare_sel2(sel.to(dev)), kd)
    y.sum().backward()
    ones = torch.ones(y.shape, dtype=torch.bfloat16)
    exp = U.run_oracle(x, keys, sel, None, ones, False, True)
    U.compare({"out": y, "x_grad": xd.grad, "keys_grad": kd.grad}, exp, 2e-2,
              names=("out", "x_grad", "keys_grad"))


def test_empty_selection():
    dev = torch.device("cuda")
    x = torch.randn(0, 16, device=dev, requires_grad=True)
    keys = torch.randn(4, 16, 8, device=dev, requires_grad=True)
    sel = torch.zeros(0, 2, dtype=torch.int64, device=dev)
    y = C.cvmm(x, C.cvmm_prepare_sel2(sel), keys)
    assert y.shape == (0, 2, 8)
    y.sum().backward()
    assert torch.equal(keys.grad, torch.zeros_like(keys))


# ---------------------------------------------------------------------------
# BASELINE configs at full size
# ---------------------------------------------------------------------------

def test_config_tiny_fp32():
    import workloads as W
    p = W.c1_tiny()
    got = U.run_hip(p.x, p.keys, p.sel, p.weights, p.grad_out, p.route_input, p.amp)
    exp = U.run_oracle(p.x, p.keys, p.sel, p.weights, p.grad_out, p.route_input, p.amp)
    U.compare(got, exp, 1e-4)


@pytest.mark.parametrize("name", ["ff_up_1024", "ff_down_1024_weighted"])
def test_config_ff_projections(name, reduce_mode):
    import workloads as W
    p = W.PROJECTIONS[name]()
    got = U.run_hip(p.x, p.keys, p.sel, p.weights, p.grad_out, p.route_input, p.amp)
    exp = U.run_oracle(p.x, p.keys, p.sel, p.weights, p.grad_out, p.route_input, p.amp, compute=np.float32)
    U.compare(got, exp, 2e-2)


@pytest.mark.parametrize("route_input", [False, True])
@pytest.mark.parametrize("D,H", [(600, 72), (64, 130), (200, 8)])
def test_small_fp32_problems(D, H, route_input):
    """fp32 problems small enough for the 16 x 64 routed-product tiles and
    the per-expert 64 x 64 weight-gradient blocks (cvmm_small.hip): K over
    several rounds of 256 with a ragged tail (600), ragged output columns,
    both weight orientations (forward n-contiguous, grad-input k-contiguous),
    an expert with more than 128 routes (weight-gradient rounds) and
    out-of-range ids, against the oracle at the fp32 tolerance."""
    x, keys, sel, w, go = _rand_case(31 + D + H, 2, 96, D, H, 5, 4, False, route_input, x_dt=torch.float32)
    sel[0, :40, 0] = 7       # out of range for 5 experts: left out, their rows zero
    go = go.float()
    got = U.run_hip(x, keys, sel, w, go, route_input, False)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, False)
    U.compare(got, exp, 1e-4)


@pytest.mark.parametrize("weighted,route_input,D,H,lowmem,x_dt", [
    (False, False, 256, 128, 0, torch.bfloat16),   # token input: route-buffer grad-input + top-k sum
    (True, True, 128, 256, 0, torch.bfloat16),     # weighted route input: routing-weight gradient too
    (True, False, 512, 256, 0, torch.bfloat16),    # weighted token input, both products long-K
    (False, False, 128, 256, 2, torch.bfloat16),   # low-memory slices of the top-k sum (an early return)
    (False, False, 256, 256, 0, torch.float32),    # fp32 x under bf16 autocast: converted x rows
])
def test_backward_on_two_streams_gives_the_same_bits(weighted, route_input, D, H, lowmem, x_dt, monkeypatch):
    """With cvmm_overlap_backward the weight gradient runs on a second stream,
    forked from and joined back into the caller's stream: the same kernels,
    so every gradient has the one-stream bits, on every return path (x in
    another dtype: the converted rows live until the join)."""
    x, keys, sel, w, go = _rand_case(71 + D + H + lowmem, 2, 256, D, H, 16, 4, weighted, route_input, skew=0.5,
                                     x_dt=x_dt)
    monkeypatch.setattr(C, "cvmm_lowmem_chunk_size", lowmem)
    runs = []
    for overlap in (False, True, True):
        monkeypatch.setattr(C, "cvmm_overlap_backward", overlap)
        runs.append(U.run_hip(x, keys, sel, w, go, route_input, True))
    for r in runs[1:]:
        for n in ("out", "x_grad", "keys_grad", "weights_grad"):
            if runs[0][n] is None:
                assert r[n] is None
            else:
                assert torch.equal(runs[0][n], r[n]), n
    U.compare(runs[1], U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)
