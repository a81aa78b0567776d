"""Pins the CPU oracle (oracle/cvmm_oracle.py) before anything is compared to it.

Every oracle function is checked against something that is not the oracle's
own formula: golden fixtures from the reference test's einsum definition,
brute-force loops, closed forms and torch's dtype conversions.  The last block
plants mistakes in the oracle and checks that the golden comparison catches
each of them.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import cvmm_oracle as O
from tests import golden_data as G
from tests import oracle_run

FIXTURES = G.fixtures()


# ---------------------------------------------------------------------------
# rounding emulation vs torch conversions
# ---------------------------------------------------------------------------

def _special_values():
    rng = np.random.default_rng(0)
    v = rng.standard_normal(20000).astype(np.float32) * np.float32(3.0)
    # exact bf16 ties (low half == 0x8000) with both parities of the kept bit
    ties = (rng.integers(0, 1 << 15, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    extra = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38, 65504.0, 65520.0,
                      6e-8, 1e-45], dtype=np.float32)
    return np.concatenate([v, ties[np.isfinite(ties)], extra])


def test_bf16_rounding_matches_torch():
    v = _special_values()
    ours = O.rnd(v, "bfloat16", np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    nan = O.rnd(np.array([np.nan], np.float32), "bfloat16", np.float32)
    assert np.isnan(nan).all()


def test_f16_rounding_matches_torch():
    v = _special_values()
    ours = O.rnd(v, "float16", np.float32)
    ref = torch.from_numpy(v).to(torch.float16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# selector metadata
# ---------------------------------------------------------------------------

def _brute_sort(flat):
    perm = sorted(range(len(flat)), key=lambda i: (int(flat[i]), i))   # stable by construction
    return np.array([flat[i] for i in perm], dtype=np.int32), np.array(perm, dtype=np.int64)


@pytest.mark.parametrize("shape,E", [((3, 5, 3), 7), ((2, 9, 1), 13), ((1, 5, 2), 32), ((4, 64, 8), 16), ((1,), 3)])
def test_prepare_sel2_matches_brute_force(shape, E):
    rng = np.random.default_rng(sum(shape) + E)
    sel = rng.integers(0, E, shape)
    k = shape[-1]
    ssel, perm = _brute_sort(sel.reshape(-1))
    m = O.prepare_sel2(sel)
    assert np.array_equal(m.raw_sel.reshape(-1), sel.reshape(-1).astype(np.int32))
    assert np.array_equal(m.sel.reshape(-1), ssel)
    assert np.array_equal(m.out_index, perm)
    assert np.array_equal(m.sel_index, perm // k)
    r = O.prepare_sel2(sel, route_input=True)
    assert r.out_index is None and np.array_equal(r.sel_index, perm)
    p = O.prepare_sel(sel, E)
    assert p.out_index is None and np.array_equal(p.sel_index, perm)
    assert m.sel.dtype == np.int32 and m.sel_index.dtype == np.int64


def test_reused_selector_matches_fresh():
    """test_cvmm_correctness.py:121-137: a route-input selector re-wrapped from
    the up-projection one is identical to a freshly prepared one."""
    rng = np.random.default_rng(1251)
    sel = rng.integers(0, 7, (3, 5, 3))
    w = rng.standard_normal((3, 5, 3)).astype(np.float32)
    x = rng.standard_normal((3, 5, 3, 16)).astype(np.float32)
    keys = rng.standard_normal((7, 16, 11)).astype(np.float32)
    reused = O.prepare_sel2(O.prepare_sel2(sel), w, route_input=True)
    fresh = O.prepare_sel2(sel, w, route_input=True)
    assert np.array_equal(reused.sel_index, fresh.sel_index) and reused.out_index is None
    a = O.forward(x, reused, keys, "bfloat16", "bfloat16")
    b = O.forward(x, fresh, keys, "bfloat16", "bfloat16")
    assert np.array_equal(a, b)


def _offsets_unique_consecutive(sorted_sel, E):
    """The reference's torch fallback (cvmm.py:72-77), used by its own offsets test."""
    s = torch.from_numpy(np.asarray(sorted_sel, dtype=np.int32))
    u, c = torch.unique_consecutive(s, return_counts=True)
    if u.numel() == E:
        return c.cumsum(0).numpy()
    ec = torch.zeros(E, dtype=c.dtype)
    ec[u.long()] = c
    return ec.cumsum(0).numpy()


@pytest.mark.parametrize("E,R", list(itertools.product((1, 7, 64, 512), (1, 13, 1000))))
def test_expert_offsets(E, R):
    """Grid of test_cvmm_correctness.py:73-86, plus bincount as a second pin."""
    rng = np.random.default_rng(E * 1000 + R)
    s = np.sort(rng.integers(0, E, R)).astype(np.int32)
    off = O.expert_offsets(s, E)
    assert off.dtype == np.int64
    assert np.array_equal(off, _offsets_unique_consecutive(s, E))
    assert np.array_equal(off, np.cumsum(np.bincount(s, minlength=E)))


# ---------------------------------------------------------------------------
# forward/backward vs golden fixtures (reference einsum definition, fp64)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("fx", FIXTURES, ids=lambda f: f.name)
def test_oracle_exact_matches_golden(fx):
    got = oracle_run.run(fx, exact=True)
    exp = oracle_run.expected(fx)
    for name in ("out", "x_grad", "keys_grad", "weights_grad"):
        if exp[name] is None:
            assert got[name] is None
            continue
        assert got[name].shape == exp[name].shape, name
        assert G.norm_rel(got[name], exp[name]) < 1e-12, name


@pytest.mark.parametrize("fx", FIXTURES, ids=lambda f: f.name)
def test_oracle_rounded_within_reference_tolerance(fx):
    """With the reference's rounding points emulated, the oracle stays inside
    the reference harness's own tolerance table (:47-66) of the exact result."""
    got = oracle_run.run(fx, exact=False)
    exp = oracle_run.expected(fx)
    for name in ("out", "x_grad", "keys_grad", "weights_grad"):
        if exp[name] is None:
            continue
        atol, rtol = G.TOLERANCES[fx.mode][name]
        np.testing.assert_allclose(got[name], exp[name], atol=atol, rtol=rtol, err_msg=name)
        assert G.norm_rel(got[name], exp[name]) < G.NORM_REL[fx.mode] * (1 if fx.mode == "float32" else 1.5), name


# ---------------------------------------------------------------------------
# brute force and closed forms
# ---------------------------------------------------------------------------

def _brute(x, sel, keys, w, gy, route_input):
    """Pure-Python loops over (token, slot, i, j): forward and all gradients."""
    B, T, K = sel.shape
    NE, N, E = keys.shape
    out = np.zeros((B, T, K, E))
    dx = np.zeros(x.shape)
    dk = np.zeros(keys.shape)
    for b in range(B):
        for t in range(T):
            for k in range(K):
                e = sel[b, t, k]
                xv = x[b, t, k] if route_input else x[b, t]
                for j in range(E):
                    out[b, t, k, j] = sum(xv[i] * keys[e, i, j] for i in range(N))
    if w is None:
        res, g_route = out, gy
    else:
        res = np.zeros((B, T, E))
        for b, t, k in itertools.product(range(B), range(T), range(K)):
            res[b, t] += w[b, t, k] * out[b, t, k]
        g_route = np.zeros((B, T, K, E))
        for b, t, k in itertools.product(range(B), range(T), range(K)):
            g_route[b, t, k] = w[b, t, k] * gy[b, t]
    dw = None if w is None else np.zeros(w.shape)
    for b, t, k in itertools.product(range(B), range(T), range(K)):
        e = sel[b, t, k]
        for i in range(N):
            xi = x[b, t, k, i] if route_input else x[b, t, i]
            acc = 0.0
            for j in range(E):
                dk[e, i, j] += xi * g_route[b, t, k, j]
                acc += keys[e, i, j] * g_route[b, t, k, j]
            if route_input:
                dx[b, t, k, i] += acc
            else:
                dx[b, t, i] += acc
        if w is not None:
            dw[b, t, k] = sum(out[b, t, k, j] * gy[b, t, j] for j in range(E))
    return res, dx, dk, dw


@pytest.mark.parametrize("weighted,route_input,K", [(False, False, 3), (True, False, 2), (True, True, 3), (False, True, 2), (False, False, 1)])
def test_oracle_matches_brute_force(weighted, route_input, K):
    rng = np.random.default_rng(7 + K + 2 * weighted + 4 * route_input)
    B, T, N, E, NE = 2, 3, 5, 4, 6
    sel = rng.integers(0, NE, (B, T, K))
    x = rng.standard_normal((B, T, K, N) if route_input else (B, T, N))
    keys = rng.standard_normal((NE, N, E))
    w = rng.standard_normal((B, T, K)) if weighted else None
    gy = rng.standard_normal((B, T, E) if weighted else (B, T, K, E))
    meta = O.prepare_sel2(sel, w, route_input=route_input)
    y = O.forward(x, meta, keys)
    dx, dk, dw = O.backward(x, meta, keys, gy)
    r, rdx, rdk, rdw = _brute(x, sel, keys, w, gy, route_input)
    assert G.norm_rel(y, r) < 1e-12
    assert G.norm_rel(dx, rdx) < 1e-12
    assert G.norm_rel(dk, rdk) < 1e-12
    if weighted:
        assert G.norm_rel(dw, rdw) < 1e-12


def test_top1_is_dense_per_token_gemm():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 9, 17))
    keys = rng.standard_normal((13, 17, 9))
    sel = rng.integers(0, 13, (2, 9, 1))
    y = O.forward(x, O.prepare_sel2(sel), keys)
    ref = np.stack([np.stack([x[b, t] @ keys[sel[b, t, 0]] for t in range(9)]) for b in range(2)])
    assert G.norm_rel(y[:, :, 0], ref) < 1e-13


def test_single_expert_is_plain_gemm():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 24))
    keys = rng.standard_normal((1, 24, 12))
    gy = rng.standard_normal((40, 1, 12))
    sel = np.zeros((40, 1), dtype=np.int64)
    meta = O.prepare_sel2(sel)
    y = O.forward(x, meta, keys)
    assert G.norm_rel(y[:, 0], x @ keys[0]) < 1e-13
    dx, dk, _ = O.backward(x, meta, keys, gy)
    assert G.norm_rel(dx, gy[:, 0] @ keys[0].T) < 1e-13
    assert G.norm_rel(dk[0], x.T @ gy[:, 0]) < 1e-13


def test_empty_experts_have_zero_weight_grad():
    rng = np.random.default_rng(5)
    NE = 32
    sel = rng.integers(0, 4, (1, 5, 2)) * 5          # only experts {0,5,10,15}
    x = rng.standard_normal((1, 5, 15))
    keys = rng.standard_normal((NE, 15, 10))
    w = rng.standard_normal((1, 5, 2))
    gy = rng.standard_normal((1, 5, 10))
    meta = O.prepare_sel2(sel, w)
    _, dk, _ = O.backward(x, meta, keys, gy)
    used = set(np.unique(sel).tolist())
    for e in range(NE):
        if e not in used:
            assert not dk[e].any()


# ---------------------------------------------------------------------------
# planted mistakes: the golden comparison must catch each one
# ---------------------------------------------------------------------------

def _golden_passes(oracle_mod):
    for fx in FIXTURES:
        if fx.mode != "float32":
            continue
        try:
            got = oracle_run.run(fx, exact=True, oracle=oracle_mod)
        except IndexError:          # a wrong index can also run off the array
            return False
        exp = oracle_run.expected(fx)
        for name in ("out", "x_grad", "keys_grad", "weights_grad"):
            if exp[name] is None:
                continue
            if got[name] is None or got[name].shape != exp[name].shape:
                return False
            if G.norm_rel(got[name], exp[name]) > 1e-6:
                return False
    return True


class _Mutant:
    """A shallow copy of the oracle module with one function replaced."""

    def __init__(self, **overrides):
        self.__dict__.update({k: getattr(O, k) for k in dir(O) if not k.startswith("__")})
        self.__dict__.update(overrides)


def _offsets_off_by_one(s, E):
    return np.searchsorted(np.asarray(s).reshape(-1), np.arange(E), side="left").astype(np.int64)


def _prepare_wrong_rows(sel, w=None, route_input=False):
    m = O.prepare_sel2(sel, w, route_input)
    if m.out_index is not None:
        m.sel_index = m.out_index.copy()          # forgot // top_k
    return m


def _prepare_reversed_weights(sel, w=None, route_input=False):
    m = O.prepare_sel2(sel, w, route_input)
    if w is not None:
        m.reduction_weight = np.ascontiguousarray(w[..., ::-1])
    return m


def _forward_transposed(x, meta, keys, op=None, out=None, compute=np.float64):
    return O.forward(x, meta, np.ascontiguousarray(np.swapaxes(keys, 1, 2)).reshape(keys.shape), op, out, compute)


@pytest.mark.parametrize("mutant", [
    _Mutant(prepare_sel2=_prepare_wrong_rows),
    _Mutant(prepare_sel2=_prepare_reversed_weights),
    _Mutant(forward=_forward_transposed),
], ids=["x-row-index", "weight-order", "transposed-keys"])
def test_golden_catches_planted_mistakes(mutant):
    assert _golden_passes(O)
    assert not _golden_passes(mutant)


def test_golden_catches_offsets_off_by_one(monkeypatch):
    monkeypatch.setattr(O, "expert_offsets", _offsets_off_by_one)
    assert not _golden_passes(O)


# ---------------------------------------------------------------------------
# router oracle (oracle/router_oracle.py) against torch's own CPU routines
# ---------------------------------------------------------------------------

def _torch_router(logits: torch.Tensor, k: int, renormalize: bool):
    """benchmark_ffn_moe.py:92-94 on the CPU in float64."""
    probs = torch.softmax(logits.double(), dim=-1)
    w, sel = probs.topk(k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-20)
    return w, sel


@pytest.mark.parametrize("T,E,k,renorm", [(64, 128, 8, True), (37, 100, 3, False), (16, 64, 64, True),
                                          (9, 1000, 1, True), (33, 17, 17, False)])
def test_router_oracle_matches_torch(T, E, k, renorm):
    from oracle import router_oracle as RO
    g = torch.Generator().manual_seed(T * 1000 + E + k)
    logits = torch.randn(T, E, generator=g) * 3
    w, sel, meta = RO.route_topk(logits.numpy(), k, renorm)
    tw, tsel = _torch_router(logits, k, renorm)
    np.testing.assert_array_equal(sel, tsel.numpy())
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-12, atol=1e-15)
    if renorm:
        np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-12)
    ref = O.prepare_sel2(tsel.numpy())
    np.testing.assert_array_equal(meta.sel, ref.sel)
    np.testing.assert_array_equal(meta.sel_index, ref.sel_index)
    np.testing.assert_array_equal(meta.out_index, ref.out_index)


@pytest.mark.parametrize("E,k,renorm", [(128, 8, True), (128, 8, False), (40, 40, True), (300, 2, True)])
def test_router_oracle_backward_matches_autograd(E, k, renorm):
    from oracle import router_oracle as RO
    g = torch.Generator().manual_seed(E * 7 + k)
    T = 24
    logits = (torch.randn(T, E, generator=g) * 2).double().requires_grad_(True)
    w, sel = _torch_router(logits, k, renorm)
    gw = torch.randn(T, k, generator=g).double()
    w.backward(gw)
    got = RO.route_topk_backward(logits.detach().numpy(), sel.numpy(), gw.numpy(), renorm)
    np.testing.assert_allclose(got, logits.grad.numpy(), rtol=1e-10, atol=1e-13)


def test_router_oracle_ties_go_to_the_lower_id():
    from oracle import router_oracle as RO
    logits = np.array([[0.0, 1.0, 1.0, 0.5, 1.0]])
    w, sel, _ = RO.route_topk(logits, 3, False)
    np.testing.assert_array_equal(sel, [[1, 2, 4]])
    np.testing.assert_allclose(w[0], RO.softmax(logits)[0, [1, 2, 4]])


def test_router_oracle_catches_a_planted_mistake(monkeypatch):
    """A dropped renormalisation term in the backward fails the autograd check."""
    from oracle import router_oracle as RO
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(8, 32, generator=g).double().requires_grad_(True)
    w, sel = _torch_router(logits, 4, True)
    gw = torch.randn(8, 4, generator=g).double()
    w.backward(gw)
    good = RO.route_topk_backward(logits.detach().numpy(), sel.numpy(), gw.numpy(), True)
    bad = RO.route_topk_backward(logits.detach().numpy(), sel.numpy(), gw.numpy(), False)
    assert np.allclose(good, logits.grad.numpy(), rtol=1e-10, atol=1e-13)
    assert not np.allclose(bad, logits.grad.numpy(), rtol=1e-6, atol=1e-9)


def test_oracle_gelu_matches_torch():
    g = torch.Generator().manual_seed(21)
    h = (torch.randn(4096, generator=g) * 3).double().requires_grad_(True)
    y = torch.nn.functional.gelu(h)
    gy = torch.randn(4096, generator=g).double()
    y.backward(gy)
    np.testing.assert_allclose(O.gelu(h.detach().numpy()), y.detach().numpy(), rtol=1e-14, atol=1e-15)
    np.testing.assert_allclose(O.gelu_backward(gy.numpy(), h.detach().numpy()), h.grad.numpy(), rtol=1e-12,
                               atol=1e-14)
    # the derivative against central differences
    x = np.linspace(-6, 6, 97)
    eps = 1e-6
    num = (O.gelu(x + eps) - O.gelu(x - eps)) / (2 * eps)
    np.testing.assert_allclose(O.gelu_backward(np.ones_like(x), x), num, rtol=1e-7, atol=1e-9)
    # bf16 rounding of the stored values, as F.gelu on bf16 tensors
    hb = torch.randn(2048, generator=g).to(torch.bfloat16)
    np.testing.assert_array_equal(O.gelu(hb.float().numpy(), "bfloat16"),
                                  torch.nn.functional.gelu(hb.double()).to(torch.bfloat16).double().numpy())


# ---------------------------------------------------------------------------
# the torch CPU path timed as bench.py's cpu_baseline (oracle/torch_cpu_path.py)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("fx", [f for f in FIXTURES if f.mode == "float32"], ids=lambda f: f.name)
def test_torch_cpu_path_matches_golden(fx):
    """The baseline's torch restatement gives the golden values (the reference
    test's einsum definition, float64) on every golden case."""
    from oracle import torch_cpu_path as P
    t = lambda a: None if a is None else torch.from_numpy(np.asarray(a, dtype=np.float64))
    out, (dx, dw, dg) = P.step(t(fx.x), torch.from_numpy(fx.sel), t(fx.keys), t(fx.weights), t(fx.grad_out),
                               fx.case["route_input"])
    exp = oracle_run.expected(fx)
    for name, got in (("out", out), ("x_grad", dx), ("keys_grad", dw), ("weights_grad", dg)):
        if exp[name] is None:
            assert got is None, name
            continue
        e = np.asarray(exp[name], dtype=np.float64)
        assert got.shape == e.shape, name
        assert np.abs(got.numpy() - e).max() <= 1e-9 * max(np.abs(e).max(), 1.0), name


def test_torch_cpu_path_catches_a_dropped_weight():
    """A planted mistake in the baseline's restatement (the reduction weight
    left out of grad_x) fails the golden comparison."""
    from oracle import torch_cpu_path as P
    fx = next(f for f in FIXTURES if f.mode == "float32" and f.weights is not None and f.case["route_input"])
    t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))
    r = P.Routes(torch.from_numpy(fx.sel), fx.keys.shape[0], True)
    dx, _, _ = P.backward(t(fx.x), r, t(fx.keys), torch.ones_like(t(fx.weights)), t(fx.grad_out))
    e = np.asarray(fx.exp_x_grad, dtype=np.float64)
    assert np.abs(dx.numpy() - e).max() > 1e-3 * np.abs(e).max()
