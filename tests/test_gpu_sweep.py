"""A seeded sweep of random shapes and modes against the CPU oracle.

Each case draws token count, top-k, expert count (many experts empty at
small token counts), both widths around the kernels' switch points (K on
both sides of 64 and 128, N at and around 64, widths that are not multiples
of 8), weighted or unweighted, route or token input, fp32 / bf16 autocast /
fp16 autocast, and optionally one hot expert. The forward output and every
gradient are compared with the oracle at the tolerances of the reference's
correctness harness (benchmark_correctness_original.py:35-66): 1e-4 relative
to the largest magnitude in fp32, 2e-2 under autocast."""
import numpy as np
import pytest
import torch

from tests import gpu_util as U

pytestmark = pytest.mark.gpu

_WIDTHS = (8, 11, 24, 33, 40, 64, 72, 96, 128, 130, 136, 200, 256, 384, 520)
_MODES = {"fp32": (torch.float32, None, 1e-4), "bf16": (torch.bfloat16, torch.bfloat16, 2e-2),
          "bf16_fp32x": (torch.float32, torch.bfloat16, 2e-2), "fp16": (torch.float16, torch.float16, 2e-2)}


def _cases(n=48, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B = int(rng.integers(1, 3))
        T = int(rng.integers(1, 1200))
        D, H = (int(rng.choice(_WIDTHS)) for _ in range(2))
        E = int(rng.choice((1, 2, 7, 16, 64, 130)))
        K = int(rng.choice((1, 2, 4, 8, 12)))
        if B * T * K * D * H > 4e8:
            continue
        weighted = bool(rng.integers(0, 2))
        route_input = bool(rng.integers(0, 2))
        mode = str(rng.choice(list(_MODES)))
        skew = 0.6 if E > 2 and rng.random() < 0.25 else None
        out.append((len(out), B, T, D, H, E, K, weighted, route_input, mode, skew))
    return out


def _make(case):
    seed, B, T, D, H, E, K, weighted, route_input, mode, skew = case
    x_dt, _, _ = _MODES[mode]
    g = torch.Generator().manual_seed(1000 + seed)
    x = torch.randn(*((B, T, K, D) if route_input else (B, T, D)), generator=g).to(x_dt)
    keys = torch.randn(E, D, H, generator=g) / D ** 0.5
    if skew is None:
        sel = torch.randint(0, E, (B, T, K), generator=g)
    else:
        sel = torch.randint(1, E, (B, T, K), generator=g)
        sel[torch.rand(B, T, K, generator=g) < skew] = 0
    w = torch.rand(B, T, K, generator=g) if weighted else None
    go_dt = x_dt if x_dt == torch.float16 else torch.bfloat16
    go = torch.randn(*((B, T, H) if weighted else (B, T, K, H)), generator=g).to(go_dt)
    return x, keys, sel, w, go


def _case_id(c):
    return "s{}-B{}T{}-D{}H{}-E{}K{}-{}{}-{}{}".format(
        c[0], c[1], c[2], c[3], c[4], c[5], c[6], "w" if c[7] else "u", "r" if c[8] else "t", c[9],
        "-hot" if c[10] else "")


def _check(case):
    x, keys, sel, w, go = _make(case)
    route_input, mode = case[8], case[9]
    _, amp_dt, tol = _MODES[mode]
    amp = amp_dt is not None
    print(f"sweep case {case}", flush=True)
    got = U.run_hip(x, keys, sel, w, go, route_input, amp, amp_dtype=amp_dt or torch.bfloat16)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, amp,
                       amp_dtype="float16" if amp_dt == torch.float16 else "bfloat16")
    U.compare(got, exp, tol)


@pytest.mark.parametrize("case", _cases(), ids=_case_id)
def test_random_case_matches_the_oracle(case):
    _check(case)


@pytest.mark.parametrize("case", [c for c in _cases() if c[9] != "fp32" and c[6] >= 2], ids=_case_id)
def test_random_case_with_dense_top_k_sums_matches_the_oracle(case):
    """The same cases (16-bit operands, top-k >= 2) with every top-k sum the
    dense GEMM over expert-slotted rows can take sent there, whatever the
    cost model would choose."""
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 2) == 0
    try:
        _check(case)
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)


@pytest.mark.parametrize("case", [c for c in _cases() if c[7] or not c[8]], ids=_case_id)
def test_random_case_with_atomic_top_k_sums_matches_the_oracle(case, monkeypatch):
    """The cases that sum over top-k (a weighted forward, or the input
    gradient of a token-input selection) with those sums taken by fp32
    atomics (CVMM_ATOMIC_REDUCE)."""
    import cvmm_codex_amd.api as C
    monkeypatch.setattr(C, "cvmm_atomic_reduce", True)
    _check(case)


@pytest.mark.parametrize("case", _cases(), ids=_case_id)
def test_random_case_with_the_backward_on_two_streams_matches_the_oracle(case, monkeypatch):
    """Every case with the weight gradient on a second stream beside the
    input gradient (CVMM_OVERLAP_BACKWARD)."""
    import cvmm_codex_amd.api as C
    monkeypatch.setattr(C, "cvmm_overlap_backward", True)
    _check(case)


@pytest.mark.parametrize("case", [c for c in _cases() if not c[7] and not c[8] and c[6] >= 4], ids=_case_id)
def test_random_case_with_low_memory_slices_matches_the_oracle(case, monkeypatch):
    """Token-input unweighted cases with top-k >= 4 with the input gradient's
    top-k sum taken over slices of two top-k columns at a time
    (CVMM_LOWMEM_CHUNK_SIZE=2)."""
    import cvmm_codex_amd.api as C
    monkeypatch.setattr(C, "cvmm_lowmem_chunk_size", 2)
    _check(case)


_BIT_KNOBS = (("RING_TILE", 1), ("RING_TILE", 2), ("RING_TILE", 3), ("GEMM_ORDER", 1), ("GEMM_ORDER", 2),
              ("WGRAD_TILE", 1), ("WGRAD_TILE", 5), ("WGRAD_ORDER", 1), ("WGRAD_ORDER", 3),
              ("PANEL_TILES_PER_WG", 1), ("PANEL_TILES_PER_WG", 3))


@pytest.mark.parametrize("case", [c for c in _cases() if c[9] != "fp32"], ids=_case_id)
def test_random_case_tile_and_order_knobs_keep_the_bits(case):
    """Tile shapes and workgroup orders of the routed GEMMs and the weight
    gradient only regroup the same products summed in the same order: every
    output that two runs of the built-in choice reproduce bit for bit is
    reproduced bit for bit under each setting."""
    from cvmm_codex_amd import _native as N
    x, keys, sel, w, go = _make(case)
    route_input, mode = case[8], case[9]
    amp_dt = _MODES[mode][1]
    print(f"sweep case {case}", flush=True)
    run = lambda: U.run_hip(x, keys, sel, w, go, route_input, True, amp_dtype=amp_dt)
    base, again = run(), run()
    stable = [n for n, t in base.items() if t is not None and torch.equal(t, again[n])]
    assert {"out", "keys_grad"} <= set(stable), stable
    lib = N.lib()
    for knob, value in _BIT_KNOBS:
        code = getattr(N, "TUNE_" + knob)
        assert lib.cvmm_tuning_set(code, value) == 0
        try:
            got = run()
        finally:
            lib.cvmm_tuning_set(code, 0)
        for n in stable:
            assert torch.equal(got[n], base[n]), (knob, value, n)


def _foreign_prepare(sd, wd, route_input=False):
    """A selector built by the caller with torch ops, the way the reference's
    pure-torch preparation builds it (cvmm.py:1786-1803): an unstable sort,
    no inverse permutation or offsets attached."""
    import cvmm_codex_amd.api as C
    fsel = sd.flatten().to(torch.int32)
    ssel, sel_index = fsel.sort()
    if route_input:
        return C.CVMMSel(fsel.view_as(sd), ssel.view_as(sd), sel_index, None, wd)
    return C.CVMMSel(fsel.view_as(sd), ssel.view_as(sd), sel_index // sd.shape[-1], sel_index, wd)


@pytest.mark.parametrize("case", _cases(), ids=_case_id)
def test_random_case_with_a_caller_built_selector_matches_the_oracle(case):
    x, keys, sel, w, go = _make(case)
    route_input, mode = case[8], case[9]
    _, amp_dt, tol = _MODES[mode]
    amp = amp_dt is not None
    print(f"sweep case {case}", flush=True)
    got = U.run_hip(x, keys, sel, w, go, route_input, amp, amp_dtype=amp_dt or torch.bfloat16,
                    prepare=_foreign_prepare)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, amp,
                       amp_dtype="float16" if amp_dt == torch.float16 else "bfloat16")
    U.compare(got, exp, tol)


def _large_cases(n=6, seed=99):
    """Larger draws (~29000-32768 routes, 256 <-> 1024 wide, 32 or 64
    experts): the forward (N = 1024) or the grad-input (N = 1024) has
    (routes / 256 + experts / 2) x 4 >= 512 tiles, where the built-in choice
    takes the eight-wave 256 x 256 long-K tiles."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        T, K = int(rng.integers(7200, 8193)), 4
        E = int(rng.choice((32, 64)))
        D, H = ((256, 1024), (1024, 256))[len(out) % 2]
        out.append((200 + len(out), 1, T, D, H, E, K, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
                    str(rng.choice(["bf16", "fp16"])), None))
    return out


@pytest.mark.parametrize("case", _large_cases(), ids=_case_id)
def test_large_random_case_matches_the_oracle(case):
    _check(case)
