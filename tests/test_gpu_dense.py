"""The dense form of the top-k sums (one GEMM over expert slots whose operand
tiles are gathered on the fly, cvmm_topk_gemm.hip): the weighted forward
combine (cvmm.py:1541-1545) and the token gradient of a token-input
selection (cvmm.py:1204-1223).

The built-in cost model takes it only at high fan-out (the full-size
SwitchHead tests run it); here the tuning knob forces it on small shapes so
that every layout is checked against the oracle at the north-star tolerance:
token and route input, weighted and not, fp16, fp32 activations under
autocast, tokens that pick one expert twice, out-of-range ids, selectors the
sort did not make (no inverse permutation), keys that are not the GEMM's row
layout (cast into the workspace), edge tiles (token, column, k and expert
counts that fill no whole tile or window) and a workspace holding garbage.
The sum over a token's routes runs in the GEMM's fp32 accumulators (one
rounding, where the routed path rounds each route's product first), which
the tolerance covers.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import cvmm_codex_amd.api as C
from cvmm_codex_amd import _native as N
from tests import gpu_util as U

pytestmark = pytest.mark.gpu


@pytest.fixture
def dense():
    lib = N.lib()
    assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 2) == 0
    yield lib
    lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)


def _case(seed, B, T, D, H, E, K, weighted, route_input, x_dt=torch.bfloat16, dup=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((B, T, K, D) if route_input else (B, T, D)), generator=g).to(x_dt)
    keys = torch.randn(E, D, H, generator=g) / D ** 0.5
    if dup:   # independent draws: some tokens pick an expert twice
        sel = torch.randint(0, E, (B, T, K), generator=g)
    else:
        sel = torch.rand(B, T, E, generator=g).topk(K, dim=-1).indices
    w = torch.rand(B, T, K, generator=g) if weighted else None
    go = torch.randn(*((B, T, H) if weighted else (B, T, K, H)), generator=g).to(torch.bfloat16)
    return x, keys, sel, w, go


@pytest.mark.parametrize("weighted,route_input,D,H,E,K", [
    (False, False, 64, 128, 16, 4),      # token gradient (unweighted token input)
    (False, False, 128, 64, 32, 8),
    (False, False, 64, 64, 64, 64),      # SwitchHead-like fan-out: 64 routes per token
    (True, True, 64, 128, 32, 16),       # weighted forward, route input (SwitchHead O / FFN down)
    (True, True, 128, 256, 16, 4),
    (True, False, 96, 64, 12, 3),        # weighted forward, token input
])
def test_dense_topk_matches_oracle(dense, weighted, route_input, D, H, E, K):
    x, keys, sel, w, go = _case(D + H + E + K, 2, 200, D, H, E, K, weighted, route_input)
    got = U.run_hip(x, keys, sel, w, go, route_input, True)
    U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True)])
def test_dense_and_routed_agree(weighted, route_input):
    """Both forms of the same sums, against each other (one rounding step
    apart) and against the oracle."""
    lib = N.lib()
    x, keys, sel, w, go = _case(5, 2, 256, 64, 128, 32, 8, weighted, route_input)
    out = {}
    try:
        for mode in (1, 2):
            assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, mode) == 0
            out[mode] = U.run_hip(x, keys, sel, w, go, route_input, True)
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    exp = U.run_oracle(x, keys, sel, w, go, route_input, True)
    for mode in (1, 2):
        U.compare(out[mode], exp, 2e-2)
    name = "out" if weighted else "x_grad"
    assert U.norm_rel(U.to_np(out[2][name]), U.to_np(out[1][name])) <= 1e-2


def test_dense_topk_is_deterministic(dense):
    x, keys, sel, w, go = _case(6, 2, 300, 64, 64, 16, 8, False, False)
    a = U.run_hip(x, keys, sel, w, go, False, True)
    b = U.run_hip(x, keys, sel, w, go, False, True)
    assert torch.equal(a["x_grad"], b["x_grad"]) and torch.equal(a["out"], b["out"])


def test_dense_topk_fp16(dense):
    for weighted, route_input in ((False, False), (True, True)):
        x, keys, sel, w, go = _case(7, 2, 128, 64, 96, 16, 4, weighted, route_input, x_dt=torch.float16)
        got = U.run_hip(x, keys, sel, w, go, route_input, True, amp_dtype=torch.float16)
        U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True, amp_dtype="float16"), 2e-2)


def test_dense_topk_fp32_activations_under_autocast(dense):
    """x stored in fp32: the slotted rows round it to the op dtype."""
    for weighted, route_input in ((False, False), (True, True)):
        x, keys, sel, w, go = _case(8, 1, 160, 64, 64, 16, 4, weighted, route_input, x_dt=torch.float32)
        got = U.run_hip(x, keys, sel, w, go, route_input, True)
        U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


def test_dense_topk_duplicate_experts(dense):
    """Tokens that pick one expert two or three times: the further routes run
    as extra passes over the experts (each route its own operand row)."""
    for weighted, route_input in ((False, False), (True, True), (True, False)):
        x, keys, sel, w, go = _case(9, 2, 128, 64, 64, 4, 6, weighted, route_input, dup=True)
        most = max(max(r.count(e) for e in set(r)) for r in sel.reshape(-1, 6).tolist())
        assert most >= 3
        got = U.run_hip(x, keys, sel, w, go, route_input, True)
        U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True)])
def test_dense_topk_heavy_repeats(dense, weighted, route_input):
    """Repeats up to the whole top-k: some tokens send all 64 routes to one
    expert, others 32 + 32 to two, others a mix, in a tile beside tokens with
    no repeats -- the tile runs up to 64 passes over the experts, each pass
    taking every token's next route on the expert from the next-route links."""
    T, K, E = 300, 64, 40
    x, keys, sel, w, go = _case(41, 1, T, 64, 72, E, K, weighted, route_input, dup=True)
    sel[0, 0, :] = 5                          # 64 routes on one expert
    sel[0, 1, :32] = 7
    sel[0, 1, 32:] = 9                        # 32 + 32
    g = torch.Generator().manual_seed(42)
    sel[0, 2:40] = torch.randint(0, 3, (38, K), generator=g)   # many repeats over three experts
    sel[0, 280, ::2] = 11                     # every other route, in the tile's second half
    got = U.run_hip(x, keys, sel, w, go, route_input, True)
    U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


def test_dense_topk_invalid_ids_contribute_nothing(dense):
    E = 8
    for weighted, route_input in ((False, False), (True, True)):
        x, keys, sel, w, go = _case(10, 2, 128, 64, 64, E, 4, weighted, route_input)
        g = torch.Generator().manual_seed(11)
        bad = torch.rand(sel.shape, generator=g) < 0.1
        sel_bad = sel.clone()
        sel_bad[bad] = torch.where(torch.rand(sel.shape, generator=g) < 0.5, -1, E + 2)[bad]
        got = U.run_hip(x, keys, sel_bad, w, go, route_input, True)
        sel_ok = sel.clone()
        sel_ok[bad] = 0
        if weighted:   # a zero routing weight: the route adds exact zeros
            w_ok = w.clone()
            w_ok[bad] = 0
            exp = U.run_oracle(x, keys, sel_ok, w_ok, go, route_input, True)
            assert U.norm_rel(U.to_np(got["out"]), exp["out"]) <= 2e-2
        else:          # a zero gradient row: the route adds exact zeros
            go_ok = go.clone()
            go_ok[bad] = 0
            exp = U.run_oracle(x, keys, sel_ok, None, go_ok, route_input, True)
            assert U.norm_rel(U.to_np(got["x_grad"]), exp["x_grad"]) <= 2e-2


def test_dense_topk_with_a_foreign_selector(dense):
    """A CVMMSel built from torch.sort (no inverse permutation attached): the
    call inverts the route index itself."""
    x, keys, sel, _, go = _case(12, 2, 200, 64, 128, 16, 4, False, False)
    sd = sel.cuda()
    fsel = sd.flatten().to(torch.int32)
    ssel, perm = fsel.sort(stable=True)
    s = C.CVMMSel(fsel.view_as(sd), ssel.view_as(sd), perm // 4, perm)
    xd = x.cuda().requires_grad_(True)
    kd = keys.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(xd, s, kd)
    y.backward(go.cuda().to(y.dtype))
    got = {"out": y.detach(), "x_grad": xd.grad, "keys_grad": kd.grad, "weights_grad": None}
    U.compare(got, U.run_oracle(x, keys, sel, None, go, False, True), 2e-2)


def test_dense_topk_keys_cast_into_the_workspace(dense):
    """Keys that are not the GEMM's op-dtype row layout (the fp32 keys
    themselves) are cast into the workspace by the call."""
    x, keys, sel, _, go = _case(13, 2, 160, 64, 64, 16, 4, False, False)
    s = C.cvmm_prepare_sel2(sel.cuda())
    C.create_kernels()
    s._resolve(16)
    xd, kd, gd = x.cuda(), keys.cuda(), go.cuda()

    class Ctx:
        op_type = torch.bfloat16

    gx, _, _ = C._backward(Ctx, gd, xd, kd, s.raw_sel, s.sel, s.sel_index, s.out_index, None, True, False, False,
                           keys_x=None)
    exp = U.run_oracle(x, keys, sel, None, go, False, True)
    assert U.norm_rel(U.to_np(gx), exp["x_grad"]) <= 2e-2
    # and the weighted forward with the fp32 keys
    x2, keys2, sel2, w2, go2 = _case(14, 2, 160, 64, 64, 16, 4, True, True)
    s2 = C.cvmm_prepare_sel2(sel2.cuda(), w2.cuda(), route_input=True)
    s2._resolve(16)
    y = C._forward(x2.cuda(), s2.sel_index, s2.sel, keys2.cuda(), s2.out_index, w2.cuda(), torch.bfloat16)
    exp2 = U.run_oracle(x2, keys2, sel2, w2, go2, True, True)
    assert U.norm_rel(U.to_np(y), exp2["out"]) <= 2e-2


def test_dense_topk_reads_either_weight_row_layout(dense):
    """The dense GEMM's B as given: the expert-interleaved copy ([N][E*K]
    rows, both operands k-contiguous; what cvmm() casts for a dense sum) or
    the routed-layout copy of the other orientation ([E*K][N] rows), for the
    token gradient and for the weighted forward, each against the oracle."""
    class Ctx:
        op_type = torch.bfloat16

    x, keys, sel, _, go = _case(15, 2, 160, 64, 128, 16, 4, False, False)
    s = C.cvmm_prepare_sel2(sel.cuda())
    C.create_kernels()
    s._resolve(16)
    xd, kd, gd = x.cuda(), keys.cuda(), go.cuda()
    exp = U.run_oracle(x, keys, sel, None, go, False, True)
    kt, _ = C._cast_keys(kd, torch.bfloat16, C._CopyPlan(True, False, 0, True, False))
    _, kn_i = C._cast_keys(kd, torch.bfloat16, C._CopyPlan(False, True, N.CAST_N_INTERLEAVED, True, False))
    assert kn_i.shape == (64, 16, 128)
    for keys_x, is_t in ((kt, True), (kn_i.permute(1, 0, 2), False)):
        gx, _, _ = C._backward(Ctx, gd, xd, kd, s.raw_sel, s.sel, s.sel_index, s.out_index, None, True, False,
                               False, keys_x=keys_x, keys_x_is_t=is_t)
        assert U.norm_rel(U.to_np(gx), exp["x_grad"]) <= 2e-2, is_t

    x2, keys2, sel2, w2, go2 = _case(16, 2, 160, 64, 128, 16, 4, True, True)
    s2 = C.cvmm_prepare_sel2(sel2.cuda(), w2.cuda(), route_input=True)
    s2._resolve(16)
    k2 = keys2.cuda()
    exp2 = U.run_oracle(x2, keys2, sel2, w2, go2, True, True)
    kt_i, kn = C._cast_keys(k2, torch.bfloat16, C._CopyPlan(True, True, N.CAST_T_INTERLEAVED, True, False))
    assert kt_i.shape == (128, 16, 64) and kn.shape == (16, 64, 128)
    for keys_op in (kn, kt_i.permute(1, 2, 0)):
        y = C._forward(x2.cuda(), s2.sel_index, s2.sel, k2, s2.out_index, w2.cuda(), torch.bfloat16, keys_op, False)
        assert U.norm_rel(U.to_np(y), exp2["out"]) <= 2e-2


def test_dense_workspace_contents_do_not_matter(dense):
    """Through the C ABI: the call builds everything it reads from the
    workspace (slot table, copies), so workspaces filled with different
    garbage give the same bits, and those match the oracle."""
    x, keys, sel, _, go = _case(15, 2, 160, 64, 96, 16, 4, False, False)
    E, D, H = keys.shape
    s = C.cvmm_prepare_sel2(sel.cuda())
    C.create_kernels()
    s._resolve(E)
    lib = N.lib()
    st = N.stream_of(torch.device("cuda"))
    kt = keys.cuda().transpose(1, 2).contiguous().to(torch.bfloat16)    # [E, d_out, d_in]
    kv = kt.transpose(1, 2)                                              # logical [E, d_in, d_out]
    g = go.cuda().reshape(-1, H).contiguous()
    R, T = sel.numel(), sel.numel() // 4
    offs = C._offsets_for(s.sel, E)
    rpos = s.out_index._cvmm_route_pos
    ws_b = lib.cvmm_bwd_x_workspace_bytes(R, E, D, H, T, 1, 0, 1, 4, N.BF16, N.BF16, 0, 0)

    def call(fill):
        ws = torch.full((ws_b,), fill, dtype=torch.uint8, device="cuda")
        gx = torch.empty(T, D, dtype=torch.bfloat16, device="cuda")
        N.check(lib.cvmm_bwd_x(N.ptr(g), N.BF16, g.shape[0], g.stride(0), N.ptr(kv), N.BF16, E, D, H,
                               *kv.stride(), N.ptr(s.sel), N.ptr(s.sel_index), N.ptr(s.out_index), R, N.ptr(offs),
                               N.ptr(rpos), None, 0, 4, None, 0, 0, 0, N.BF16, N.ptr(gx), N.BF16, T, D, None, 0,
                               0, N.ptr(ws), ws_b, st), "cvmm_bwd_x")
        torch.cuda.synchronize()
        return gx

    a, b, c = call(0x5A), call(0xFF), call(0)
    assert torch.equal(a, b) and torch.equal(b, c)
    exp = U.run_oracle(x, keys, sel, None, go, False, True)
    assert U.norm_rel(U.to_np(a), exp["x_grad"].reshape(T, D)) <= 2e-2


@pytest.mark.parametrize("weighted,route_input,T,D,H,E,K", [
    (False, False, 300, 72, 200, 20, 5),    # 300 tokens: a part-filled token tile; N = 72, K = 200 (4 k slices)
    (True, True, 259, 136, 104, 20, 6),     # K = 136: a part-filled k slice; E = 20: a part-filled window
    (True, False, 97, 64, 520, 33, 7),      # N = 520: three column tiles, the last part-filled
])
def test_dense_topk_edge_tiles(dense, weighted, route_input, T, D, H, E, K):
    x, keys, sel, w, go = _case(T + D + H, 1, T, D, H, E, K, weighted, route_input)
    got = U.run_hip(x, keys, sel, w, go, route_input, True)
    U.compare(got, U.run_oracle(x, keys, sel, w, go, route_input, True), 2e-2)


def test_dense_topk_rows_not_16_byte_aligned(dense):
    """x rows one element into rows of D + 1: the operand rows cannot move 16
    bytes at a time, so the call copies them into the workspace first."""
    g = torch.Generator().manual_seed(23)
    T, K, D, H, E = 150, 4, 64, 64, 16
    big = torch.randn(T, K, D + 1, generator=g).to(torch.bfloat16)
    keys = torch.randn(E, D, H, generator=g) / D ** 0.5
    sel = torch.rand(1, T, E, generator=g).topk(K, dim=-1).indices
    w = torch.rand(1, T, K, generator=g)
    go = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    xd = big.to(dev)[..., 1:].reshape(1, T, K, D)
    assert xd.stride(-2) == D + 1
    s = C.cvmm_prepare_sel2(sel.to(dev), w.to(dev), route_input=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(xd, s, keys.to(dev))
    torch.cuda.synchronize()
    exp = U.run_oracle(big[..., 1:].reshape(1, T, K, D).contiguous(), keys, sel, w, go, True, True, need_w=False)
    assert U.norm_rel(U.to_np(y), exp["out"]) <= 2e-2


@pytest.mark.parametrize("mode,D,kept", [
    (2, 64, True),      # dense top-k sum: its operand rows
    (1, 64, True),      # route buffer, small-K product: its activation fragments
    (1, 256, False),    # route buffer, long-K product: nothing kept
])
def test_kept_scaled_rows_give_the_weight_gradient_bits(mode, D, kept):
    """cvmm_fwd_keep_scaled: a weighted forward over route input keeps the
    rows x'_r = rnd(rnd(w_r) * x_r) where it makes them (equal bit for bit to
    the same product in torch), its output is cvmm_fwd's, and cvmm_bwd_w given
    those rows with CVMM_FLAG_ROWS_SCALED writes the bits of its own scaling
    pass.  Where the product makes no such rows nothing is written."""
    import ctypes
    lib = N.lib()
    B, T, H, E, K = 2, 96, 128, 32, 16
    x, keys, sel, w, go = _case(41 + D, B, T, D, H, E, K, True, True)
    x, keys, w, go = x.cuda(), keys.cuda(), w.cuda(), go.cuda()
    s = C.cvmm_prepare_sel2(sel.cuda(), w, route_input=True)
    s._resolve(E)
    R, Tn = B * T * K, B * T
    offs = C._offsets_for(s.sel, E)
    rp = s.out_index if s.out_index is not None else s.sel_index
    rpos = C._route_pos(rp, R)
    assert s.out_index is None and rpos is not None
    xr = x.reshape(R, D).contiguous()
    wf = w.reshape(-1).contiguous()
    # the long-K product reads a [E][d_out][d_in] copy: keys as the op-dtype
    # per-expert layout the fast kernels take (k contiguous)
    kt = keys.to(torch.bfloat16).transpose(1, 2).contiguous()
    st = N.stream_of(x.device)
    bf = N.BF16

    def fwd(keep):
        out = torch.empty(Tn, H, dtype=torch.bfloat16, device="cuda")
        ws_b = lib.cvmm_fwd_workspace_bytes(R, E, D, H, Tn, bf, bf, 1, 1, 0)
        ws = torch.full((max(ws_b, 1),), 0x5A, dtype=torch.uint8, device="cuda")
        args = [N.ptr(xr), bf, R, D, N.ptr(kt), bf, E, D, H, kt.stride(0), 1, kt.stride(1),
                N.ptr(s.sel), N.ptr(s.sel_index), None, R, N.ptr(offs), N.ptr(rpos), N.ptr(wf), N.F32, K, bf,
                N.ptr(out), bf, Tn, H]
        if not keep:
            N.check(lib.cvmm_fwd(*args, 0, N.ptr(ws), ws_b, st), "cvmm_fwd")
            return out, None, None
        xs = torch.full((R, D), 7.0, dtype=torch.bfloat16, device="cuda")
        written = ctypes.c_int32(-1)
        N.check(lib.cvmm_fwd_keep_scaled(*args, N.ptr(xs), ctypes.addressof(written), 0, N.ptr(ws), ws_b, st),
                "cvmm_fwd_keep_scaled")
        return out, xs, written.value

    def bwd_w(xin, flags, room):
        dw = torch.empty(E, D, H, dtype=torch.float32, device="cuda")
        ws_b = lib.cvmm_bwd_w_workspace_bytes_ex(R, E, D, H, bf, 1, 1 if room else 0)
        ws = torch.zeros(ws_b, dtype=torch.uint8, device="cuda")
        N.check(lib.cvmm_bwd_w(N.ptr(xin), bf, R, D, N.ptr(go), bf, Tn, H, E, D, H, N.ptr(s.sel),
                               N.ptr(s.sel_index), None, R, N.ptr(offs), N.ptr(wf), N.F32, K, bf, N.ptr(dw), N.F32,
                               dw.stride(0), dw.stride(1), dw.stride(2), flags, N.ptr(ws), ws_b, st), "cvmm_bwd_w")
        return dw

    assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, mode) == 0
    try:
        out_plain, _, _ = fwd(False)
        out_keep, xs, written = fwd(True)
        torch.cuda.synchronize()
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    assert torch.equal(out_keep, out_plain)
    if not kept:
        assert written == 0 and bool((xs == 7.0).all())
        return
    assert written == 1
    ref = (wf.to(torch.bfloat16).float()[:, None] * xr.float()).to(torch.bfloat16)
    assert torch.equal(xs, ref)
    dw_scaled_here = bwd_w(xr, 0, True)
    dw_kept = bwd_w(xs, N.FLAG_ROWS_SCALED, False)
    torch.cuda.synchronize()
    assert torch.equal(dw_kept, dw_scaled_here)
