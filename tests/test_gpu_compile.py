"""torch.compile through the API (the reference registers its forward as a
torch.library op with a fake implementation for this, cvmm.py:808-812,
:1436-1456): compiled steps (aot_eager and inductor) match the CPU oracle at
the north-star tolerance (2e-2 under bf16 autocast, 1e-4 in fp32), compiled
and eager steps run the same kernels and agree bit for bit under aot_eager,
and the ops pass torch.library.opcheck."""
from __future__ import annotations

import pytest
import torch

import cvmm_codex_amd as C
from cvmm_codex_amd import compile_ops as ops
from tests import gpu_util as U

pytestmark = pytest.mark.gpu


def _case(seed, weighted, route_input, B=2, T=96, D=128, H=64, E=12, K=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*((B, T, K, D) if route_input else (B, T, D)), generator=g).to(torch.bfloat16).cuda()
    keys = (torch.randn(E, D, H, generator=g) / D ** 0.5).cuda()
    sel = torch.randint(0, E, (B, T, K), generator=g).cuda()
    w = torch.rand(B, T, K, generator=g).cuda() if weighted else None
    go = torch.randn(*((B, T, H) if weighted else (B, T, K, H)), generator=g).to(torch.bfloat16).cuda()
    return x, keys, sel, w, go


def _step(x, keys, sel, w, route_input):
    s = C.cvmm_prepare_sel2(sel, w, route_input=route_input)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        return C.cvmm(x, s, keys)


def _run(fn, x, keys, sel, w, go, route_input):
    xs = x.clone().requires_grad_(True)
    ks = keys.clone().requires_grad_(True)
    ws = None if w is None else w.clone().requires_grad_(True)
    y = fn(xs, ks, sel, ws, route_input)
    y.backward(go.to(y.dtype))
    torch.cuda.synchronize()
    return y.detach(), xs.grad, ks.grad, None if ws is None else ws.grad


def _oracle(case, route_input, amp=True):
    x, keys, sel, w, go = (None if t is None else t.cpu() for t in case)
    return U.run_oracle(x, keys, sel, w, go, route_input, amp)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True), (True, False)])
def test_compiled_step_matches_eager_and_oracle(weighted, route_input):
    """One graph (fullgraph=True): selector, forward and backward all traced."""
    torch._dynamo.reset()
    case = _case(3, weighted, route_input)
    eager = _run(_step, *case, route_input)
    compiled = _run(torch.compile(_step, backend="aot_eager", fullgraph=True), *case, route_input)
    names = ("out", "x_grad", "keys_grad", "weights_grad")
    for name, a, b in zip(names, eager, compiled):
        if a is None:
            assert b is None, name
        else:
            assert torch.equal(a, b), name
    U.compare(dict(zip(names, compiled)), _oracle(case, route_input), 2e-2)


@pytest.mark.parametrize("weighted,route_input", [(False, False), (True, True)])
def test_inductor_step_matches_oracle(weighted, route_input):
    """The same step compiled by inductor (the default backend): the custom
    ops and their fakes hold up under its graph passes."""
    torch._dynamo.reset()
    case = _case(6, weighted, route_input)
    compiled = _run(torch.compile(_step, fullgraph=True), *case, route_input)
    names = ("out", "x_grad", "keys_grad", "weights_grad")
    U.compare(dict(zip(names, compiled)), _oracle(case, route_input), 2e-2)


def _step_fp32(x, keys, sel, w, route_input):
    s = C.cvmm_prepare_sel2(sel, w, route_input=route_input)
    return C.cvmm(x, s, keys)


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_fp32_step_matches_oracle(backend):
    """fp32 mode (no autocast): 1e-4 against the oracle."""
    torch._dynamo.reset()
    x, keys, sel, w, go = _case(7, True, False)
    x = x.float()
    compiled = _run(torch.compile(_step_fp32, backend=backend, fullgraph=True), x, keys, sel, w, go, False)
    names = ("out", "x_grad", "keys_grad", "weights_grad")
    U.compare(dict(zip(names, compiled)), _oracle((x, keys, sel, w, go), False, amp=False), 1e-4)


def test_compiled_step_with_transposed_x_matches_oracle():
    """x as a permuted (dense, non-contiguous) view: the fake's grad_x layout
    must be the real op's (a contiguous tensor of x's shape)."""
    torch._dynamo.reset()
    x, keys, sel, w, go = _case(8, False, False)
    xt = x.transpose(0, 1).contiguous().transpose(0, 1)          # [B, T, D] with T-major storage
    assert not xt.is_contiguous()

    def run(fn):
        xs = xt.clone(memory_format=torch.preserve_format).requires_grad_(True)
        ks = keys.clone().requires_grad_(True)
        y = fn(xs, ks, sel, None, False)
        y.backward(go.to(y.dtype))
        torch.cuda.synchronize()
        return {"out": y.detach(), "x_grad": xs.grad, "keys_grad": ks.grad, "weights_grad": None}

    exp = _oracle((x, keys, sel, None, go), False)
    for backend in ("aot_eager", "inductor"):
        torch._dynamo.reset()
        got = run(torch.compile(_step, backend=backend, fullgraph=True))
        U.compare(got, exp, 2e-2)


def test_ops_pass_opcheck():
    x, keys, sel, w, go = _case(4, True, False)
    raw = sel.reshape(-1)
    E = keys.shape[0]
    utils = ("test_schema", "test_faketensor")
    torch.library.opcheck(ops.sort_routes, (raw, E, 3), test_utils=utils)
    ssel, perm, tok, off, _ = ops.sort_routes(raw, E, 3)
    torch.library.opcheck(ops.expert_offsets, (ssel, E), test_utils=utils)
    torch.library.opcheck(ops.cast_keys, (keys, torch.bfloat16), test_utils=utils)
    xf = x.reshape(-1, x.shape[-1])
    torch.library.opcheck(ops.forward, (xf, keys, None, True, ssel, tok, perm, off, w, torch.bfloat16, 0),
                          test_utils=utils)
    gy = go.reshape(-1, go.shape[-1])
    torch.library.opcheck(ops.backward, (gy, xf, keys, None, False, ssel, tok, perm, off, w, 3, torch.bfloat16,
                                         True, True, True, 0), test_utils=utils)
    minus1 = torch.full((1,), -1, dtype=torch.int64, device="cuda")
    torch.library.opcheck(ops.cvmm_triton, (xf, tok, ssel, keys, torch.bfloat16, perm, torch.bfloat16),
                          test_utils=utils)
    torch.library.opcheck(ops.cvmm_triton, (xf, tok, ssel, keys, torch.bfloat16, minus1, torch.bfloat16),
                          test_utils=utils)


def test_reference_op_schema_matches_the_api_forward():
    """cvmm_triton (the reference op's schema) gives the per-route forward of
    cvmm(), and the oracle's."""
    x, keys, sel, _, _ = _case(5, False, False)
    s = C.cvmm_prepare_sel2(sel)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = C.cvmm(x, s, keys)
    z = C.cvmm_triton_call(x.reshape(-1, x.shape[-1]), s.sel_index, s.sel, keys.to(torch.bfloat16),
                           torch.bfloat16, s.out_index, torch.bfloat16)
    assert z.shape == y.shape
    assert torch.equal(z, y)
    exp = _oracle((x, keys, sel, None, torch.zeros(*sel.shape, keys.shape[2])), False)
    assert U.norm_rel(U.to_np(z), exp["out"]) <= 2e-2


def test_reference_op_rounds_once_to_out_dtype():
    """out_dtype float32 with a bf16 op: products of bf16 operands, stored in
    float32 directly (cvmm.py:832-833, :862-863), i.e. not rounded to bf16 on
    the way; route-input form (out_index = the -1 sentinel)."""
    from oracle import cvmm_oracle as O
    x, keys, sel, _, _ = _case(9, False, True)
    s = C.cvmm_prepare_sel2(sel, route_input=True)
    minus1 = torch.full((1,), -1, dtype=torch.int64, device="cuda")
    z = C.cvmm_triton_call(x.reshape(-1, x.shape[-1]), s.sel_index, s.sel, keys, torch.float32, minus1,
                           torch.bfloat16)
    assert z.dtype == torch.float32
    meta = O.prepare_sel2(sel.cpu().numpy(), route_input=True)
    xn, kn = U.to_np(x), U.to_np(keys)
    once = O.forward(xn, meta, kn, "bfloat16", "float32")
    twice = O.forward(xn, meta, kn, "bfloat16", "bfloat16")
    zn = U.to_np(z)
    assert U.norm_rel(zn, once) <= 1e-5
    assert U.norm_rel(zn, twice) > 1e-4          # would be ~bf16 epsilon off with the extra rounding


def _router_ffn(x, gate, w_up, w_down, k=4):
    """benchmark_ffn_moe.py:89-98 with the fused router."""
    B, T, D = x.shape
    H = w_up.shape[2]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        logits = x @ gate
        weights, _, sel_up = C.cvmm_route_topk(logits, k, True)
        hidden = torch.nn.functional.gelu(C.cvmm(x, sel_up, w_up))
        sel_down = C.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        return C.cvmm(hidden.view(B, T, k, H), sel_down, w_down)


def test_compiled_router_stack_matches_eager():
    """The FFN stack with the fused router, one graph: router op (with its
    registered backward), both projections and the gate gradient."""
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(8)
    x0 = torch.randn(2, 64, 128, generator=g).to(torch.bfloat16).cuda()
    gate0 = (torch.randn(128, 16, generator=g) / 12).cuda()
    up0 = (torch.randn(16, 128, 64, generator=g) / 12).cuda()
    down0 = (torch.randn(16, 64, 128, generator=g) / 8).cuda()
    gy = torch.randn(2, 64, 128, generator=g).cuda()

    def run(fn):
        ts = [t.clone().requires_grad_(True) for t in (x0, gate0, up0, down0)]
        y = fn(*ts)
        y.backward(gy.to(y.dtype))
        torch.cuda.synchronize()
        return [y.detach()] + [t.grad for t in ts]

    eager = run(_router_ffn)
    compiled = run(torch.compile(_router_ffn, backend="aot_eager", fullgraph=True))
    for name, a, b in zip(("out", "x", "gate", "up", "down"), eager, compiled):
        assert torch.equal(a, b), name


def test_router_ops_pass_opcheck():
    g = torch.Generator().manual_seed(9)
    logits = (torch.randn(40, 24, generator=g)).to(torch.bfloat16).cuda()
    utils = ("test_schema", "test_faketensor")
    torch.library.opcheck(ops.route_topk, (logits, 5, True), test_utils=utils)
    w, sel, *_ = ops.route_topk(logits, 5, True)
    gw = torch.randn(40, 5, generator=g).cuda()
    torch.library.opcheck(ops.route_topk_backward, (logits, sel, gw, 5, True), test_utils=utils)
