"""Seeded synthetic inputs for the BASELINE.json CVMM configs (CPU generator,
so every run and every machine draws the same tensors).

C1 tiny fp32, C2 ff_up_1024, C3 ff_down_1024_weighted, C4 SwitchHead V/O,
C5 full MoE FFN stack with Zipf-skewed routing.  Each projection is returned
as a ``Projection``: x, keys, sel, optional reduction weight, grad_out, whether
x is route-major, and whether autocast bf16 is on.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F


@dataclass
class Projection:
    name: str
    x: torch.Tensor
    keys: torch.Tensor
    sel: torch.Tensor
    weights: Optional[torch.Tensor]
    grad_out: torch.Tensor
    route_input: bool
    amp: bool

    @property
    def routes(self) -> int:
        return self.sel.numel()

    @property
    def flops(self) -> float:
        """6 * R * d_in * d_out: forward, grad-input and grad-weight GEMMs."""
        return 6.0 * self.routes * self.keys.shape[1] * self.keys.shape[2]

    def to(self, device) -> "Projection":
        mv = lambda t: None if t is None else t.to(device)
        return Projection(self.name, mv(self.x), mv(self.keys), mv(self.sel), mv(self.weights),
                          mv(self.grad_out), self.route_input, self.amp)


def _g(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def c1_tiny() -> Projection:
    g = _g(0)
    x = torch.randn(4, 128, 256, generator=g)
    keys = torch.randn(16, 256, 64, generator=g) / 16
    sel = torch.randint(0, 16, (4, 128, 4), generator=g)
    gy = torch.randn(4, 128, 4, 64, generator=g)
    return Projection("tiny_fp32", x, keys, sel, None, gy, False, False)


def _c2_routing(g):
    x = torch.randn(16, 512, 1024, generator=g).to(torch.bfloat16)
    keys = torch.randn(64, 1024, 128, generator=g) / 32
    router = torch.randn(1024, 64, generator=g) / 32
    p = torch.softmax(x.float() @ router, dim=-1)
    gate, sel = p.topk(8, dim=-1)
    return x, keys, gate, sel


def c2_ff_up() -> Projection:
    g = _g(1)
    x, keys, _, sel = _c2_routing(g)
    gy = torch.randn(16, 512, 8, 128, generator=g).to(torch.bfloat16)
    return Projection("ff_up_1024", x, keys, sel, None, gy, False, True)


def c3_ff_down() -> Projection:
    _, _, gate, sel = _c2_routing(_g(1))
    g = _g(2)
    x = F.gelu(torch.randn(16, 512, 8, 128, generator=g)).to(torch.bfloat16)
    keys = torch.randn(64, 128, 1024, generator=g) / math.sqrt(128)
    gy = torch.randn(16, 512, 1024, generator=g).to(torch.bfloat16)
    return Projection("ff_down_1024_weighted", x, keys, sel, gate.contiguous(), gy, True, True)


def _c4_routing(g):
    lg = torch.randn(8, 1024, 32, 8, generator=g)
    pv, iv = torch.softmax(lg, dim=-1).topk(2, dim=-1)
    head = torch.arange(32).view(1, 1, 32, 1)
    sel = (iv + 8 * head).reshape(8, 1024, 64)
    return pv.reshape(8, 1024, 64).contiguous(), sel


def c4_switch_v() -> Projection:
    g = _g(3)
    _, sel = _c4_routing(g)
    x = torch.randn(8, 1024, 2048, generator=g).to(torch.bfloat16)
    keys = torch.randn(256, 2048, 64, generator=g) / math.sqrt(2048)
    gy = torch.randn(8, 1024, 64, 64, generator=g).to(torch.bfloat16)
    return Projection("switch_v_2048", x, keys, sel, None, gy, False, True)


def c4_switch_o() -> Projection:
    g = _g(3)
    pv, sel = _c4_routing(g)
    g2 = _g(30)
    x = torch.randn(8, 1024, 64, 64, generator=g2).to(torch.bfloat16)
    keys = torch.randn(256, 64, 2048, generator=g2) / 8
    gy = torch.randn(8, 1024, 2048, generator=g2).to(torch.bfloat16)
    return Projection("switch_o_2048_weighted", x, keys, sel, pv, gy, True, True)


def zipf_bias(n: int = 128, s: float = 1.1) -> torch.Tensor:
    ranks = torch.arange(1, n + 1, dtype=torch.float64)
    pmf = ranks ** (-s)
    pmf = pmf / pmf.sum()
    return pmf.log().float()


@dataclass
class FFNStack:
    x: torch.Tensor
    gate: torch.Tensor
    bias: torch.Tensor
    w_up: torch.Tensor
    w_down: torch.Tensor
    grad_out: torch.Tensor
    k: int

    def to(self, device) -> "FFNStack":
        return FFNStack(*(t.to(device) for t in (self.x, self.gate, self.bias, self.w_up, self.w_down,
                                                   self.grad_out)), self.k)

    @property
    def flops(self) -> float:
        T = self.x.shape[0] * self.x.shape[1]
        D = self.x.shape[2]
        E, _, H = self.w_up.shape
        return 6.0 * T * self.k * (D * H + H * D) + 6.0 * T * D * E


def c5_ffn_stack() -> FFNStack:
    g = _g(4)
    x = torch.randn(8, 2048, 2048, generator=g).to(torch.bfloat16)
    gate = torch.randn(2048, 128, generator=g) / math.sqrt(2048)
    w_up = torch.randn(128, 2048, 512, generator=g) / math.sqrt(2048)
    w_down = torch.randn(128, 512, 2048, generator=g) / math.sqrt(512)
    gy = torch.randn(8, 2048, 2048, generator=g).to(torch.bfloat16)
    return FFNStack(x, gate, zipf_bias(128, 1.1), w_up, w_down, gy, 8)


def ffn_forward(s: FFNStack, cvmm_mod, x, gate, w_up, w_down):
    """benchmark_ffn_moe.py:89-98 with the Zipf bias added to the gate logits."""
    B, T, D = x.shape
    E, _, H = w_up.shape
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = x @ gate + s.bias
        probs = torch.softmax(logits.float(), dim=-1)
        weights, sel = probs.topk(s.k, dim=-1)
        weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-20)
        sel_up = cvmm_mod.cvmm_prepare_sel2(sel)
        hidden = F.gelu(cvmm_mod.cvmm(x, sel_up, w_up))
        sel_down = cvmm_mod.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        return cvmm_mod.cvmm(hidden.view(B, T, s.k, H), sel_down, w_down)


def ffn_forward_fused(s: FFNStack, cvmm_mod, x, gate, w_up, w_down):
    """ffn_forward with the library's router projection (cvmm_gate_logits),
    fused router (cvmm_route_topk) and up projection + GELU (cvmm_gelu) in
    place of the torch lines."""
    B, T, D = x.shape
    E, _, H = w_up.shape
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = cvmm_mod.cvmm_gate_logits(x, gate) + s.bias
        weights, _, sel_up = cvmm_mod.cvmm_route_topk(logits, s.k, True)
        hidden = cvmm_mod.cvmm_gelu(x, sel_up, w_up)
        sel_down = cvmm_mod.cvmm_prepare_sel2(sel_up, weights, route_input=True)
        return cvmm_mod.cvmm(hidden.view(B, T, s.k, H), sel_down, w_down)


PROJECTIONS = {
    "tiny_fp32": c1_tiny,
    "ff_up_1024": c2_ff_up,
    "ff_down_1024_weighted": c3_ff_down,
    "switch_v_2048": c4_switch_v,
    "switch_o_2048_weighted": c4_switch_o,
}
