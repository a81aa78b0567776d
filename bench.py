"""CVMM forward+backward benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload ff_up_1024]

A step = one pass of the CVMM hot path over one batch of synthetic input:
selector preparation (stable counting sort), forward, and backward (grad x,
grad keys, grad reduction weight), launched by the drop-in API exactly as a
training step would.  ``value`` is whole-job TFLOP/s = 6*R*d_in*d_out / step
time (inputs resident in HBM).  Every kernel is also timed on its own: the
library brackets each launch with HIP events on the stream it runs on, and the
GEMM class with the most device time per step gives ``roofline`` (its
algorithmic flops or bytes per launch / its average launch time, against the
config's bound: MFMA for the wide projections, HBM for the narrow SwitchHead
ones, with both fractions reported); ``step_roofline`` does the same for the
whole step.  ``cpu_baseline`` times the reference's PyTorch CPU path (sort +
per-expert gather/matmul) on the host cores.  ``--ffn`` measures the full MoE
FFN stack the same way.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import workloads as W  # noqa: E402

METRIC = "CVMM fwd+bwd ms/iter and TFLOP/s (% of MI355X roofline), 1 GPU"
PEAK = {"bf16": 2500.0, "fp16": 2500.0, "fp32": 157.3}     # dense MFMA TFLOP/s
HBM_PEAK_GBS = 8000.0
DEFAULT_WORKLOAD = "ff_up_1024"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Runner:
    """Holds one projection's device tensors and runs steps through the API."""

    def __init__(self, proj: W.Projection, device):
        import cvmm_codex_amd.api as C
        self.C = C
        self.p = proj.to(device)
        self.x = self.p.x.detach().requires_grad_(True)
        self.keys = self.p.keys.detach().requires_grad_(True)
        self.w = None if self.p.weights is None else self.p.weights.detach().requires_grad_(True)
        self.E = self.keys.shape[0]
        self.n_steps = 0    # steps run by this process (profile summaries divide trace counts by it)

    def prepare(self):
        # the public call pattern (benchmark_ffn_moe.py:95-98): the selection
        # is sorted inside cvmm(), which knows the expert count, in the same
        # launches as the step's weight cast
        return self.C.cvmm_prepare_sel2(self.p.sel, self.w, route_input=self.p.route_input)

    def forward(self, s):
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=self.p.amp):
            return self.C.cvmm(self.x, s, self.keys)

    def backward(self, y):
        y.backward(self.p.grad_out.to(y.dtype))

    def zero(self):
        self.x.grad = None
        self.keys.grad = None
        if self.w is not None:
            self.w.grad = None

    def step(self):
        self.zero()
        s = self.prepare()
        y = self.forward(s)
        self.backward(y)
        self.n_steps += 1


def time_steps(runner: Runner, steps: int, warmup: int):
    for _ in range(warmup):
        runner.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        runner.step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def grads_of(runner: Runner):
    out = [runner.x.grad, runner.keys.grad]
    if runner.w is not None:
        out.append(runner.w.grad)
    return [g.detach().clone() for g in out]


def time_steps_graph(runner: Runner, steps: int, warmup: int):
    """Steps as replays of one HIP graph captured from a step (selector,
    forward, backward: every launch of the step, re-run on each replay), for
    steps whose host submission takes longer than their kernels.  Returns
    the ms per replay and whether a replay's gradients equal an eager
    step's bit for bit."""
    runner.step()
    torch.cuda.synchronize()
    eager = grads_of(runner)
    # warm-up on the capture's side stream, then capture with the gradients
    # unset, so the backward allocates them from the graph's pool
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            runner.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    runner.zero()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s = runner.prepare()
        y = runner.forward(s)
        runner.backward(y)
    for _ in range(max(warmup, 1)):
        graph.replay()
    torch.cuda.synchronize()
    same = all(torch.equal(a, b) for a, b in zip(grads_of(runner), eager))
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    same = same and all(torch.equal(a, b) for a, b in zip(grads_of(runner), eager))  # after the timed replays
    runner.n_steps += max(warmup, 1) + steps  # replays (the eager steps count themselves)
    del graph
    runner.zero()
    return ms, same


def time_phases(runner: Runner, iters: int):
    """GPU time of the phases of a step, from HIP events on torch's stream
    between them: selector preparation, forward (which runs the selector's
    sort), backward.  The iterations run back to back with no synchronisation,
    so where the host stays ahead of the GPU the events time the GPU's work,
    not host submission (in a host-bound step, as at the tiny fp32 shape, they
    also hold the GPU's waits for the host); call it after warm-up steps."""
    # one event per phase boundary: an iteration's end is the next one's start
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3 * iters + 1)]
    ev[0].record()
    for i in range(iters):
        runner.zero()
        s = runner.prepare()
        ev[3 * i + 1].record()
        y = runner.forward(s)
        ev[3 * i + 2].record()
        runner.backward(y)
        ev[3 * i + 3].record()
        runner.n_steps += 1
    torch.cuda.synchronize()
    acc = np.zeros(3)
    for i in range(iters):
        acc += [ev[3 * i + j].elapsed_time(ev[3 * i + j + 1]) for j in range(3)]
    return dict(zip(("prepare", "fwd", "bwd"), (acc / iters).tolist()))


def breakdown(phases, kt):
    """The step's GPU time split as the reference's benchmark reports it
    (benchmark_moe_shapes.py:100-124: sel, forward, backward): "sel" is the
    device time of the selector launches (the id copy and the stable sort;
    the sort runs inside cvmm(), in the same launches as the step's weight
    cast when the shapes allow), "fwd" the rest of the forward, "bwd" the
    backward.  Sums to the phases' GPU time."""
    sel = kt["sort"]["ms_per_step"] if "sort" in kt else 0.0
    return {"sel": sel, "fwd": phases["prepare"] + phases["fwd"] - sel, "bwd": phases["bwd"]}


def kernel_launchers(runner: Runner):
    """One C-ABI phase per entry, with every input already on the device, for
    ``--only`` (rocprofv3 runs of a single phase): routed GEMM forward, weight
    gradient, grad-input, bf16 weight copies."""
    C = runner.C
    s = runner.prepare()
    op = torch.bfloat16 if runner.p.amp else torch.float32
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=runner.p.amp):
        y = C.cvmm(runner.x, s, runner.keys)
    go = runner.p.grad_out.to(y.dtype)

    class Ctx:
        op_type = op

    args = (runner.x.detach(), runner.keys.detach(), s.raw_sel, s.sel, s.sel_index, s.out_index,
            None if runner.w is None else runner.w.detach())
    keys = runner.keys.detach()
    fast = C._fast_path(op, keys.shape[1], keys.shape[2])
    k = runner.p.weights.shape[-1] if runner.w is not None else runner.p.sel.shape[-1]
    plan = C._plan_copies(keys, op, runner.p.routes, k, runner.w is not None, not runner.p.route_input, True)
    kt, kn = C._cast_keys(keys, op, plan) if fast else (None, None)
    keys_f, fwd_t = C._copy_view(plan, kt, kn, True) if fast else (None, True)
    keys_x, bwd_t = C._copy_view(plan, kt, kn, False) if fast else (None, False)

    def cast():
        C._cast_keys(keys, op, plan)

    def fwd():
        C._forward(runner.x.detach(), s.sel_index, s.sel, keys, s.out_index, args[6], op, keys_f, fwd_t)

    def bwd_w():
        C._backward(Ctx, go, *args, False, True, False)

    def bwd_x():
        C._backward(Ctx, go, *args, True, False, runner.w is not None, keys_x=keys_x, keys_x_is_t=bwd_t)

    out = {"fwd": fwd, "bwd_w": bwd_w, "bwd_x": bwd_x}
    if fast:
        out["cast_keys"] = cast
    return out


# kernel classes timed by the library's hooks (CVMM_KC_* in include/cvmm_hip.h)
def _classes():
    from cvmm_codex_amd import _native as N
    return {"sort": N.KC_SORT, "offsets": N.KC_OFFSETS, "cast_keys": N.KC_CAST_KEYS,
            "gemm_fwd": N.KC_GEMM_FWD, "gemm_bwd_x": N.KC_GEMM_BWDX, "wgrad": N.KC_WGRAD,
            "combine": N.KC_COMBINE, "fill": N.KC_FILL}


def kernel_times(runner: Runner, steps: int):
    """Per-launch device time of every kernel class over `steps` training steps:
    the library brackets each launch with HIP events on its own stream."""
    import ctypes
    from cvmm_codex_amd import _native as N
    lib = N.lib()
    classes = _classes()
    runner.step()
    torch.cuda.synchronize()
    lib.cvmm_timing_enable(sum(classes.values()))
    try:
        for _ in range(steps):
            runner.step()
        torch.cuda.synchronize()
    finally:
        lib.cvmm_timing_enable(0)
    out = {}
    for name, cls in classes.items():
        ms, n = ctypes.c_double(), ctypes.c_int64()
        N.check(lib.cvmm_timing_result(cls, ctypes.byref(ms), ctypes.byref(n)), "cvmm_timing_result")
        if n.value:
            out[name] = {"avg_ms": ms.value / n.value, "launches_per_step": n.value / steps,
                         "ms_per_step": ms.value / steps}
    return out


# Roofline bound of each config (the per-config table of the measurement plan:
# wide experts are MFMA-bound, the narrow SwitchHead products HBM-bound on the
# per-route byte model).
BOUND = {"tiny_fp32": "mfma", "ff_up_1024": "mfma", "ff_down_1024_weighted": "mfma",
         "switch_v_2048": "hbm", "switch_o_2048_weighted": "hbm", "ffn_stack": "mfma"}
# kernel class -> phase of the byte model
PHASE = {"gemm_fwd": "fwd", "gemm_bwd_x": "dx", "wgrad": "dw"}


def phase_work(proj: W.Projection, phase: str):
    """Algorithmic flops and bytes of one phase (fwd, dx or dw) of one
    projection, on the per-route gather model: every route reads its own
    input row and dY row (a bytes per element: 2 under autocast, 4 in fp32),
    the fp32 weights are read once per phase, outputs are written once at
    op granularity (token rows for top-k sums), 12 bytes of route metadata
    per route.  fwd: R*Din*a + E*Din*Dout*4 + out + R*12, out = R*Dout*a or
    T*Dout*a + R*4 (weighted); dx: R*Dout*a + E*Din*Dout*4 + dX + R*12, dX =
    x_rows*Din*a or 2*R*Din*a + 2*R*4 (weighted: x re-read for the gate
    gradient, which is written); dw: R*Din*a + R*Dout*a (+ R*4 weighted) +
    E*Din*Dout*4 + R*12."""
    R = proj.routes
    E, d_in, d_out = proj.keys.shape
    top_k = proj.sel.shape[-1]
    a = 2 if proj.amp else 4
    tokens = R // top_k
    weighted = proj.weights is not None
    x_rows = R if proj.route_input else tokens
    w32 = E * d_in * d_out * 4
    flops = 2.0 * R * d_in * d_out
    if phase == "fwd":
        out = tokens * d_out * a + R * 4 if weighted else R * d_out * a
        return flops, R * d_in * a + w32 + out + R * 12
    if phase == "dx":
        dx = 2 * R * d_in * a + 2 * R * 4 if weighted else x_rows * d_in * a
        return flops, R * d_out * a + w32 + dx + R * 12
    if phase == "dw":
        return flops, R * d_in * a + R * d_out * a + (R * 4 if weighted else 0) + w32 + R * 12
    raise ValueError(phase)


def kernel_work(proj: W.Projection, name: str):
    """Algorithmic flops and bytes of ONE launch of a GEMM kernel class: those
    of its phase (phase_work); (None, None) for the other classes."""
    if name not in PHASE:
        return None, None
    return phase_work(proj, PHASE[name])


def step_work(proj: W.Projection):
    """(flops, route bytes) of a whole step: the three phases."""
    f, b = zip(*(phase_work(proj, ph) for ph in ("fwd", "dx", "dw")))
    return sum(f), sum(b)


def roofline_of(bound: str, dtype: str, flops: float, nbytes: float, sec: float, traffic=None):
    """Both fractions of one launch (or step) taking `sec` seconds; `frac` is
    the one of the config's bound."""
    mfma = flops / sec / 1e12
    hbm = nbytes / sec / 1e9
    out = {"bound": bound}
    if bound == "mfma":
        out.update({"achieved": round(mfma, 3), "peak": PEAK[dtype], "unit": "TFLOP/s",
                    "frac": round(mfma / PEAK[dtype], 5)})
    else:
        out.update({"achieved": round(hbm, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(hbm / HBM_PEAK_GBS, 5)})
    out.update({"traffic": traffic, "mfma_frac": round(mfma / PEAK[dtype], 5),
                "hbm_frac": round(hbm / HBM_PEAK_GBS, 5), "algorithmic_flops": flops,
                "algorithmic_bytes": int(nbytes),
                "traffic_over_algorithmic": None if traffic is None else round(traffic / nbytes, 3)})
    return out


def copy_calibration(nbytes: int = 256 << 20, iters: int = 5):
    """A plain device copy of known size: the reference reading of FETCH_SIZE
    and WRITE_SIZE (nbytes read and nbytes written per launch)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {nbytes} bytes {iters} times")


def _cpu_model() -> str:
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:  # pragma: no cover
        pass
    return "unknown"


def cpu_baseline(proj: W.Projection, cap_s: float = 120.0):
    """The reference's PyTorch CPU CVMM path (oracle/torch_cpu_path.py: stable
    sort, per-expert gather + matmul, forward and backward) on the host cores
    in float32: 1 warmup and 3 timed iterations of the full workload, median.
    Threads: torch's count (the box's CPU share, OMP_NUM_THREADS)."""
    from oracle import torch_cpu_path as P
    x = proj.x.float()
    keys = proj.keys.float()
    w = None if proj.weights is None else proj.weights.float()
    gy = proj.grad_out.float()
    times = []
    for i in range(4):
        t0 = time.perf_counter()
        P.step(x, proj.sel, keys, w, gy, proj.route_input)
        el = time.perf_counter() - t0
        if i > 0:
            times.append(el)
        if el > cap_s:
            return {"value": None, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
                    "sample": f"skipped: one iteration took {el:.0f} s (> {cap_s:.0f} s)"}
    med = sorted(times)[1]
    return {"value": round(proj.flops / med / 1e12, 6), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "ms_per_iter": round(med * 1e3, 2), "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "cpu_model": _cpu_model(),
            "sample": f"full {proj.name} workload in float32, torch CPU path (sort + per-expert gather/matmul, "
                      f"fwd + bwd), 1 warmup + 3 timed iterations, median of "
                      f"{', '.join(f'{t * 1e3:.0f}' for t in times)} ms"}


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch of a kernel class from its profile.sh counters
    (profiles/traffic_<class>_<workload>.json), None where none were taken."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if os.path.exists(path):
        with open(path) as f:
            d = json.load(f)
        return d.get("bytes_per_launch") if isinstance(d, dict) else None
    return None


def fabric_of(workload: str, ms: float):
    """The fabric side of a step: FETCH_SIZE + WRITE_SIZE bytes of every
    kernel of a step (profiles/traffic_step_<workload>.json, from a profile.sh
    run) over the measured step time, as a fraction of 8 TB/s -- beside the
    route-byte model's fraction, which counts gathers that L2 and MALL serve."""
    path = os.path.join(ROOT, "profiles", f"traffic_step_{workload}.json")
    if not os.path.exists(path):
        return {"fabric_frac": None}
    with open(path) as f:
        b = json.load(f)["fabric_bytes_per_step"]
    return {"fabric_bytes_per_step": b, "fabric_gbs": round(b / (ms * 1e-3) / 1e9, 1),
            "fabric_frac": round(b / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)}


def router_times(iters: int = 50, T: int = 16384, E: int = 128, k: int = 8):
    """The router of the FFN stack ([16384, 128]
    bf16 logits, top-8, renormalised) two ways: the reference callers' torch
    lines (softmax, topk, renormalise; benchmark_ffn_moe.py:92-95) followed by
    this library's selector sort, and the fused cvmm_route_topk.  Forward, and
    forward + backward to the logits; HIP events around `iters` calls each."""
    import cvmm_codex_amd as C
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(T, E, generator=g) * 2).to(torch.bfloat16).cuda().requires_grad_(True)
    gw = torch.randn(T, k, generator=g).cuda()

    def torch_lines(backward):
        probs = torch.softmax(logits.float(), dim=-1)
        w, sel = probs.topk(k, dim=-1)
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-20)
        s = C.cvmm_prepare_sel2(sel)
        s._resolve(E)
        if backward:
            w.backward(gw)

    def fused(backward):
        w, _, _ = C.cvmm_route_topk(logits, k, True)
        if backward:
            w.backward(gw)

    def timed(fn, backward):
        for _ in range(5):
            fn(backward)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn(backward)
        b.record()
        b.synchronize()
        return a.elapsed_time(b) * 1000.0 / iters

    out = {"shape": {"tokens": T, "experts": E, "top_k": k, "logits": "bf16"}}
    for name, fn in (("torch_lines", torch_lines), ("fused", fused)):
        out[name] = {"fwd_us": round(timed(fn, False), 2), "fwd_bwd_us": round(timed(fn, True), 2)}
    return out


class _Shape:
    """Shape stand-in of a Projection for phase_work (meta tensors)."""

    def __init__(self, R, k, E, d_in, d_out, weighted, route_input):
        m = torch.device("meta")
        self.sel = torch.empty(R // k, k, device=m)
        self.keys = torch.empty(E, d_in, d_out, device=m)
        self.weights = torch.empty(R // k, k, device=m) if weighted else None
        self.route_input, self.amp = route_input, True

    @property
    def routes(self):
        return self.sel.numel()


def ffn_line(steps: int = 10, warmup: int = 3, kernel_iters: int = 10, variant: str = "both"):
    """The FFN stack of BASELINE.json configs[4] (16384 tokens, 2048 -> 512 ->
    2048, 128 experts, top-8, Zipf-skewed gate; benchmark_ffn_moe.py:89-98),
    forward + backward, as one bench line: the library's fused router and up
    projection + GELU (``value``), beside the stack written as the
    reference's callers write it (torch router lines, F.gelu around cvmm).
    variant "fused" runs the fused stack only (profile runs: one stack per
    trace)."""
    s = W.c5_ffn_stack().to(torch.device("cuda"))
    params = [t.clone().requires_grad_(True) for t in (s.x, s.gate, s.w_up, s.w_down)]
    import cvmm_codex_amd as C

    n_steps = [0]

    def step(fwd):
        for t in params:
            t.grad = None
        out = fwd(s, C, *params)
        out.backward(s.grad_out)
        n_steps[0] += 1

    def timed(fwd, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            step(fwd)
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / n

    res = {"composed": None}
    stacks = (("composed", W.ffn_forward), ("fused", W.ffn_forward_fused))
    for name, fwd in stacks if variant == "both" else stacks[1:]:
        for _ in range(warmup):
            step(fwd)
        torch.cuda.synchronize()
        res[name] = timed(fwd, steps)
    ms = res["fused"]

    class _Runner:
        def step(self):
            step(W.ffn_forward_fused)

    kt = kernel_times(_Runner(), kernel_iters)
    log(f"steps run: {n_steps[0]}")
    T, D = s.x.shape[0] * s.x.shape[1], s.x.shape[2]
    E, _, H = s.w_up.shape
    R = T * s.k
    up = _Shape(R, s.k, E, D, H, False, False)
    down = _Shape(R, s.k, E, H, D, True, True)
    dom = max((k for k in kt if k in PHASE), key=lambda k: kt[k]["ms_per_step"])
    # both projections' launches of a class have the same flops (2 R D H)
    flops = phase_work(up, PHASE[dom])[0]
    nbytes = (phase_work(up, PHASE[dom])[1] + phase_work(down, PHASE[dom])[1]) / 2
    roofline = roofline_of("mfma", "bf16", flops, nbytes, kt[dom]["avg_ms"] * 1e-3, load_traffic(dom, "ffn_stack"))
    roofline.update({"kernel": dom, "avg_launch_ms": round(kt[dom]["avg_ms"], 5),
                     "note": "per launch; the class runs once per projection, bytes averaged over the two"})
    gate_flops = 6.0 * T * D * E
    route_bytes = step_work(up)[1] + step_work(down)[1] + 3 * T * D * 2 + 3 * D * E * 4
    step_roof = roofline_of("mfma", "bf16", s.flops, route_bytes, ms * 1e-3)
    return {
        "metric": METRIC, "value": round(s.flops / (ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded CPU generator, BASELINE.json recipe)",
        "config": {"workload": "ffn_stack", "tokens": T, "d_model": D, "hidden": H, "n_experts": E,
                   "top_k": s.k, "gate": "softmax top-8, Zipf(1.1) bias", "step": "router+up+gelu+down fwd+bwd",
                   "gflop_per_step": round(s.flops / 1e9, 3), "gate_gflop": round(gate_flops / 1e9, 3)},
        "composed_ms_per_step": None if res["composed"] is None else round(res["composed"], 5),
        "step_roofline": step_roof,
        "kernel_ms_per_launch": {k: round(v["avg_ms"], 5) for k, v in kt.items()},
        "kernel_launches_per_step": {k: v["launches_per_step"] for k, v in kt.items()},
        "roofline": roofline,
        "cpu_baseline": None,
    }


# ---------------------------------------------------------------------------
# summaries of profile.sh runs (rocprofv3 CSVs -> the markdown under profiles/)
# ---------------------------------------------------------------------------
N_XCC, CU_NUM, SIMD_NUM = 8, 256, 1024
COPY_BYTES = 256 << 20                      # the copy calibration's bytes read and written per launch


def _demangle(names):
    """Demangled kernel names; the bf16 type's mangling (DF16b) is given to
    c++filt as a vendor type named bf16, which it does understand."""
    import subprocess
    names = list(names)
    fixed = [n.replace("DF16b", "u4bf16") if n.startswith("_Z") else n for n in names]
    try:
        out = subprocess.run(["c++filt"], input="\n".join(fixed), capture_output=True, text=True,
                             timeout=30).stdout.splitlines()
        return out if len(out) == len(names) else names
    except Exception:  # pragma: no cover
        return names


def _template_args(name: str):
    """Top-level template arguments of a demangled kernel name."""
    i = name.find("<")
    if i < 0:
        return []
    depth, cur, out = 0, "", []
    for ch in name[i + 1:]:
        if ch == "<":
            depth += 1
        elif ch == ">":
            if depth == 0:
                out.append(cur.strip())
                break
            depth -= 1
        elif ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
            continue
        cur += ch
    return out


def kernel_role(name: str):
    """The kernel class of a demangled cvmm kernel name: its Role template
    argument tells the forward GEMM (0) from the grad-input GEMM (1)."""
    base = name.split("<")[0].split("(")[0].split()[-1] if name else ""
    args = _template_args(name)
    role_pos = {"cvmm::routed_gemm_ring_kernel": 7, "cvmm::routed_gemm_panel_kernel": 4,
                "cvmm::routed_gemm_nt_kernel": 3, "cvmm::routed_gemm_nloop_kernel": 3}
    if "wgrad" in base:
        return "wgrad"
    if base in role_pos and len(args) > role_pos[base]:
        return "gemm_bwd_x" if args[role_pos[base]] == "1" else "gemm_fwd"
    if base == "cvmm::routed_gemm_kernel":
        return "gemm"
    return None


def kernel_class(name: str):
    """kernel_role for the routed GEMMs and the weight gradient; the other
    kernels of a step by name: the dense top-k GEMM, its preparation (slot
    table, weighted row scaling, operand copy), the combine, the sort, the
    weight cast; torch's own kernels (the gate GEMMs of the FFN stack, its
    elementwise ops) are "torch"."""
    role = kernel_role(name)
    if role is not None:
        return role
    base = name.split("<")[0].split("(")[0].split()[-1] if name else ""
    if base.startswith("cvmm::"):
        for key, cls in (("routed_small", "gemm"), ("topk_gemm", "dense_topk"), ("topk_slot_table", "dense_prep"),
                         ("scale_rows", "dense_prep"), ("copy_rows_op", "dense_prep"),
                         ("combine_rows", "combine"), ("sort_", "sort"), ("cast_keys", "cast"),
                         ("copy_ids", "sort"), ("sum_partials", "dgate"), ("fill_zero", "fill"), ("gelu", "gelu"),
                         ("route", "router")):
            if key in base:
                return cls
        return "cvmm"
    if name:
        return "torch"
    return None


def _short(name: str, width: int = 90) -> str:
    n = name.replace("__hip_bfloat16", "bf16").replace("_Float16", "f16").replace("cvmm::", "")
    n = n.split("(")[0] if n.startswith("void ") or "(" in n else n
    n = n.replace("void ", "")
    return n if len(n) <= width else n[:width - 3] + "..."


def _read_csv(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def _counters(pass_dir):
    """{demangled kernel name: {counter: [per-dispatch values]}} of one pass."""
    import glob
    out = {}
    files = glob.glob(os.path.join(pass_dir, "**", "*counter_collection.csv"), recursive=True)
    rows = [r for f in files for r in _read_csv(f)]
    names = dict(zip(sorted({r["Kernel_Name"] for r in rows}), _demangle(sorted({r["Kernel_Name"] for r in rows}))))
    for r in rows:
        d = out.setdefault(names[r["Kernel_Name"]], {})
        d.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return out


def _copy_factors(copy_dir):
    """Bytes per counter byte of FETCH_SIZE and WRITE_SIZE: what a plain
    device copy of COPY_BYTES moves / what the counter reads for it."""
    f = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = []
        for name, cs in _counters(os.path.join(copy_dir, c)).items():
            vals += [v for v in cs.get(c, []) if v * 1024 > COPY_BYTES / 8]     # the big copy launches
        if vals:
            f[c] = COPY_BYTES / (sum(vals) / len(vals) * 1024)
    return f


def step_fabric(dirpath: str, copy_dir: str):
    """FETCH_SIZE + WRITE_SIZE bytes of one step on the fabric side: every
    traced kernel's bytes per dispatch (counter runs, copy-calibrated) times
    its dispatches in the kernel-trace run, over the steps that run made
    (its "steps run: N" log line).  Kernels without counters are left out;
    `covered` is the share of traced kernel time that has them."""
    import glob
    import re
    stats = glob.glob(os.path.join(dirpath, "trace", "**", "*kernel_stats.csv"), recursive=True)
    log_path = os.path.join(dirpath, "trace.log")
    if not stats or not os.path.exists(log_path) or not copy_dir:
        return None
    runs = re.findall(r"steps run: (\d+)", open(log_path).read())
    if not runs:
        return None
    n = int(runs[-1])
    cnt = {}
    for pas in ("fetch", "write"):
        for k, d in _counters(os.path.join(dirpath, pas)).items():
            cnt.setdefault(k, {}).update(d)
    fac = _copy_factors(copy_dir)
    rows = _read_csv(stats[0])
    names = _demangle([r["Name"] for r in rows])
    total_b = covered_t = all_t = 0.0
    for r, name in zip(rows, names):
        t = float(r["TotalDurationNs"])
        all_t += t
        d = cnt.get(name)
        if not d or not d.get("FETCH_SIZE") or not d.get("WRITE_SIZE"):
            continue
        per = (sum(d["FETCH_SIZE"]) / len(d["FETCH_SIZE"]) * fac["FETCH_SIZE"] +
               sum(d["WRITE_SIZE"]) / len(d["WRITE_SIZE"]) * fac["WRITE_SIZE"]) * 1024
        total_b += per * int(r["Calls"])
        covered_t += t
    return {"kernel": "step", "workload": os.path.basename(os.path.normpath(dirpath)), "steps_traced": n,
            "fabric_bytes_per_step": int(total_b / n), "covered": round(covered_t / all_t, 4) if all_t else None,
            "copy_factor_fetch": fac["FETCH_SIZE"], "copy_factor_write": fac["WRITE_SIZE"]}


def summarize(dirpath: str, copy_dir=None) -> str:
    import glob
    W_name = os.path.basename(os.path.normpath(dirpath))
    lines = [f"# {W_name} -- rocprofv3 evidence", ""]
    lines += ["Commands (repo root, one MI355X):", "", "```",
              f"export TMPDIR=/tmp",
              f"bash profile.sh {W_name} gpurun_out/prof   # bench line, kernel trace, three counter passes",
              "bash profile.sh copy gpurun_out/prof         # FETCH_SIZE / WRITE_SIZE calibration",
              f"python bench.py --summarize gpurun_out/prof/{W_name} --copy-dir gpurun_out/prof/copy", "```", ""]
    bench = None
    bj = os.path.join(dirpath, "bench.json")
    if os.path.exists(bj):
        txt = [ln for ln in open(bj).read().splitlines() if ln.strip().startswith("{")]
        bench = json.loads(txt[-1]) if txt else None
    if bench:
        rf, sr = bench["roofline"], bench["step_roofline"]
        lines += ["## bench.py line (HIP events)", "",
                  f"- step: {bench['ms_per_step'] * 1e3:.1f} us = {bench['value']:.1f} TFLOP/s; step roofline "
                  f"({sr['bound']}): frac {sr['frac']:.4f} (MFMA {sr['mfma_frac']:.4f}, HBM route bytes "
                  f"{sr['hbm_frac']:.4f})",
                  f"- dominant kernel `{rf['kernel']}`: {rf['avg_launch_ms'] * 1e3:.1f} us per launch, "
                  f"{rf['achieved']} {rf['unit']} = frac {rf['frac']:.4f} of {rf['peak']} ({rf['bound']}); "
                  f"MFMA frac {rf['mfma_frac']:.4f}, HBM frac {rf['hbm_frac']:.4f}",
                  f"- kernel us per launch: " + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in
                                                          bench["kernel_ms_per_launch"].items())]
        cfg = bench.get("config", {})
        if cfg.get("launch") == "hip_graph":
            lines.append(f"- steps timed as HIP graph replays of one captured step (selector, forward, backward; "
                         f"eager step {cfg['eager_ms_per_step'] * 1e3:.1f} us on the same box, host-bound); "
                         f"replay gradients bit-identical to an eager step's: {cfg['graph_bit_identical']}")
        if "breakdown_ms" in bench:
            lines.append("- step breakdown (GPU time): " + ", ".join(
                f"{k} {v * 1e3:.1f} us" for k, v in bench["breakdown_ms"].items()) +
                f" (sum {sum(bench['breakdown_ms'].values()) * 1e3:.1f} us)")
        fab = step_fabric(dirpath, copy_dir)
        if fab:
            gbs = fab["fabric_bytes_per_step"] / (bench["ms_per_step"] * 1e-3) / 1e9
            lines.append(f"- fabric side: FETCH + WRITE {fab['fabric_bytes_per_step'] / 1e6:.1f} MB per step "
                         f"({fab['steps_traced']} traced steps, {fab['covered'] * 100:.1f} % of kernel time "
                         f"counted) = {gbs:.0f} GB/s = frac {gbs / HBM_PEAK_GBS:.4f} of 8 TB/s, beside the "
                         f"route-byte model's {sr['hbm_frac']:.4f}")
        lines.append("")
    stats = glob.glob(os.path.join(dirpath, "trace", "**", "*kernel_stats.csv"), recursive=True)
    avg_us = {}
    if stats:
        rows = _read_csv(stats[0])
        names = _demangle([r["Name"] for r in rows])
        lines += ["## Kernel trace (`rocprofv3 --kernel-trace --stats`, bench run of 20 steps)", "",
                  "| kernel | class | calls | avg us | % |", "|---|---|---:|---:|---:|"]
        for r, n in zip(rows, names):
            avg_us[n] = float(r["AverageNs"]) / 1e3
            if float(r["Percentage"]) < 0.5:
                continue
            lines.append(f"| `{_short(n)}` | {kernel_class(n) or ''} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} "
                         f"| {float(r['Percentage']):.1f} |")
        lines.append("")
    cnt = {}
    for pas in ("fetch", "write", "sq"):
        for k, d in _counters(os.path.join(dirpath, pas)).items():
            cnt.setdefault(k, {}).update(d)
    fac = _copy_factors(copy_dir) if copy_dir else {}
    proj = None
    if W_name in W.PROJECTIONS:
        proj = W.PROJECTIONS[W_name]()
    if cnt:
        lines += ["## Counters per dispatch (averages over the counter runs' dispatches)", "",
                  "FETCH/WRITE: `FETCH_SIZE` / `WRITE_SIZE` (KiB) x 1024 x the copy factor "
                  f"(fetch {fac.get('FETCH_SIZE', float('nan')):.3f}, write {fac.get('WRITE_SIZE', float('nan')):.3f}: "
                  "bytes a 256 MiB device copy moves / what the counter reads for it).  MFMA busy = "
                  "`SQ_VALU_MFMA_BUSY_CYCLES` / (`GRBM_GUI_ACTIVE` / 8 XCDs x 1024 SIMDs).  MFMA GFLOP = "
                  "`SQ_INSTS_VALU_MFMA_MOPS_*` x 512.  LDS conflict = `SQ_LDS_BANK_CONFLICT` cycles per "
                  "`SQ_INSTS_LDS` instruction and as % of CU time (`SQ_LDS_BANK_CONFLICT` / (`GRBM_GUI_ACTIVE`/8 x 256)).  "
                  "L2 hit = `TCC_HIT_sum` / (`TCC_HIT_sum` + `TCC_MISS_sum`).", "",
                  "| kernel | class | trace us | FETCH MB | WRITE MB | alg. MB | traffic / alg. | L2 hit % | "
                  "MFMA busy % | MFMA GFLOP (alg.) | LDS confl. cyc/inst | LDS confl. % |",
                  "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
        def order(item):
            c = kernel_class(item[0])
            return (c not in PHASE, -avg_us.get(item[0], 0.0))
        for k, d in sorted(cnt.items(), key=order):
            role = kernel_class(k)
            if role is None or avg_us.get(k, 0.0) < 1.0:
                continue
            mean = lambda c: (sum(d[c]) / len(d[c])) if c in d and d[c] else float("nan")
            fetch = mean("FETCH_SIZE") * 1024 * fac.get("FETCH_SIZE", float("nan")) / 1e6
            write = mean("WRITE_SIZE") * 1024 * fac.get("WRITE_SIZE", float("nan")) / 1e6
            alg = phase_work(proj, PHASE[role])[1] / 1e6 if proj is not None and role in PHASE else float("nan")
            hit = mean("TCC_HIT_sum") / (mean("TCC_HIT_sum") + mean("TCC_MISS_sum")) * 100
            grbm = mean("GRBM_GUI_ACTIVE") / N_XCC
            busy = mean("SQ_VALU_MFMA_BUSY_CYCLES") / (grbm * SIMD_NUM) * 100
            mops = (mean("SQ_INSTS_VALU_MFMA_MOPS_BF16") if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in d else 0) + \
                   (mean("SQ_INSTS_VALU_MFMA_MOPS_F32") if "SQ_INSTS_VALU_MFMA_MOPS_F32" in d else 0)
            gflop = mops * 512 / 1e9
            alg_gf = phase_work(proj, PHASE[role])[0] / 1e9 if proj is not None and role in PHASE else float("nan")
            conf = mean("SQ_LDS_BANK_CONFLICT")
            per_inst = conf / mean("SQ_INSTS_LDS") if mean("SQ_INSTS_LDS") else float("nan")
            conf_pct = conf / (grbm * CU_NUM) * 100
            us = avg_us.get(k, float("nan"))
            ratio = f"{(fetch + write) / alg:.2f}" if alg == alg else "-"
            alg_s = f"{alg:.1f}" if alg == alg else "-"
            gf = f"{gflop:.2f} ({alg_gf:.2f})" if alg_gf == alg_gf else f"{gflop:.2f}"
            lines.append(f"| `{_short(k, 70)}` | {role} | {us:.1f} | {fetch:.1f} | {write:.1f} | {alg_s} | "
                         f"{ratio} | {hit:.1f} | {busy:.1f} | {gf} | {per_inst:.3f} | {conf_pct:.2f} |")
        lines.append("")
    return "\n".join(lines)


def traffic_json(dirpath: str, copy_dir: str, cls: str):
    if cls == "step":
        return step_fabric(dirpath, copy_dir)
    return _traffic_json(dirpath, copy_dir, cls)


def _traffic_json(dirpath: str, copy_dir: str, cls: str):
    """FETCH_SIZE + WRITE_SIZE bytes per launch of the class's kernel (the
    `traffic` field of bench.py's roofline), from a profile.sh run.  A GEMM
    class that ran as the dense top-k path counts the dense GEMM plus its
    preparation launches (slot table, and the row scaling when weighted)."""
    cnt = {}
    for pas in ("fetch", "write"):
        for k, d in _counters(os.path.join(dirpath, pas)).items():
            cnt.setdefault(k, {}).update(d)
    fac = _copy_factors(copy_dir)

    def per_launch(d):
        f = sum(d["FETCH_SIZE"]) / len(d["FETCH_SIZE"]) * 1024 * fac["FETCH_SIZE"]
        w = sum(d["WRITE_SIZE"]) / len(d["WRITE_SIZE"]) * 1024 * fac["WRITE_SIZE"]
        return f, w

    base = {"kernel": cls, "workload": os.path.basename(os.path.normpath(dirpath)),
            "copy_factor_fetch": fac["FETCH_SIZE"], "copy_factor_write": fac["WRITE_SIZE"]}
    for k, d in cnt.items():
        if kernel_role(k) == cls and "FETCH_SIZE" in d and "WRITE_SIZE" in d:
            f, w = per_launch(d)
            return {**base, "kernel_name": k, "bytes_per_launch": int(f + w), "fetch_bytes": int(f),
                    "write_bytes": int(w)}
    if cls in ("gemm_fwd", "gemm_bwd_x"):
        dense = [(k, d) for k, d in cnt.items() if kernel_class(k) in ("dense_topk", "dense_prep")
                 and "FETCH_SIZE" in d and "WRITE_SIZE" in d]
        if any(kernel_class(k) == "dense_topk" for k, _ in dense):
            f = w = 0.0
            for k, d in dense:
                df, dw = per_launch(d)
                f, w = f + df, w + dw
            return {**base, "kernel_name": "dense top-k: " + ", ".join(k for k, _ in dense),
                    "bytes_per_launch": int(f + w), "fetch_bytes": int(f), "write_bytes": int(w)}
    return None



def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(W.PROJECTIONS))
    ap.add_argument("--kernel-iters", type=int, default=100)
    ap.add_argument("--graph", action="store_true",
                    help="time the K steps as replays of one HIP graph captured from a step (for a "
                         "host-bound step, as at the tiny fp32 shape); phases and kernels stay eager")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["fwd", "bwd_w", "bwd_x", "cast_keys", "copy"], default=None,
                    help="launch only this phase --steps times, or the copy calibration (rocprofv3 runs)")
    ap.add_argument("--ffn", action="store_true",
                    help="time the FFN stack (configs[4]) with the fused router and GELU, beside the composed "
                         "stack (one JSON line) and exit")
    ap.add_argument("--ffn-variant", choices=["both", "fused"], default="both",
                    help="with --ffn: time the composed stack too (both) or the fused one only")
    ap.add_argument("--router", action="store_true",
                    help="time the fused router against the torch router lines (one JSON line) and exit")
    ap.add_argument("--summarize", metavar="DIR", default=None,
                    help="print the markdown summary of a profile.sh output directory (no GPU needed) and exit")
    ap.add_argument("--copy-dir", metavar="DIR", default=None,
                    help="with --summarize: the profile.sh copy-calibration directory")
    ap.add_argument("--traffic", metavar="CLASS", default=None,
                    help="with --summarize: print the traffic JSON of this kernel class (gemm_fwd, gemm_bwd_x, "
                         "wgrad), or of the whole step (step)")
    ap.add_argument("--tune", action="append", default=[], metavar="KNOB=VALUE",
                    help="set a library tuning knob (panel_tiles_per_wg, wgrad_order, wgrad_tile, gemm_order, "
                         "dense_topk, sort_chunk, ring_tile, wgrad_chunk) before running")
    args = ap.parse_args()

    if args.summarize:
        if args.traffic:
            print(json.dumps(traffic_json(args.summarize, args.copy_dir, args.traffic), indent=1))
        else:
            print(summarize(args.summarize, args.copy_dir))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard over experts, which is not built here)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    from cvmm_codex_amd import _native as N
    knobs = {"panel_tiles_per_wg": N.TUNE_PANEL_TILES_PER_WG, "wgrad_order": N.TUNE_WGRAD_ORDER,
             "gemm_order": N.TUNE_GEMM_ORDER,
             "wgrad_tile": N.TUNE_WGRAD_TILE, "dense_topk": N.TUNE_DENSE_TOPK,
             "sort_chunk": N.TUNE_SORT_CHUNK, "ring_tile": N.TUNE_RING_TILE, "wgrad_chunk": N.TUNE_WGRAD_CHUNK}
    for kv in args.tune:
        name, _, value = kv.partition("=")
        if name not in knobs:
            ap.error(f"--tune: unknown knob {name!r} (known: {', '.join(sorted(knobs))})")
        rc = N.lib().cvmm_tuning_set(knobs[name], int(value))
        if rc != 0:
            ap.error(f"--tune {kv}: {N.lib().cvmm_last_error().decode()}")

    dev = torch.device("cuda:0")
    if args.router:
        print(json.dumps({"router": router_times()}), flush=True)
        return
    import cvmm_codex_amd.api as C
    C.cvmm_log_shapes = False   # stdout carries the one JSON line
    if args.ffn:
        print(json.dumps(ffn_line(args.steps, args.warmup, args.kernel_iters, args.ffn_variant)), flush=True)
        return
    if args.only == "copy":
        copy_calibration(iters=args.steps)
        return
    proj = W.PROJECTIONS[args.workload]()
    runner = Runner(proj, dev)

    if args.only:
        fn = kernel_launchers(runner)[args.only]
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        log(f"launched {args.only} {args.steps} times")
        return

    log(f"workload {proj.name}: R={proj.routes} d_in={proj.keys.shape[1]} d_out={proj.keys.shape[2]} "
        f"E={proj.keys.shape[0]}")
    # W warm-up steps, then the per-phase and per-kernel passes, then the
    # timed steps (after W more): a fresh process runs its first ~100 steps
    # up to 8 % slower on the GPU (per-step GPU time falls from ~160 to ~149
    # us at ff_up; host submission stays ~90 us ahead)
    for _ in range(args.warmup):
        runner.step()
    phases = time_phases(runner, max(10, args.steps // 2))
    log(f"phases {phases}")
    kt = kernel_times(runner, args.kernel_iters)
    log("kernel ms/launch " + json.dumps({k: round(v["avg_ms"], 5) for k, v in kt.items()}))
    ms = time_steps(runner, args.steps, args.warmup)
    log(f"step {ms:.4f} ms")
    launch = {"launch": "eager"}
    if args.graph:
        eager_ms = ms
        ms, same = time_steps_graph(runner, args.steps, args.warmup)
        log(f"graph replay {ms:.4f} ms per step (eager {eager_ms:.4f}), gradients bit-identical: {same}")
        if not same:
            raise SystemExit("bench: graph replay gradients differ from an eager step's")
        launch = {"launch": "hip_graph", "eager_ms_per_step": round(eager_ms, 5),
                  "graph_bit_identical": same}
    dtype = "bf16" if proj.amp else "fp32"
    bound = BOUND[proj.name]
    # dominant kernel: the GEMM class with the most device time per step
    dom = max((k for k in kt if k in PHASE), key=lambda k: kt[k]["ms_per_step"])
    flops, nbytes = kernel_work(proj, dom)
    roofline = roofline_of(bound, dtype, flops, nbytes, kt[dom]["avg_ms"] * 1e-3, load_traffic(dom, proj.name))
    roofline.update({"kernel": dom, "avg_launch_ms": round(kt[dom]["avg_ms"], 5)})
    sflops, sbytes = step_work(proj)
    step_roof = roofline_of(bound, dtype, sflops, sbytes, ms * 1e-3)
    step_roof.update(fabric_of(proj.name, ms))
    log(f"steps run: {runner.n_steps}")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(proj)

    value = proj.flops / (ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded CPU generator, BASELINE.json recipe)",
        "config": {"workload": proj.name, "routes": proj.routes, "d_in": proj.keys.shape[1],
                   "d_out": proj.keys.shape[2], "n_experts": proj.keys.shape[0],
                   "top_k": proj.sel.shape[-1], "weighted": proj.weights is not None,
                   "step": "sel+fwd+bwd", "gflop_per_step": round(proj.flops / 1e9, 3), **launch},
        "step_roofline": step_roof,
        "breakdown_ms": {k: round(v, 5) for k, v in breakdown(phases, kt).items()},
        "kernel_ms_per_launch": {k: round(v["avg_ms"], 5) for k, v in kt.items()},
        "kernel_ms_per_step": {k: round(v["ms_per_step"], 5) for k, v in kt.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
