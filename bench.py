"""CVMM forward+backward benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload ff_up_1024]

A step = one pass of the CVMM hot path over one batch of synthetic input:
selector preparation (stable counting sort), forward, and backward (grad x,
grad keys, grad reduction weight), launched by the drop-in API exactly as a
training step would.  ``value`` is whole-job TFLOP/s = 6*R*d_in*d_out / step
time (inputs resident in HBM).  Every kernel is also timed on its own: the
library brackets each launch with HIP events on the stream it runs on, and the
kernel class with the most device time per step gives ``roofline``
(algorithmic bytes or flops of one launch / its average launch time).  The CPU
oracle is timed on a bounded sample of the same workload as ``cpu_baseline``.
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


def time_steps(runner: Runner, steps: int, warmup: int):
    for _ in range(warmup):
        runner.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        runner.step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def time_phases(runner: Runner, iters: int):
    """HIP events between the phases of a step (current stream).  "sel" is the
    selector bookkeeping; the sort itself runs in "fwd" (inside cvmm())."""
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    acc = np.zeros(3)
    for _ in range(iters):
        runner.zero()
        ev[0].record()
        s = runner.prepare()
        ev[1].record()
        y = runner.forward(s)
        ev[2].record()
        runner.backward(y)
        ev[3].record()
        torch.cuda.synchronize()
        acc += [ev[i].elapsed_time(ev[i + 1]) for i in range(3)]
    return dict(zip(("sel", "fwd", "bwd"), (acc / iters).tolist()))


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
    kt, kn = C._cast_keys(keys, op, True, True) if fast else (None, None)

    def cast():
        C._cast_keys(keys, op, True, True)

    def fwd():
        C._forward(runner.x.detach(), s.sel_index, s.sel, keys, s.out_index, args[6], op, kt)

    def bwd_w():
        C._backward(Ctx, go, *args, False, True, False)

    def bwd_x():
        C._backward(Ctx, go, *args, True, False, runner.w is not None, keys_n=kn)

    out = {"fwd": fwd, "bwd_w": bwd_w, "bwd_x": bwd_x}
    if fast:
        out["cast_keys"] = cast
    return out


# kernel classes timed by the library's hooks (CVMM_KC_* in include/cvmm_hip.h)
def _classes():
    from cvmm_codex_amd import _native as N
    return {"sort": N.KC_SORT, "offsets": N.KC_OFFSETS, "cast_keys": N.KC_CAST_KEYS,
            "gemm_fwd": N.KC_GEMM_FWD, "gemm_bwd_x": N.KC_GEMM_BWDX, "wgrad": N.KC_WGRAD,
            "combine": N.KC_COMBINE, "fill": N.KC_FILL, "reduce": N.KC_REDUCE}


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


def kernel_work(proj: W.Projection, name: str):
    """Algorithmic flops and HBM bytes of ONE launch of a hot kernel class:
    every operand byte read once and every result byte written once, at the
    storage widths the fast path uses (16-bit operands under autocast, fp32
    weight gradient)."""
    R = proj.routes
    E, d_in, d_out = proj.keys.shape
    top_k = proj.sel.shape[-1]
    b = 2 if proj.amp else 4
    tokens = R // top_k
    weighted = proj.weights is not None
    x_rows = R if proj.route_input else tokens
    keys_b = E * d_in * d_out * b
    flops = 2.0 * R * d_in * d_out
    if name == "gemm_fwd":
        # x rows + weight copy + y (output rows, or the route-ordered buffer the combine reads)
        return flops, x_rows * d_in * b + keys_b + R * d_out * b
    if name == "gemm_bwd_x":
        g_rows = tokens if weighted else R
        by = g_rows * d_out * b + keys_b + R * d_in * b
        if weighted:  # routing-weight gradient: x rows re-read, one fp32 partial per route and n-tile
            by += x_rows * d_in * b + R * max(1, d_in // 128) * 4
        return flops, by
    if name == "wgrad":
        g_rows = tokens if weighted else R
        return flops, x_rows * d_in * b + g_rows * d_out * b + E * d_in * d_out * 4
    if name == "reduce":
        # top-k sum without a route buffer (weighted forward of route rows, or
        # the token gradient): gathered route rows (K wide), 8 bytes of route
        # info per route, the weight copy, one output row (N wide) per token
        K, n = (d_in, d_out) if proj.route_input else (d_out, d_in)
        return flops, R * K * b + R * 8 + keys_b + tokens * n * b
    return None, None


def copy_calibration(nbytes: int = 256 << 20, iters: int = 5):
    """A plain device copy of known size: the reference reading of FETCH_SIZE
    and WRITE_SIZE (nbytes read and nbytes written per launch)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {nbytes} bytes {iters} times")


def cpu_baseline(proj: W.Projection, budget_s: float = 12.0):
    """The oracle on the host cores: forward+backward of the same workload in
    float32 (the fp32 gather + per-expert matmul CPU path; rounding points
    off), repeated until the time budget is spent (at least once)."""
    from oracle import cvmm_oracle as O
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    op = None
    xn = proj.x.float().numpy()
    kn = proj.keys.float().numpy()
    wn = None if proj.weights is None else proj.weights.float().numpy()
    gn = proj.grad_out.float().numpy()
    sel = proj.sel.numpy()
    n = 0
    t0 = time.perf_counter()
    while True:
        meta = O.prepare_sel2(sel, wn, route_input=proj.route_input)
        O.forward(xn, meta, kn, op, op, compute=np.float32)
        O.backward(xn, meta, kn, gn, op, compute=np.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    per = el / n
    return {"value": round(proj.flops / per / 1e12, 6), "unit": "TFLOP/s", "cores": int(threads),
            "kind": "port",
            "sample": f"full {proj.name} workload, {n} oracle sel+fwd+bwd iterations in {el:.1f}s "
                      f"(numpy float32, rounding points off), {per * 1e3:.1f} ms/iter"}


def load_traffic(kernel: str, workload: str):
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    return None


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


def ffn_times(steps: int = 10, warmup: int = 3):
    """The FFN stack of BASELINE.json configs[4] (16384 tokens, 2048 -> 512 ->
    2048, 128 experts, top-8, Zipf-skewed gate; benchmark_ffn_moe.py:89-98),
    forward + backward, two ways: written as the reference's callers write it
    (torch router lines, F.gelu around cvmm) and with the library's fused
    router and up projection + GELU."""
    s = W.c5_ffn_stack().to(torch.device("cuda"))
    params = [t.clone().requires_grad_(True) for t in (s.x, s.gate, s.w_up, s.w_down)]
    import cvmm_codex_amd as C

    def step(fwd):
        for t in params:
            t.grad = None
        out = fwd(s, C, *params)
        out.backward(s.grad_out)

    res = {"shape": {"tokens": 16384, "d_model": 2048, "hidden": 512, "experts": 128, "top_k": 8}}
    for name, fwd in (("composed", W.ffn_forward), ("fused", W.ffn_forward_fused)):
        for _ in range(warmup):
            step(fwd)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            step(fwd)
        b.record()
        b.synchronize()
        ms = a.elapsed_time(b) / steps
        res[name] = {"ms_per_step": round(ms, 4), "tflops": round(s.flops / (ms * 1e-3) / 1e12, 2)}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(W.PROJECTIONS))
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["fwd", "bwd_w", "bwd_x", "cast_keys", "copy"], default=None,
                    help="launch only this phase --steps times, or the copy calibration (rocprofv3 runs)")
    ap.add_argument("--ffn", action="store_true",
                    help="time the FFN stack (configs[4]) composed vs with the fused router and GELU (one JSON "
                         "line) and exit")
    ap.add_argument("--router", action="store_true",
                    help="time the fused router against the torch router lines (one JSON line) and exit")
    ap.add_argument("--tune", action="append", default=[], metavar="KNOB=VALUE",
                    help="set a library tuning knob (panel_tiles_per_wg, wgrad_order, wgrad_tile, gemm_order, "
                         "reduce_min_topk) before running")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard over experts, which is not built here)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    from cvmm_codex_amd import _native as N
    knobs = {"panel_tiles_per_wg": N.TUNE_PANEL_TILES_PER_WG, "wgrad_order": N.TUNE_WGRAD_ORDER,
             "gemm_order": N.TUNE_GEMM_ORDER, "reduce_min_topk": N.TUNE_REDUCE_MIN_TOPK,
             "wgrad_tile": N.TUNE_WGRAD_TILE}
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
    if args.ffn:
        print(json.dumps({"ffn": ffn_times()}), flush=True)
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
    ms = time_steps(runner, args.steps, args.warmup)
    log(f"step {ms:.4f} ms")
    phases = time_phases(runner, max(10, args.steps // 2))
    log(f"phases {phases}")

    kt = kernel_times(runner, args.kernel_iters)
    log("kernel ms/launch " + json.dumps({k: round(v["avg_ms"], 5) for k, v in kt.items()}))
    dtype = "bf16" if proj.amp else "fp32"
    peak = PEAK[dtype]
    # dominant kernel: the hot kernel class with the most device time per step
    dom = max((k for k in kt if kernel_work(proj, k)[0] is not None), key=lambda k: kt[k]["ms_per_step"])
    flops, nbytes = kernel_work(proj, dom)
    sec = kt[dom]["avg_ms"] * 1e-3
    t_mfma, t_hbm = flops / (peak * 1e12), nbytes / (HBM_PEAK_GBS * 1e9)
    if t_hbm >= t_mfma:
        roofline = {"bound": "hbm", "achieved": round(nbytes / sec / 1e9, 2), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 5)}
    else:
        roofline = {"bound": "mfma", "achieved": round(flops / sec / 1e12, 3), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(flops / sec / 1e12 / peak, 5)}
    roofline.update({"traffic": load_traffic(dom, proj.name), "kernel": dom,
                     "avg_launch_ms": round(kt[dom]["avg_ms"], 5), "algorithmic_bytes": int(nbytes),
                     "algorithmic_flops": flops})

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
                   "step": "sel+fwd+bwd", "gflop_per_step": round(proj.flops / 1e9, 3)},
        "step_roofline_frac": round(value / PEAK[dtype], 5),
        "breakdown_ms": {k: round(v, 5) for k, v in phases.items()},
        "kernel_ms_per_launch": {k: round(v["avg_ms"], 5) for k, v in kt.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
