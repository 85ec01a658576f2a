#!/usr/bin/env python3
"""Benchmark of the Nott training-backward path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--dtype bf16|f32]

Prints ONE JSON line.  A "step" is one pass of the workload's hot path over
one batch of synthetic input already resident in HBM:

  conv_bwd  (default)  conv2d dgrad + wgrad, N=128,
            Cin=64, Cout=128, 56x56, 3x3 s1 p1, NCHW, no bias.  TFLOP/s.
  ln_bwd    LayerNorm backward 16384x1024 (configs[2]a).  GB/s.
  xent      fused softmax-CE gradient 16384x32000 (configs[2]b).  GB/s.
  adamw     fused AdamW over a flat 1e8-parameter buffer (configs[2]c).  GB/s.

Besides `value`, the line carries `roofline` for the dominant kernel (its
algorithmic work per launch over its HIP-event-timed launch duration on the
launch stream) and `cpu_baseline`: the reference's own libtorch CPU path
(oracle/_ref, kind "reference") or the plain-C oracle (kind "port"), timed on
a bounded sample on this host's cores.  `extra` reports the LayerNorm-backward
and AdamW bandwidth legs that BASELINE's metric also names.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}
METRIC = "train samples/s; conv-bwd TFLOP/s (%MFMA peak); LN-bwd+AdamW GB/s (%HBM)"


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


# ----------------------------------------------------------------- workloads
class Workload:
    name = ""
    unit = ""
    bound = "hbm"
    dtype = "f32"

    def setup(self, torch, ops): ...

    def step(self):
        """Runs one pass; returns nothing.  The dominant kernel's launches are
        bracketed by self.ev0 / self.ev1 when they are set."""

    def work_per_step(self) -> float:
        """Algorithmic FLOPs or bytes of one step (the unit of `value`)."""

    def dominant(self):
        """(name, algorithmic work per launch)."""

    def cpu_baseline(self, budget_s: float):
        return None


def _timed(wl, fn):
    if wl.ev0 is not None:
        wl.ev0.record()
    fn()
    if wl.ev1 is not None:
        wl.ev1.record()


class ConvBwd(Workload):
    name = "conv_bwd"
    unit = "TFLOP/s"
    bound = "mfma"
    N, C, K, H, W = 128, 64, 128, 56, 56

    def __init__(self, dtype):
        self.dtype = dtype

    def setup(self, torch, ops):
        self.ops = ops
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float32
        g = torch.Generator(device="cuda").manual_seed(0)
        self.d = ops.conv_desc((self.N, self.C, self.H, self.W), (self.K, self.C, 3, 3), padding=(1, 1))
        self.x = torch.randn((self.N, self.C, self.H, self.W), generator=g, device="cuda").to(dt)
        self.w = (torch.randn((self.K, self.C, 3, 3), generator=g, device="cuda") / math.sqrt(self.C * 9)).to(dt)
        self.dy = torch.randn((self.N, self.K, self.H, self.W), generator=g, device="cuda").to(dt)
        self.dx = torch.empty_like(self.x)
        self.dw = torch.empty((self.K, self.C, 3, 3), dtype=torch.float32, device="cuda")
        self.flop_one = 2.0 * self.N * self.H * self.W * self.K * self.C * 9
        self.ev_d = [None, None]
        self.ev_w = [None, None]

    def step(self):
        ops = self.ops
        if self.ev_d[0] is not None:
            self.ev_d[0].record()
        ops.conv2d_bwd_data(self.dy, self.w, self.d, out=self.dx)
        if self.ev_d[1] is not None:
            self.ev_d[1].record()
            self.ev_w[0].record()
        ops.conv2d_bwd_weight(self.x, self.dy, self.d, dw=self.dw)
        if self.ev_w[1] is not None:
            self.ev_w[1].record()

    def work_per_step(self):
        return 2 * self.flop_one

    def cpu_baseline(self, budget_s):
        from oracle_lib import Ref, f32, rng
        import numpy as np
        if not Ref.available():
            return None
        ref = Ref()
        cores = host_cores()
        ref.set_threads(cores)
        n = 8
        g = rng(0)
        d = self.ops.conv_desc((n, self.C, self.H, self.W), (self.K, self.C, 3, 3), padding=(1, 1))
        x = f32(g.standard_normal((n, self.C, self.H, self.W)))
        w = f32(g.standard_normal((self.K, self.C, 3, 3)) / math.sqrt(self.C * 9))
        dy = f32(g.standard_normal((n, self.K, self.H, self.W)))
        sec = ref.conv2d_bwd_time(d, x, w, dy, 1)
        iters = max(1, min(50, int(budget_s / max(sec, 1e-6))))
        sec = ref.conv2d_bwd_time(d, x, w, dy, iters)
        flop = 2 * 2.0 * n * self.H * self.W * self.K * self.C * 9
        return {"value": flop / sec / 1e12, "unit": "TFLOP/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"Nott Conv2d (libtorch CPU autograd) dgrad+wgrad at N={n} of 128, fp32, "
                          f"{iters} passes x {sec * 1e3:.1f} ms"}


class LnBwd(Workload):
    name = "ln_bwd"
    unit = "GB/s"
    R, D = 16384, 1024

    def __init__(self, dtype):
        self.dtype = dtype

    def setup(self, torch, ops):
        self.ops = ops
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float32
        g = torch.Generator(device="cuda").manual_seed(1)
        self.x = torch.randn((self.R, self.D), generator=g, device="cuda").to(dt)
        self.gamma = (1 + 0.1 * torch.randn(self.D, generator=g, device="cuda")).to(dt)
        beta = torch.zeros(self.D, device="cuda").to(dt)
        self.dy = torch.randn((self.R, self.D), generator=g, device="cuda").to(dt)
        _, self.mean, self.rstd = ops.layernorm_fwd(self.x, self.gamma, beta)
        self.dx = torch.empty_like(self.x)
        self.dg = torch.empty(self.D, device="cuda")
        self.db = torch.empty(self.D, device="cuda")
        s = 2 if self.dtype == "bf16" else 4
        self.bytes = 3 * self.R * self.D * s + self.D * s + 2 * self.R * 4 + 2 * self.D * 4

    def step(self):
        self.ops.layernorm_bwd(self.x, self.dy, self.mean, self.rstd, self.gamma, dgamma=self.dg, dbeta=self.db,
                               out=self.dx)

    def work_per_step(self):
        return self.bytes

    def cpu_baseline(self, budget_s):
        return None


class Xent(Workload):
    name = "xent"
    unit = "GB/s"
    N, C = 16384, 32000

    def __init__(self, dtype):
        self.dtype = dtype

    def setup(self, torch, ops):
        self.ops = ops
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float32
        g = torch.Generator(device="cuda").manual_seed(2)
        self.z = (2 * torch.randn((self.N, self.C), generator=g, device="cuda")).to(dt)
        self.y = torch.randint(0, self.C, (self.N,), generator=g, device="cuda")
        self.dz = torch.empty_like(self.z)
        s = 2 if self.dtype == "bf16" else 4
        self.bytes = 2 * self.N * self.C * s + self.N * 8

    def step(self):
        self.ops.softmax_xent_bwd(self.z, self.y, out=self.dz, with_loss=False)

    def work_per_step(self):
        return self.bytes


class AdamW(Workload):
    name = "adamw"
    unit = "GB/s"
    NP = 100_000_000

    def __init__(self, dtype):
        self.dtype = dtype

    def setup(self, torch, ops):
        self.ops = ops
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float32
        g = torch.Generator(device="cuda").manual_seed(3)
        self.p = (0.02 * torch.randn(self.NP, generator=g, device="cuda")).to(dt)
        self.g = (1e-3 * torch.randn(self.NP, generator=g, device="cuda")).to(dt)
        self.m = torch.zeros(self.NP, device="cuda")
        self.v = torch.zeros(self.NP, device="cuda")
        self.bytes = self.NP * (22 if self.dtype == "bf16" else 28)

    def step(self):
        self.ops.adam_step(self.p, self.g, self.m, self.v, lr=3e-4, weight_decay=0.01, step=10, decoupled=True)

    def work_per_step(self):
        return self.bytes

    def cpu_baseline(self, budget_s):
        from oracle_lib import Ref
        if not Ref.available():
            return None
        ref = Ref()
        ref.set_threads(host_cores())
        n = 10_000_000
        sec = ref.adamw_time(n, 1)
        iters = max(1, min(100, int(budget_s / max(sec, 1e-6))))
        sec = ref.adamw_time(n, iters)
        return {"value": n * 28 / sec / 1e9, "unit": "GB/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"Nott AdamW (torch::optim CPU) on a flat 1e7-param fp32 buffer, {iters} steps x "
                          f"{sec * 1e3:.1f} ms"}


WORKLOADS = {"conv_bwd": ConvBwd, "ln_bwd": LnBwd, "xent": Xent, "adamw": AdamW}


def time_workload(torch, wl, steps, warmup):
    """Wall-clock ms per step over `steps` timed steps, synchronised on both sides."""
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return ms


def kernel_ms(torch, wl, steps, pairs_attr):
    """Average duration of one launch group, from HIP events on torch's current
    stream (the stream the C ABI launches on)."""
    out = {}
    totals = {k: 0.0 for k in pairs_attr}
    for _ in range(steps):
        pairs = {}
        for k in pairs_attr:
            pairs[k] = [torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
            getattr(wl, k)[0], getattr(wl, k)[1] = pairs[k]
        wl.step()
        torch.cuda.synchronize()
        for k in pairs_attr:
            totals[k] += pairs[k][0].elapsed_time(pairs[k][1])
    for k in pairs_attr:
        getattr(wl, k)[0] = getattr(wl, k)[1] = None
        out[k] = totals[k] / steps
    return out


def simple_kernel_ms(torch, wl, steps):
    """Event-timed average of one whole step (for one-entry-point workloads)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    tot = 0.0
    for _ in range(steps):
        e0.record()
        wl.step()
        e1.record()
        torch.cuda.synchronize()
        tot += e0.elapsed_time(e1)
    return tot / steps


def run_bandwidth_leg(torch, ops, cls, dtype, steps, warmup):
    wl = cls(dtype)
    wl.setup(torch, ops)
    ms = time_workload(torch, wl, steps, warmup)
    kms = simple_kernel_ms(torch, wl, steps)
    gbs = wl.work_per_step() / (kms * 1e-3) / 1e9
    return wl, ms, kms, gbs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="conv_bwd", choices=sorted(WORKLOADS))
    ap.add_argument("--dtype", default=None, choices=["bf16", "f32"])
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU work for cpu_baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (collectives, sharding and "
              "rank code are out of scope); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from thot_amd import ops
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    sys.path.insert(0, os.path.join(REPO, "tests"))

    dtype = args.dtype or ("bf16" if args.workload == "conv_bwd" else "f32")
    wl = WORKLOADS[args.workload](dtype)
    wl.setup(torch, ops)
    wl.ev0 = wl.ev1 = None
    ms = time_workload(torch, wl, args.steps, args.warmup)
    value_per_s = wl.work_per_step() / (ms * 1e-3)

    if args.workload == "conv_bwd":
        kms = kernel_ms(torch, wl, args.steps, ["ev_d", "ev_w"])
        value = value_per_s / 1e12
        per = {"dgrad": kms["ev_d"], "wgrad": kms["ev_w"]}
        dom = max(per, key=per.get)
        ach = wl.flop_one / (per[dom] * 1e-3) / 1e12
        peak = MFMA_PEAK_TFLOPS[dtype]
        roof = {"bound": "mfma", "kernel": f"conv2d_{dom}", "achieved": round(ach, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": None,
                "per_kernel_ms": {k: round(v, 4) for k, v in per.items()},
                "per_kernel_tflops": {k: round(wl.flop_one / (v * 1e-3) / 1e12, 2) for k, v in per.items()}}
        metric_part = "conv-bwd TFLOP/s"
        cfg = {"workload": "conv2d_bwd (BASELINE configs[1])", "n": wl.N, "c_in": wl.C, "c_out": wl.K,
               "hw": wl.H, "kernel": "3x3 s1 p1", "layout": "NCHW", "bias": False}
    else:
        kms = simple_kernel_ms(torch, wl, args.steps)
        value = wl.work_per_step() / (ms * 1e-3) / 1e9
        ach = wl.work_per_step() / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": wl.name, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "launch_ms": round(kms, 4)}
        metric_part = {"ln_bwd": "LN-bwd GB/s", "xent": "CE-grad GB/s", "adamw": "AdamW GB/s"}[wl.name]
        cfg = {"workload": wl.name}

    extra = {}
    if not args.no_extra and args.workload == "conv_bwd":
        for nm, cls in (("ln_bwd", LnBwd), ("adamw", AdamW)):
            for dt in ("f32", "bf16"):
                leg, lms, lk, gbs = run_bandwidth_leg(torch, ops, cls, dt, args.steps, args.warmup)
                extra[f"{nm}_{dt}"] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                       "kernel_ms": round(lk, 4)}
                del leg
                torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        try:
            cpu = wl.cpu_baseline(args.cpu_budget)
        except Exception as e:  # reported, never fatal for the GPU measurement
            cpu = {"error": repr(e)}

    line = {
        "metric": f"{metric_part} (of: {METRIC})",
        "value": round(value, 3),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded torch generator on device; inputs resident in HBM)",
        "config": cfg,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    if extra:
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
