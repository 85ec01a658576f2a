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
  mha_bwd   causal MHA backward with projection grads.  TFLOP/s.
  small_cnn configs[0] training step, batch 64 (fp32).  samples/s.
  resnet18  configs[4] training step, batch 64 (bf16 or fp32).  samples/s.

Besides `value`, the line carries `roofline` for the dominant kernel (its
algorithmic work per launch over its HIP-event-timed launch duration on the
launch stream) and `cpu_baseline`: the reference's own libtorch CPU path
(oracle/_ref, kind "reference") or the plain-C oracle (kind "port"), timed on
a bounded sample on this host's cores.  `extra` reports the other legs the
metric names: LayerNorm-backward, AdamW and CE-gradient bandwidth (fp32 and
bf16), conv backward in fp32, MHA backward, and the configs[0] / configs[4]
training steps in samples/s (with their own CPU baselines).
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


# HBM bytes per launch of the dominant kernel (all kernels of the bracketed
# entry point), from two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE,
# KiB per dispatch), each divided by what the same counter reads for a plain
# 256 MiB device copy (FETCH_SIZE reads 0.5 x the bytes, WRITE_SIZE 1.0 x).
# The passes and their commands are in profiles/.  Keyed by (workload, dtype,
# kernel); None where no pass has been recorded.
TRAFFIC = {
    ("conv_bwd", "bf16", "dgrad"): 183.36e6,   # conv3x3_wprep + conv3x3_same
    ("conv_bwd", "bf16", "wgrad"): 230.21e6,   # conv3x3_wgrad + conv3x3_wgrad_reduce
    ("ln_bwd", "f32", None): 210.93e6,         # ln_bwd_kernel + col_reduce_grouped_kernel
    ("ln_bwd", "bf16", None): 109.77e6,
    ("adamw", "f32", None): 2799.94e6,
    ("adamw", "bf16", None): 2200.00e6,
    ("xent", "f32", None): 4199.32e6,          # xent_count_kernel + xent_rows_vec_kernel
    ("xent", "bf16", None): 2101.43e6,
}


def traffic_for(workload, dtype, kernel):
    return TRAFFIC.get((workload, dtype, kernel))


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
        iters = max(1, min(20000, int(budget_s / max(sec, 1e-6))))
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


class TrainStep(Workload):
    """One full training step (forward, CE mean, backward, fused Adam/AdamW,
    zero_grad) through the C++ host layer: configs[0] small CNN (fp32, Adam)
    or configs[4] ResNet-18 (AdamW; fp32 or bf16 mixed precision), batch 64."""
    unit = "samples/s"
    bound = "mfma"
    BATCH = 64

    graph = True   # forward + loss + backward replayed from a captured HIP graph (AdamW eager)

    def __init__(self, dtype, model):
        self.dtype = dtype
        self.name = model

    def setup(self, torch, ops):
        import importlib
        host = importlib.import_module("thot_amd._nott_host")
        g = torch.Generator(device="cuda").manual_seed(4)
        if self.name == "small_cnn":
            self.tr = host.SmallCNNTrainer(0, 0, 1e-3)
            self.x = torch.rand((self.BATCH, 1, 28, 28), generator=g, device="cuda")
            self.y = torch.randint(0, 10, (self.BATCH,), generator=g, device="cuda")
            # forward 2*MACs: conv1 1*32*9*784, conv2 32*64*9*196, fc 3136*128 + 128*10; training ~ 3x forward
            self.flop_sample = 3 * 2.0 * (32 * 9 * 784 + 32 * 64 * 9 * 196 + 3136 * 128 + 128 * 10)
        else:
            self.tr = host.ResNet18Trainer(0, 0, self.dtype == "bf16", 1e-3, 1e-2, 1000)
            self.x = torch.rand((self.BATCH, 3, 224, 224), generator=g, device="cuda")
            self.y = torch.randint(0, 1000, (self.BATCH,), generator=g, device="cuda")
            self.flop_sample = 3 * 2 * 1.814e9   # ResNet-18 at 224^2: 1.814 GMAC forward
        self.tr.step(self.x, self.y)
        if self.graph:
            try:
                self.tr.capture(self.x, self.y, 2)
            except RuntimeError as e:   # reported in the JSON line via hip_graph = false
                print(f"bench: HIP graph capture failed, stepping eagerly: {e}", file=sys.stderr)
                self.graph = False

    def step(self):
        if self.graph:
            self.tr.step_graph(self.x, self.y)
        else:
            self.tr.step(self.x, self.y)

    def work_per_step(self):
        return self.BATCH

    def cpu_baseline(self, budget_s):
        from oracle_lib import Ref
        if not Ref.available():
            return None
        ref = Ref()
        ref.set_threads(host_cores())
        batch = 64 if self.name == "small_cnn" else 8
        sec = ref.train_step_time(self.name, batch, 1)
        iters = max(1, min(20000, int(budget_s / max(sec, 1e-6))))
        sec = ref.train_step_time(self.name, batch, iters)
        what = "configs[0] small CNN + Adam" if self.name == "small_cnn" else "configs[4] ResNet-18 + AdamW"
        return {"value": batch / sec, "unit": "samples/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"{what}, fp32 libtorch CPU step built from Nott's layer descriptors, batch {batch}, "
                          f"{iters} steps x {sec * 1e3:.1f} ms"}


class MhaBwd(Workload):
    """causal multi-head attention backward, bf16, B=8, H=16,
    T=1024, dh=64, with the projection-weight gradients of the 1024->3x1024
    input and 1024->1024 output projections.  One step: output-projection
    backward, attention backward, input-projection backward.  The attention
    reads q, k, v as token-major views of the packed [B·T, 3·E] projection
    output and dO as a view of the output projection's dX, and writes dq, dk,
    dv into the packed [B·T, 3·E] gradient the input projection consumes, so
    no head split or merge copies run.  Work: 34.36 GFLOP causal core (dV,
    dP, dQ, dK GEMMs) + 137.44 GFLOP projections."""
    name = "mha_bwd"
    unit = "TFLOP/s"
    bound = "mfma"
    B, H, T, DH = 8, 16, 1024, 64

    def __init__(self, dtype):
        self.dtype = dtype

    def setup(self, torch, ops):
        self.torch, self.ops = torch, ops
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float32
        B, H, T, DH = self.B, self.H, self.T, self.DH
        E = H * DH
        g = torch.Generator(device="cuda").manual_seed(5)
        self.x = torch.randn((B * T, E), generator=g, device="cuda").to(dt)
        self.w_in = (0.02 * torch.randn((3 * E, E), generator=g, device="cuda")).to(dt)
        self.w_out = (0.02 * torch.randn((E, E), generator=g, device="cuda")).to(dt)
        self.d = ops.attn_desc(B, H, T, T, DH, True, token_major=True, ld_qkv=3 * E)
        qkv = torch.randn((B, T, 3 * E), generator=g, device="cuda").to(dt)
        self.q, self.k, self.v = (qkv[:, :, i * E:(i + 1) * E].view(B, T, H, DH) for i in range(3))
        self.qkv = qkv
        self.o, self.lse = ops.attention_fwd(self.q, self.k, self.v, self.d)
        self.attn_out = self.o.view(B * T, E)
        self.dy = torch.randn((B * T, E), generator=g, device="cuda").to(dt)
        self.dqkv = torch.empty((B, T, 3 * E), dtype=dt, device="cuda")
        self.dqkv_views = tuple(self.dqkv[:, :, i * E:(i + 1) * E].view(B, T, H, DH) for i in range(3))
        self.dw_in = torch.empty((3 * E, E), device="cuda")
        self.db_in = torch.empty((3 * E,), device="cuda")
        self.dw_out = torch.empty((E, E), device="cuda")
        self.db_out = torch.empty((E,), device="cuda")
        self.core_flop = 4 * 2.0 * B * H * DH * (T * (T + 1) / 2)
        self.proj_flop = 2 * 2.0 * B * T * E * 3 * E + 2 * 2.0 * B * T * E * E
        self.ev_a = [None, None]

    def step(self):
        ops = self.ops
        B, H, T, DH = self.B, self.H, self.T, self.DH
        dattn, _, _ = ops.linear_bwd(self.dy, self.attn_out, self.w_out, dw=self.dw_out, db=self.db_out)
        dO = dattn.view(B, T, H, DH)
        if self.ev_a[0] is not None:
            self.ev_a[0].record()
        ops.attention_bwd(self.q, self.k, self.v, self.o, dO, self.lse, self.d, out=self.dqkv_views)
        if self.ev_a[1] is not None:
            self.ev_a[1].record()
        ops.linear_bwd(self.dqkv.view(B * T, 3 * H * DH), self.x, self.w_in, dw=self.dw_in, db=self.db_in)

    def work_per_step(self):
        return self.core_flop + self.proj_flop


WORKLOADS = {"conv_bwd": ConvBwd, "ln_bwd": LnBwd, "xent": Xent, "adamw": AdamW, "mha_bwd": MhaBwd,
             "small_cnn": lambda dt: TrainStep(dt, "small_cnn"), "resnet18": lambda dt: TrainStep(dt, "resnet18")}


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
    """Average duration of each bracketed launch group, from HIP events recorded
    on torch's current stream (the stream the C ABI launches on).  The steps
    are queued back to back with one synchronisation at the end, so a start
    event fires when the previous step's work drains, not when the host gets
    round to the next launch."""
    wl.step()
    pairs = []
    for _ in range(steps):
        step_pairs = {}
        for k in pairs_attr:
            step_pairs[k] = [torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
            getattr(wl, k)[0], getattr(wl, k)[1] = step_pairs[k]
        wl.step()
        pairs.append(step_pairs)
    torch.cuda.synchronize()
    out = {}
    for k in pairs_attr:
        getattr(wl, k)[0] = getattr(wl, k)[1] = None
        out[k] = sum(p[k][0].elapsed_time(p[k][1]) for p in pairs) / steps
    return out


def simple_kernel_ms(torch, wl, steps):
    """Event-timed average of one whole step (for one-entry-point workloads),
    steps queued back to back on the launch stream."""
    wl.step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        wl.step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


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
    ap.add_argument("--eager", action="store_true",
                    help="training-step workloads: run every step eagerly instead of replaying a captured HIP graph")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first run 3 plain 256 MiB device copies (the known-size kernel that calibrates "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
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
    if args.copy_probe:
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    dtype = args.dtype or ("f32" if args.workload in ("ln_bwd", "xent", "adamw", "small_cnn") else "bf16")
    TrainStep.graph = not args.eager
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
                "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": traffic_for("conv_bwd", dtype, dom), "traffic_unit": "B",
                "per_kernel_ms": {k: round(v, 4) for k, v in per.items()},
                "per_kernel_tflops": {k: round(wl.flop_one / (v * 1e-3) / 1e12, 2) for k, v in per.items()}}
        metric_part = "conv-bwd TFLOP/s"
        cfg = {"workload": "conv2d_bwd (BASELINE configs[1])", "n": wl.N, "c_in": wl.C, "c_out": wl.K,
               "hw": wl.H, "kernel": "3x3 s1 p1", "layout": "NCHW", "bias": False}
    elif args.workload == "mha_bwd":
        kms = kernel_ms(torch, wl, args.steps, ["ev_a"])["ev_a"]
        value = value_per_s / 1e12
        ach = wl.core_flop / (kms * 1e-3) / 1e12
        peak = MFMA_PEAK_TFLOPS[dtype]
        roof = {"bound": "mfma", "kernel": "attention_bwd (dq + dkdv)", "achieved": round(ach, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": None, "launch_ms": round(kms, 4)}
        metric_part = "MHA-bwd TFLOP/s"
        cfg = {"workload": "mha_bwd (BASELINE configs[3])", "b": wl.B, "heads": wl.H, "t": wl.T, "dh": wl.DH,
               "causal": True, "projections": "1024->3x1024 in, 1024->1024 out"}
    elif args.workload in ("small_cnn", "resnet18"):
        value = value_per_s
        ach = wl.flop_sample * value / 1e12
        peak = MFMA_PEAK_TFLOPS[dtype]
        roof = {"bound": "mfma", "kernel": "whole training step (model FLOPs, ~3x forward)", "achieved": round(ach, 2),
                "peak": peak, "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": None}
        metric_part = "train samples/s"
        cfg = {"workload": f"{wl.name} training step (BASELINE configs[{0 if wl.name == 'small_cnn' else 4}])",
               "batch": wl.BATCH, "optimizer": "Adam" if wl.name == "small_cnn" else "AdamW",
               "hip_graph": wl.graph}
    else:
        kms = simple_kernel_ms(torch, wl, args.steps)
        value = wl.work_per_step() / (ms * 1e-3) / 1e9
        ach = wl.work_per_step() / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": wl.name, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic_for(wl.name, dtype, None), "traffic_unit": "B",
                "launch_ms": round(kms, 4)}
        metric_part = {"ln_bwd": "LN-bwd GB/s", "xent": "CE-grad GB/s", "adamw": "AdamW GB/s"}[wl.name]
        cfg = {"workload": wl.name}

    extra = {}
    if not args.no_extra and args.workload == "conv_bwd":
        del wl.x, wl.dy, wl.dx
        torch.cuda.empty_cache()
        for nm, cls in (("ln_bwd", LnBwd), ("adamw", AdamW), ("xent", Xent)):
            for dt in ("f32", "bf16"):
                leg, lms, lk, gbs = run_bandwidth_leg(torch, ops, cls, dt, args.steps, args.warmup)
                extra[f"{nm}_{dt}"] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                       "kernel_ms": round(lk, 4)}
                del leg
                torch.cuda.empty_cache()
        leg = ConvBwd("f32")
        leg.setup(torch, ops)
        lms = time_workload(torch, leg, max(3, args.steps // 4), 1)
        extra["conv_bwd_f32"] = {"TFLOP/s": round(leg.work_per_step() / (lms * 1e-3) / 1e12, 2),
                                 "frac_mfma": round(leg.work_per_step() / (lms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f32"], 4)}
        del leg
        torch.cuda.empty_cache()
        leg = MhaBwd("bf16")
        leg.setup(torch, ops)
        lms = time_workload(torch, leg, args.steps, args.warmup)
        ams = kernel_ms(torch, leg, args.steps, ["ev_a"])["ev_a"]
        extra["mha_bwd_bf16"] = {"TFLOP/s": round(leg.work_per_step() / (lms * 1e-3) / 1e12, 2), "ms": round(lms, 4),
                                 "core_TFLOP/s": round(leg.core_flop / (ams * 1e-3) / 1e12, 2)}
        del leg
        torch.cuda.empty_cache()
        for model, dt in (("small_cnn", "f32"), ("resnet18", "bf16"), ("resnet18", "f32")):
            leg = TrainStep(dt, model)
            leg.setup(torch, ops)
            lms = time_workload(torch, leg, args.steps, args.warmup)
            rec = {"samples/s": round(leg.BATCH / (lms * 1e-3), 1), "ms_per_step": round(lms, 3), "hip_graph": leg.graph,
                   "batch": leg.BATCH}
            if not args.no_cpu and dt == "f32":
                try:
                    rec["cpu_baseline"] = leg.cpu_baseline(args.cpu_budget / 2)
                except Exception as e:
                    rec["cpu_baseline"] = {"error": repr(e)}
            extra[f"{model}_{dt}"] = rec
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
