#!/usr/bin/env python3
"""Benchmark of the Nott training-backward path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--dtype bf16|f32]

Prints ONE JSON line.  A "step" is one pass of the workload's hot path over
one batch of synthetic input already resident in HBM:

  conv_bwd  (default)  conv2d dgrad + wgrad, N=128,
            Cin=64, Cout=128, 56x56, 3x3 s1 p1, NCHW, no bias.  TFLOP/s.
            The headline is fp32 (the reference's arithmetic); the bf16 leg
            with its own roofline sits beside it in `legs`.
  ln_bwd    LayerNorm backward 16384x1024 (configs[2]a).  GB/s.
  xent      fused softmax-CE gradient 16384x32000 (configs[2]b).  GB/s.
  adamw     fused AdamW over a flat 1e8-parameter buffer (configs[2]c).  GB/s.
  mha_bwd   causal MHA backward with projection grads.  TFLOP/s.
  small_cnn configs[0] training step, batch 64 (fp32).  samples/s.
  resnet18  configs[4] training step, batch 64 (bf16 or fp32).  samples/s.

Every leg carries `roofline` for its dominant kernel (algorithmic work per
launch over the HIP-event-timed launch duration on the launch stream) and
`cpu_baseline`: the reference's own libtorch CPU path (oracle/_ref, kind
"reference") timed on a bounded sample on this host's cores.  The default
run (conv_bwd) reports every other BASELINE leg in `legs`.
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
# kernel group); None where no pass has been recorded.
TRAFFIC = {
    ("conv_bwd", "f32", "dgrad"): 446.25e6,    # conv3x3_wprep + conv3x3_same + conv3x3_split_reduce (tail tiles)
    ("conv_bwd", "f32", "wgrad"): 385.08e6,    # conv3x3_wgrad + conv3x3_wgrad_reduce
    ("conv_bwd", "bf16", "dgrad"): 182.82e6,
    ("conv_bwd", "bf16", "wgrad"): 230.20e6,
    ("ln_bwd", "f32", "all"): 206.31e6,        # ln_bwd_kernel + col_reduce_grouped_kernel
    ("ln_bwd", "bf16", "all"): 105.54e6,
    ("adamw", "f32", "all"): 2799.95e6,
    ("adamw", "bf16", "all"): 2200.00e6,
    ("xent", "f32", "all"): 4200.27e6,         # xent_count_kernel + xent_rows_vec_kernel
    ("xent", "bf16", "all"): 2101.67e6,
    ("mha_bwd", "bf16", "out_proj"): 194.04e6,   # dA GEMM + dW_o split GEMM + reduce
    ("mha_bwd", "bf16", "attention"): 241.85e6,  # attn_dq64 + attn_dkdv64
    ("mha_bwd", "bf16", "in_proj"): 480.57e6,    # dX GEMM + dW_qkv split GEMM + reduce
}


def host_info() -> dict:
    """What the CPU baselines ran on: logical CPUs, the CPUs this process may
    use, physical cores, the CPU model, and the thread count P used.  P is the
    CPUs this process may use, capped by OMP_NUM_THREADS where it is set (the
    GPU box's CPU share for one GPU is 16 and sets it to that)."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    model, phys, ident = None, set(), {}
    try:
        pid = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k in ("cpu family", "model", "stepping", "cache size", "cpu MHz") and k not in ident:
                    ident[k] = v
                elif k == "physical id":
                    pid = v
                elif k == "core id":
                    core = v
                elif not k and pid is not None:
                    phys.add((pid, core))
                    pid = core = None
        if pid is not None:
            phys.add((pid, core))
    except OSError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    p = aff if not (omp and omp.isdigit() and int(omp) > 0) else min(aff, int(omp))
    # /proc/cpuinfo's model name can be generic under virtualisation ("AMD
    # EPYC"); the family / model / stepping numbers and the cache identify the part.
    if model is not None and ident:
        model = (f"{model} (family {ident.get('cpu family', '?')}, model {ident.get('model', '?')}, "
                 f"stepping {ident.get('stepping', '?')}, cache {ident.get('cache size', '?')}, "
                 f"{ident.get('cpu MHz', '?')} MHz)")
    return {"nproc": os.cpu_count(), "affinity_cpus": aff, "physical_cores": len(phys) or None,
            "model": model, "threads": p, "omp_num_threads": omp}


def cpu_threads() -> int:
    return host_info()["threads"]


def _ref():
    from oracle_lib import Ref
    if not Ref.available():
        return None
    ref = Ref()
    ref.set_threads(cpu_threads())
    return ref


def _iters_for(sec_one: float, budget_s: float, cap: int = 20000) -> int:
    """Timed iterations for a CPU baseline: what fits the budget, at least 20
    (the reference's times are the median of these, after 5 warm-ups)."""
    return max(20, min(cap, int(budget_s / max(sec_one, 1e-6))))


# ----------------------------------------------------------------- workloads
class Workload:
    """A BASELINE leg.  `groups` names the launch groups bracketed by HIP
    events inside step(); `group_work` gives each group's algorithmic work per
    launch (FLOP or bytes); `dominant` is the group the roofline is quoted on."""
    name = ""
    unit = ""
    scale = 1.0          # value = work_per_step / seconds / scale
    bound = "hbm"
    dtype = "f32"
    groups = ("all",)

    def __init__(self, dtype):
        self.dtype = dtype
        self.ev = {}

    def mark(self, group, i):
        e = self.ev.get(group)
        if e is not None:
            e[i].record()

    def setup(self, torch, ops): ...

    def step(self): ...

    def work_per_step(self) -> float: ...

    def group_work(self) -> dict:
        return {"all": self.work_per_step()}

    def dominant(self, per_ms: dict) -> str:
        return max(per_ms, key=per_ms.get)

    def peak(self):
        return HBM_PEAK_GBS if self.bound == "hbm" else MFMA_PEAK_TFLOPS[self.dtype]

    def cpu_baseline(self, budget_s: float):
        return None

    def config(self) -> dict:
        return {"workload": self.name}


class ConvBwd(Workload):
    name = "conv_bwd"
    unit = "TFLOP/s"
    scale = 1e12
    bound = "mfma"
    groups = ("dgrad", "wgrad")
    N, C, K, H, W = 128, 64, 128, 56, 56

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

    def step(self):
        self.mark("dgrad", 0)
        self.ops.conv2d_bwd_data(self.dy, self.w, self.d, out=self.dx)
        self.mark("dgrad", 1)
        self.mark("wgrad", 0)
        self.ops.conv2d_bwd_weight(self.x, self.dy, self.d, dw=self.dw)
        self.mark("wgrad", 1)

    def work_per_step(self):
        return 2 * self.flop_one

    def group_work(self):
        return {"dgrad": self.flop_one, "wgrad": self.flop_one}

    def config(self):
        return {"workload": "conv2d_bwd (BASELINE configs[1])", "n": self.N, "c_in": self.C, "c_out": self.K,
                "hw": self.H, "kernel": "3x3 s1 p1", "layout": "NCHW", "bias": False}

    def cpu_baseline(self, budget_s):
        import numpy as np
        from oracle_lib import f32, rng
        ref = _ref()
        if ref is None:
            return None
        n = 8
        g = rng(0)
        d = self.ops.conv_desc((n, self.C, self.H, self.W), (self.K, self.C, 3, 3), padding=(1, 1))
        x = f32(g.standard_normal((n, self.C, self.H, self.W)))
        w = f32(g.standard_normal((self.K, self.C, 3, 3)) / math.sqrt(self.C * 9))
        dy = f32(g.standard_normal((n, self.K, self.H, self.W)))
        iters = _iters_for(ref.conv2d_bwd_time(d, x, w, dy, 1), budget_s)
        sec = ref.conv2d_bwd_time(d, x, w, dy, iters)
        flop = 2 * 2.0 * n * self.H * self.W * self.K * self.C * 9
        return {"value": round(flop / sec / 1e12, 4), "unit": "TFLOP/s", "cores": ref.get_threads(),
                "kind": "reference",
                "sample": f"Nott Conv2d (libtorch CPU autograd) dgrad+wgrad, fp32, N={n} of 128 "
                          f"(per-image work, scaled by FLOPs), median of {iters} passes after 5 warm-ups {sec * 1e3:.1f} ms"}


class LnBwd(Workload):
    name = "ln_bwd"
    unit = "GB/s"
    scale = 1e9
    R, D = 16384, 1024

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
        self.mark("all", 0)
        self.ops.layernorm_bwd(self.x, self.dy, self.mean, self.rstd, self.gamma, dgamma=self.dg, dbeta=self.db,
                               out=self.dx)
        self.mark("all", 1)

    def work_per_step(self):
        return self.bytes

    def config(self):
        return {"workload": "layernorm_bwd (BASELINE configs[2]a)", "rows": self.R, "d": self.D}

    def cpu_baseline(self, budget_s):
        ref = _ref()
        if ref is None:
            return None
        iters = _iters_for(ref.layernorm_bwd_time(self.R, self.D, 1), budget_s, 1000)
        sec = ref.layernorm_bwd_time(self.R, self.D, iters)
        b32 = 3 * self.R * self.D * 4 + self.D * 4 + 2 * self.R * 4 + 2 * self.D * 4
        return {"value": round(b32 / sec / 1e9, 2), "unit": "GB/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"at::native_layer_norm_backward (the op LayerNorm's autograd node runs), fp32, full "
                          f"{self.R}x{self.D}, median of {iters} calls after 5 warm-ups {sec * 1e3:.2f} ms; GB/s on the fp32 algorithmic "
                          f"bytes (the reference has no bf16 path)"}


class Xent(Workload):
    name = "xent"
    unit = "GB/s"
    scale = 1e9
    N, C = 16384, 32000

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
        self.mark("all", 0)
        self.ops.softmax_xent_bwd(self.z, self.y, out=self.dz, with_loss=False)
        self.mark("all", 1)

    def work_per_step(self):
        return self.bytes

    def config(self):
        return {"workload": "softmax_xent_grad (BASELINE configs[2]b)", "rows": self.N, "classes": self.C}

    def cpu_baseline(self, budget_s):
        ref = _ref()
        if ref is None:
            return None
        rows = 512
        iters = _iters_for(ref.cross_entropy_time(rows, self.C, 1), budget_s, 1000)
        sec = ref.cross_entropy_time(rows, self.C, iters)
        b32 = 2 * rows * self.C * 4 + rows * 8
        return {"value": round(b32 / sec / 1e9, 2), "unit": "GB/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"Nott CrossEntropy forward + backward (log_softmax + nll_loss, libtorch CPU autograd), "
                          f"fp32, {rows} of {self.N} rows x {self.C}, median of {iters} passes after 5 warm-ups {sec * 1e3:.2f} ms; GB/s on "
                          f"the fp32 algorithmic bytes of those rows"}


class AdamW(Workload):
    name = "adamw"
    unit = "GB/s"
    scale = 1e9
    NP = 100_000_000

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
        self.mark("all", 0)
        self.ops.adam_step(self.p, self.g, self.m, self.v, lr=3e-4, weight_decay=0.01, step=10, decoupled=True)
        self.mark("all", 1)

    def work_per_step(self):
        return self.bytes

    def config(self):
        return {"workload": "adamw_flat (BASELINE configs[2]c)", "params": self.NP, "step": 10}

    def cpu_baseline(self, budget_s):
        ref = _ref()
        if ref is None:
            return None
        n = 10_000_000
        iters = _iters_for(ref.adamw_time(n, 1), budget_s, 200)
        sec = ref.adamw_time(n, iters)
        return {"value": round(n * 28 / sec / 1e9, 2), "unit": "GB/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"Nott AdamW (torch::optim CPU) on a flat 1e7-param fp32 buffer, median of "
                          f"{iters} steps after 5 warm-ups {sec * 1e3:.1f} ms"}


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
    scale = 1e12
    bound = "mfma"
    groups = ("out_proj", "attention", "in_proj")
    B, H, T, DH = 8, 16, 1024, 64

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
        self.dattn = torch.empty((B * T, E), dtype=dt, device="cuda")
        self.dqkv = torch.empty((B, T, 3 * E), dtype=dt, device="cuda")
        self.dqkv_views = tuple(self.dqkv[:, :, i * E:(i + 1) * E].view(B, T, H, DH) for i in range(3))
        self.dx = torch.empty((B * T, E), dtype=dt, device="cuda")
        self.dw_in = torch.empty((3 * E, E), device="cuda")
        self.db_in = torch.empty((3 * E,), device="cuda")
        self.dw_out = torch.empty((E, E), device="cuda")
        self.db_out = torch.empty((E,), device="cuda")
        self.core_flop = 4 * 2.0 * B * H * DH * (T * (T + 1) / 2)
        self.out_flop = 2 * 2.0 * B * T * E * E
        self.in_flop = 2 * 2.0 * B * T * E * 3 * E

    def step(self):
        ops = self.ops
        B, H, T, DH = self.B, self.H, self.T, self.DH
        self.mark("out_proj", 0)
        ops.linear_bwd(self.dy, self.attn_out, self.w_out, dx=self.dattn, dw=self.dw_out, db=self.db_out)
        self.mark("out_proj", 1)
        dO = self.dattn.view(B, T, H, DH)
        self.mark("attention", 0)
        ops.attention_bwd(self.q, self.k, self.v, self.o, dO, self.lse, self.d, out=self.dqkv_views)
        self.mark("attention", 1)
        self.mark("in_proj", 0)
        ops.linear_bwd(self.dqkv.view(B * T, 3 * H * DH), self.x, self.w_in, dx=self.dx, dw=self.dw_in,
                       db=self.db_in)
        self.mark("in_proj", 1)

    def work_per_step(self):
        return self.core_flop + self.out_flop + self.in_flop

    def group_work(self):
        return {"out_proj": self.out_flop, "attention": self.core_flop, "in_proj": self.in_flop}

    def config(self):
        return {"workload": "mha_bwd (BASELINE configs[3])", "b": self.B, "heads": self.H, "t": self.T,
                "dh": self.DH, "causal": True, "projections": "1024->3x1024 in, 1024->1024 out"}

    def cpu_baseline(self, budget_s):
        ref = _ref()
        if ref is None:
            return None
        b = 1
        E = self.H * self.DH
        iters = _iters_for(ref.mha_bwd_time(b, self.T, E, self.H, True, 1), budget_s, 200)
        sec = ref.mha_bwd_time(b, self.T, E, self.H, True, iters)
        flop = self.work_per_step() * b / self.B
        return {"value": round(flop / sec / 1e12, 4), "unit": "TFLOP/s", "cores": ref.get_threads(),
                "kind": "reference",
                "sample": f"Nott MultiHeadAttention backward (libtorch CPU autograd through the saved graph), fp32, "
                          f"batch {b} of {self.B}, median of {iters} passes after 5 warm-ups {sec * 1e3:.1f} ms; TFLOP/s on the same "
                          f"algorithmic FLOPs per sample"}


class TrainStep(Workload):
    """One full training step (forward, CE mean, backward, fused Adam/AdamW,
    zero_grad) through the C++ host layer: configs[0] small CNN (fp32, Adam)
    or configs[4] ResNet-18 (AdamW; fp32 or bf16 mixed precision), batch 64."""
    unit = "samples/s"
    bound = "mfma"
    BATCH = 64
    groups = ()

    graph = True   # forward + loss + backward + AdamW replayed from a captured HIP graph

    def __init__(self, dtype, model):
        super().__init__(dtype)
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
            self.flop_sample = 681.5e9 / 64   # 3 x 1.814 GMAC forward - stem dgrad, per image
        self.tr.step(self.x, self.y)
        self.mode_ms = None
        if self.graph:
            try:
                self.tr.capture(self.x, self.y, 2)
            except RuntimeError as e:   # reported in the JSON line via hip_graph = false
                print(f"bench: HIP graph capture failed, stepping eagerly: {e}", file=sys.stderr)
                self.graph = False
        if self.graph:
            # The replayed graph and the eager step do the same work (the
            # graph adds the two input copies); which is faster depends on
            # the model: the eager launches overlap the weight-gradient side
            # stream better than the replayed branches, a small model's
            # launch overhead favours the graph.  Both are timed here, the
            # faster one is the timed step, and both rates go in the line.
            def ms(fn, n=8):
                for _ in range(2):
                    fn()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(n):
                    fn()
                torch.cuda.synchronize()
                return (time.perf_counter() - t0) * 1e3 / n
            g_ms = ms(lambda: self.tr.step_graph(self.x, self.y))
            e_ms = ms(lambda: self.tr.step(self.x, self.y))
            self.mode_ms = {"graph": round(g_ms, 4), "eager": round(e_ms, 4)}
            self.graph = g_ms <= e_ms

    def step(self):
        if self.graph:
            self.tr.step_graph(self.x, self.y)
        else:
            self.tr.step(self.x, self.y)

    def work_per_step(self):
        return self.BATCH

    def config(self):
        c = {"workload": f"{self.name} training step (BASELINE configs[{0 if self.name == 'small_cnn' else 4}])",
             "batch": self.BATCH, "optimizer": "Adam" if self.name == "small_cnn" else "AdamW",
             "hip_graph": self.graph}
        if self.mode_ms:
            c["setup_ms_per_step"] = self.mode_ms   # both modes, timed at setup; the faster is the timed step
        return c

    def cpu_baseline(self, budget_s):
        ref = _ref()
        if ref is None:
            return None
        batch = 64   # the GPU leg's batch
        # A ResNet-18 CPU step at batch 64 takes about a second: the minimum
        # 20 timed steps, without a probe.
        iters = 20 if self.name == "resnet18" else _iters_for(ref.train_step_time(self.name, batch, 1), budget_s)
        sec = ref.train_step_time(self.name, batch, iters)
        what = "configs[0] small CNN + Adam" if self.name == "small_cnn" else "configs[4] ResNet-18 + AdamW"
        note = "" if self.dtype == "f32" else " (the reference has no bf16 path: its fp32 step)"
        return {"value": round(batch / sec, 2), "unit": "samples/s", "cores": ref.get_threads(), "kind": "reference",
                "sample": f"{what}, fp32 libtorch CPU step built from Nott's layer descriptors{note}, batch {batch}, "
                          f"median of {iters} steps after 5 warm-ups {sec * 1e3:.1f} ms"}


WORKLOADS = {"conv_bwd": ConvBwd, "ln_bwd": LnBwd, "xent": Xent, "adamw": AdamW, "mha_bwd": MhaBwd,
             "small_cnn": lambda dt: TrainStep(dt, "small_cnn"), "resnet18": lambda dt: TrainStep(dt, "resnet18")}
DEFAULT_DTYPE = {"conv_bwd": "f32", "ln_bwd": "f32", "xent": "f32", "adamw": "f32", "mha_bwd": "bf16",
                 "small_cnn": "f32", "resnet18": "bf16"}


def time_workload(torch, wl, steps, warmup):
    """Wall-clock ms per step over `steps` timed steps, synchronised on both sides."""
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def group_ms(torch, wl, steps):
    """Average duration of each bracketed launch group, from HIP events recorded
    on torch's current stream (the stream the C ABI launches on).  The steps
    are queued back to back with one synchronisation at the end, so a start
    event fires when the previous work drains, not when the host gets round
    to the next launch."""
    if not wl.groups:
        return {}
    wl.step()
    if len(wl.groups) == 1:
        # One launch group per step: the steps are captured once into a HIP
        # graph and the replay is timed with one event pair, so the launches
        # run back to back as on the device (a short kernel launched eagerly
        # from Python can leave the GPU waiting for the host between steps).
        # Falls back to eager back-to-back launches if capture is refused.
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        try:
            graph = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                wl.step()
                torch.cuda.synchronize()
                with torch.cuda.graph(graph, stream=side):
                    for _ in range(steps):
                        wl.step()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            wl.graph_timed = True
        except RuntimeError:
            torch.cuda.synchronize()
            e0.record()
            for _ in range(steps):
                wl.step()
            e1.record()
            torch.cuda.synchronize()
            wl.graph_timed = False
        return {wl.groups[0]: e0.elapsed_time(e1) / steps}
    pairs = []
    for _ in range(steps):
        wl.ev = {k: [torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)] for k in wl.groups}
        wl.step()
        pairs.append(wl.ev)
    torch.cuda.synchronize()
    wl.ev = {}
    return {k: sum(p[k][0].elapsed_time(p[k][1]) for p in pairs) / steps for k in wl.groups}


def measure(torch, ops, wl, steps, warmup):
    """One leg on the GPU: value from wall-clock steps, roofline from
    event-timed groups."""
    wl.setup(torch, ops)
    ms = time_workload(torch, wl, steps, warmup)
    rec = {"value": round(wl.work_per_step() / (ms * 1e-3) / wl.scale, 3), "unit": wl.unit, "dtype": wl.dtype,
           "ms_per_step": round(ms, 4), "config": wl.config()}
    per = group_ms(torch, wl, steps)
    if per:
        work = wl.group_work()
        dom = wl.dominant(per)
        peak = wl.peak()
        unit = "GB/s" if wl.bound == "hbm" else "TFLOP/s"
        div = 1e9 if wl.bound == "hbm" else 1e12
        ach = work[dom] / (per[dom] * 1e-3) / div
        rec["roofline"] = {"bound": wl.bound, "kernel": f"{wl.name}:{dom}", "achieved": round(ach, 2), "peak": peak,
                           "timing": ("HIP graph replay of the timed steps" if getattr(wl, "graph_timed", False)
                                      else "HIP events around each launch group, steps queued back to back"),
                           "unit": unit, "frac": round(ach / peak, 4),
                           "traffic": TRAFFIC.get((wl.name, wl.dtype, dom)), "traffic_unit": "B",
                           "per_group_ms": {k: round(v, 4) for k, v in per.items()},
                           "per_group_rate": {k: round(work[k] / (v * 1e-3) / div, 2) for k, v in per.items()}}
    else:   # whole training steps: model FLOPs over the step
        ach = wl.flop_sample * (wl.BATCH / (ms * 1e-3)) / 1e12
        peak = wl.peak()
        rec["roofline"] = {"bound": "mfma", "kernel": f"{wl.name}: whole training step (model FLOPs)",
                           "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                           "traffic": None}
    return rec


def cpu_part(wl, budget):
    """The reference's CPU path on a bounded sample of the leg's workload."""
    try:
        return wl.cpu_baseline(budget)
    except Exception as e:  # reported, never fatal for the GPU measurement
        return {"error": repr(e)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="conv_bwd", choices=sorted(WORKLOADS))
    ap.add_argument("--dtype", default=None, choices=["bf16", "f32"])
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU work for the headline cpu_baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline leg only")
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

    TrainStep.graph = not args.eager
    dtype = args.dtype or DEFAULT_DTYPE[args.workload]
    cpu_budget = 0.0 if args.no_cpu else args.cpu_budget
    # Every GPU measurement runs before any CPU baseline: the baselines'
    # worker threads keep spinning for a while after they finish, which slows
    # the host launches of a GPU leg that follows.
    head_wl = WORKLOADS[args.workload](dtype)
    head = measure(torch, ops, head_wl, args.steps, args.warmup)

    legs = {}
    kept = []
    if not args.no_extra and args.workload == "conv_bwd":
        # The training steps run right after the conv legs: their eager
        # steps issue ~300 launches each and are the legs most sensitive to
        # host-side state left behind by the multi-GB element-wise legs.
        plan = [("conv_bwd", "bf16" if dtype == "f32" else "f32"), ("small_cnn", "f32"), ("resnet18", "bf16"),
                ("resnet18", "f32"), ("ln_bwd", "f32"), ("ln_bwd", "bf16"), ("adamw", "f32"), ("adamw", "bf16"),
                ("xent", "f32"), ("xent", "bf16"), ("mha_bwd", "bf16")]
        for name, dt in plan:
            wl = WORKLOADS[name](dt)
            legs[f"{name}_{dt}"] = measure(torch, ops, wl, args.steps, args.warmup)
            kept.append((name, dt, wl))
            torch.cuda.empty_cache()
    if cpu_budget > 0:
        head["cpu_baseline"] = cpu_part(head_wl, cpu_budget)
        leg_budget = max(1.0, args.cpu_budget / 3)
        cpu_done = {}
        for name, dt, wl in kept:
            # One CPU baseline per workload (the reference computes in fp32 only).
            if name not in cpu_done:
                cpu_done[name] = cpu_part(wl, leg_budget)
            legs[f"{name}_{dt}"]["cpu_baseline"] = cpu_done[name]

    metric_part = {"conv_bwd": "conv-bwd TFLOP/s", "ln_bwd": "LN-bwd GB/s", "xent": "CE-grad GB/s",
                   "adamw": "AdamW GB/s", "mha_bwd": "MHA-bwd TFLOP/s", "small_cnn": "train samples/s",
                   "resnet18": "train samples/s"}[args.workload]
    line = {
        "metric": f"{metric_part} (of: {METRIC})",
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded torch generator on device; inputs resident in HBM)",
        "config": head["config"],
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "host": host_info(),
    }
    if legs:
        line["legs"] = legs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
