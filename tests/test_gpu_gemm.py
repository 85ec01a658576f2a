"""GPU parity of the MFMA kernels (Linear and Conv2d forward / dgrad / wgrad)
against the CPU oracle, through the C ABI.  Same seeded inputs on both sides;
bf16 inputs are rounded once and the oracle sees the rounded values.

Shapes: the reference's golden conv cases (every stride / padding / dilation
variant on the path), the small-CNN and ResNet-18
layer shapes at reduced batch, and the standalone conv at full
size through size-independent checks (per-image slices against the oracle,
adjoint identities) plus a torch fp32 reference."""
import math
import os

import numpy as np
import pytest
import torch

from gpu_util import check, dev, host, host_input
from oracle_lib import conv_out, f32, rng

pytestmark = pytest.mark.gpu

DTYPES = ["f32", "bf16"]
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ops():
    from thot_amd import ops as _ops
    assert torch.cuda.is_available()
    return _ops


# ------------------------------------------------------------------ linear
LIN = [(1, 1, 1), (7, 5, 3), (64, 3136, 128), (64, 128, 10), (64, 512, 1000), (129, 70, 33), (256, 1024, 1024),
       # bf16 fast-path shapes: partial 128-tiles, split-K over 4096 rows
       (384, 192, 256), (136, 64, 64), (4096, 64, 64), (1024, 320, 192),
       # 64x64-tile grids (run_small): forward split over 16 stages with a
       # partial last stage; dW split over 2000 rows, ragged tiles
       (33, 1000, 17), (2000, 40, 24)]


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("m,kin,nout", LIN)
def test_linear(ops, oracle, dt, m, kin, nout):
    g = rng(11 + m + kin + nout)
    x = host_input(g.standard_normal((m, kin)), dt)
    w = host_input(g.standard_normal((nout, kin)) / math.sqrt(kin), dt)
    b = f32(g.standard_normal(nout) * 0.1)
    dy = host_input(g.standard_normal((m, nout)), dt)
    y = ops.linear_fwd(dev(x, dt), dev(w, dt), dev(b))
    dx, dw, db = ops.linear_bwd(dev(dy, dt), dev(x, dt), dev(w, dt))
    torch.cuda.synchronize()
    check(host(y), oracle.linear_fwd(x, w, b), dt, "linear y")
    rdx, rdw, rdb = oracle.linear_bwd(dy, x, w)
    check(host(dx), rdx, dt, "linear dx")
    check(host(dw), rdw, "f32" if dt == "f32" else dt, "linear dw")
    check(host(db), rdb, "f32" if dt == "f32" else dt, "linear db")


# bf16 shapes chosen for the direct-to-LDS GEMM's tile plans, each with
# partial tiles: (4104, 192, 2056) forward on 256x128 tiles; (2048, 1288,
# 1544) dW on 256x256 tiles split over K with the fused bias gradient;
# (1024, 200, 320) dX on unsplit 128x128 and dW split 4 ways; (256, 384, 256)
# dW unsplit over three tile columns (the bias gradient is summed once);
# (4100, 2048, 4104) forward on unsplit 256x256 tiles (17 x 17, K = 2048).
DMA_LIN = [(4104, 192, 2056), (2048, 1288, 1544), (1024, 200, 320), (256, 384, 256), (4100, 2048, 4104)]


def _edge(idx, n):
    return np.unique(np.clip(np.asarray(idx), 0, n - 1))


@pytest.mark.parametrize("accumulate", [False, True], ids=["set", "accumulate"])
@pytest.mark.parametrize("m,kin,nout", DMA_LIN)
def test_linear_bf16_tile_shapes(ops, oracle, m, kin, nout, accumulate):
    """Rows of y and dx, and output rows of dw and db (sums over every
    token), at the tile edges, against the oracle; accumulate adds into
    existing fp32 gradients."""
    dt = "bf16"
    g = rng(5 + m + kin + nout)
    x = host_input(g.standard_normal((m, kin)), dt)
    w = host_input(g.standard_normal((nout, kin)) / math.sqrt(kin), dt)
    b = f32(g.standard_normal(nout) * 0.1)
    dy = host_input(g.standard_normal((m, nout)), dt)
    xd, wd, dyd = dev(x, dt), dev(w, dt), dev(dy, dt)
    dw0 = f32(g.standard_normal((nout, kin))) if accumulate else np.zeros((nout, kin), np.float32)
    db0 = f32(g.standard_normal(nout)) if accumulate else np.zeros(nout, np.float32)
    y = ops.linear_fwd(xd, wd, dev(b))
    dx, dw, db = ops.linear_bwd(dyd, xd, wd, dw=dev(dw0), db=dev(db0), accumulate=accumulate)
    torch.cuda.synchronize()
    rows = _edge(np.r_[0:4, 124:132, 252:260, m // 2:m // 2 + 4, m - 4:m], m)
    check(host(y)[rows], oracle.linear_fwd(x[rows], w, b), dt, "y rows")
    rdx, _, _ = oracle.linear_bwd(dy[rows], x[rows], w)
    check(host(dx)[rows], rdx, dt, "dx rows")
    outs = _edge(np.r_[0:4, 124:132, 252:260, nout - 4:nout], nout)
    _, rdw, rdb = oracle.linear_bwd(np.ascontiguousarray(dy[:, outs]), x, np.ascontiguousarray(w[outs]))
    check(host(dw)[outs], dw0[outs] + rdw, dt, "dw rows")
    check(host(db)[outs], db0[outs] + rdb, dt, "db rows")


# The FC layer's ReLU in the GEMM epilogues: forward y = relu(x·wᵀ + b), and
# a dx that takes the previous layer's ReLU backward (x a ReLU output, zeros
# included), each bit-identical to the separate passes; on the small CNN's
# FC shapes (fp32) and on the bf16 direct-to-LDS / split plans.
LIN_ACT = [("f32", 64, 3136, 128), ("f32", 64, 128, 10), ("f32", 50, 40, 30), ("bf16", 1024, 200, 320),
           ("bf16", 4104, 192, 2056), ("bf16", 256, 384, 256), ("bf16", 2048, 1288, 1544)]


@pytest.mark.parametrize("dt,m,kin,nout", LIN_ACT)
def test_linear_relu_epilogues(ops, dt, m, kin, nout):
    g = rng(17 + m + kin + nout)
    x = host_input(g.standard_normal((m, kin)), dt)
    w = host_input(g.standard_normal((nout, kin)) / math.sqrt(kin), dt)
    b = f32(g.standard_normal(nout) * 0.1)
    xd, wd, bd = dev(x, dt), dev(w, dt), dev(b)
    iv = torch.int16 if dt == "bf16" else torch.int32
    y = ops.linear_fwd(xd, wd, bd, relu=True)
    y_ref = ops.relu_fwd(ops.linear_fwd(xd, wd, bd))
    assert torch.equal(y.view(iv), y_ref.view(iv))
    h = ops.relu_fwd(xd)                       # a ReLU output: about half zeros
    dy = dev(host_input(g.standard_normal((m, nout)), dt), dt)
    dx, dw, db = ops.linear_bwd(dy, h, wd, relu_input=True)
    dx0, dw0, db0 = ops.linear_bwd(dy, h, wd)
    assert torch.equal(dx.view(iv), ops.relu_bwd(h, dx0).view(iv))
    assert torch.equal(dw, dw0) and torch.equal(db, db0)


def test_linear_golden(ops):
    z = np.load(os.path.join(GOLD, "linear.npz"))
    x, w, b, dy = (f32(z[k]) for k in ("x", "w", "b", "dy"))
    y = ops.linear_fwd(dev(x), dev(w), dev(b))
    dx, dw, db = ops.linear_bwd(dev(dy), dev(x), dev(w))
    torch.cuda.synchronize()
    check(host(y), z["y"], what="golden y")
    check(host(dx), z["dx"], what="golden dx")
    check(host(dw), z["dw"], what="golden dw")
    check(host(db), z["db"], what="golden db")


def test_linear_accumulate_and_partial_outputs(ops, oracle):
    g = rng(3)
    x, w, dy = f32(g.standard_normal((50, 40))), f32(g.standard_normal((30, 40))), f32(g.standard_normal((50, 30)))
    dw0, db0 = f32(g.standard_normal((30, 40))), f32(g.standard_normal(30))
    dwd, dbd = dev(dw0), dev(db0)
    dx, _, _ = ops.linear_bwd(dev(dy), dev(x), dev(w), dw=dwd, db=dbd, accumulate=True)
    _, dw2, db2 = ops.linear_bwd(dev(dy), dev(x), dev(w), need_dx=False)
    torch.cuda.synchronize()
    rdx, rdw, rdb = oracle.linear_bwd(dy, x, w)
    check(host(dwd), dw0 + rdw, what="accumulated dw")
    check(host(dbd), db0 + rdb, what="accumulated db")
    check(host(dw2), rdw, what="dw without dx")
    check(host(db2), rdb, what="db without dx")
    # dW split over the rows (64x64-tile grid): the reduce adds the existing values
    x, w, dy = f32(g.standard_normal((3000, 40))), f32(g.standard_normal((30, 40))), f32(g.standard_normal((3000, 30)))
    dwd, dbd = dev(dw0), dev(db0)
    ops.linear_bwd(dev(dy), dev(x), dev(w), dw=dwd, db=dbd, accumulate=True, need_dx=False)
    torch.cuda.synchronize()
    _, rdw, rdb = oracle.linear_bwd(dy, x, w)
    check(host(dwd), dw0 + rdw, what="accumulated split dw")
    check(host(dbd), db0 + rdb, what="accumulated split db")


# -------------------------------------------------------------------- conv
# (n, c, h, w, k, r, s, stride, pad, dil)
CONV = [
    (2, 3, 9, 9, 4, 3, 3, 1, 1, 1),            # 3x3 s1 p1
    (2, 5, 11, 9, 6, 3, 3, 2, 1, 1),           # 3x3 s2 p1, odd sizes
    (2, 3, 15, 15, 8, 7, 7, 2, 3, 1),          # ResNet stem 7x7 s2 p3
    (2, 8, 10, 10, 16, 1, 1, 2, 0, 1),         # 1x1 s2 projection
    (1, 4, 12, 10, 5, 3, 3, 1, 2, 2),          # dilation 2
    (4, 1, 28, 28, 32, 3, 3, 1, 1, 1),         # configs[0] conv1 (batch 4)
    (4, 32, 14, 14, 64, 3, 3, 1, 1, 1),        # configs[0] conv2 (batch 4)
    (2, 64, 56, 56, 64, 3, 3, 1, 1, 1),        # ResNet stage 1
    (2, 64, 56, 56, 128, 3, 3, 2, 1, 1),       # ResNet stage 2 entry
    (2, 128, 28, 28, 128, 3, 3, 1, 1, 1),      # ResNet stage 2
    (2, 256, 14, 14, 256, 3, 3, 1, 1, 1),      # ResNet stage 3
    (2, 256, 14, 14, 512, 1, 1, 2, 0, 1),      # ResNet stage 4 projection
    (2, 512, 7, 7, 512, 3, 3, 1, 1, 1),        # ResNet stage 4
    (3, 64, 5, 13, 64, 3, 3, 1, 1, 1),         # 3x3 tile spanning three images
    (2, 32, 60, 60, 128, 3, 3, 1, 1, 1),       # widest row the 3x3 kernel takes
    (5, 128, 7, 7, 192, 3, 3, 1, 1, 1),        # ragged last pixel tile
    (3, 16, 12, 12, 48, 3, 3, 1, 1, 1),        # partial 64-channel output blocks (48; dgrad 16)
    (2, 80, 8, 8, 64, 3, 3, 1, 1, 1),          # partial last x-channel block in wgrad, dgrad 80 outputs
    (3, 1, 9, 7, 40, 3, 3, 1, 1, 1),           # one input channel (direct kernels), odd sizes
    # bf16 column path (n·p·q a multiple of 64): strided 3x3, 1x1 projection,
    # 7x7 stem, small-width 3x3 wgrad, odd channel counts
    (4, 64, 56, 56, 128, 3, 3, 2, 1, 1),
    (4, 64, 56, 56, 128, 1, 1, 2, 0, 1),
    (1, 3, 64, 64, 64, 7, 7, 2, 3, 1),
    (16, 64, 14, 14, 64, 3, 3, 1, 1, 1),
    (64, 32, 7, 7, 64, 3, 3, 1, 1, 1),
    (2, 5, 16, 16, 64, 3, 3, 1, 1, 2),
    (2, 3, 15, 15, 64, 7, 7, 2, 3, 1),         # column-path dgrad at an odd width: one-output-per-thread col2im
    # LDS-staged tap kernels (conv_tap.hip): strided 3x3 with odd sizes and a
    # partial 64-channel block (parity classes of different sizes in dgrad),
    # 1x1 stride 2 at odd sizes (dgrad classes no tap reaches stay zero),
    # 3x3 stride 1 wider than the 3x3 kernels take, 1x1 stride 1, and a
    # stride-2 pass small enough to split its channel chunks
    (4, 64, 15, 15, 64, 3, 3, 2, 1, 1),
    (3, 64, 13, 11, 96, 3, 3, 2, 1, 1),
    (2, 64, 9, 9, 64, 1, 1, 2, 0, 1),
    (2, 32, 70, 70, 32, 3, 3, 1, 1, 1),
    (4, 32, 8, 8, 32, 1, 1, 1, 0, 1),
    (1, 128, 8, 8, 64, 3, 3, 2, 1, 1),
    (2, 32, 40, 40, 256, 3, 3, 2, 1, 1),       # one channel chunk: the bf16 forward takes the tap kernel unsplit
    (3, 3, 30, 26, 64, 7, 7, 2, 3, 1),         # stem forward kernel: odd output sizes, tiles across images
    (1, 16, 66, 70, 64, 3, 3, 1, 1, 1),        # tap weight gradient at stride 1 (rows wider than the 3x3 kernel's)
]


def _desc(ops, case, layout=0):
    n, c, h, w, k, r, s, st, pad, dil = case
    return ops.conv_desc((n, c, h, w), (k, c, r, s), stride=(st, st), padding=(pad, pad), dilation=(dil, dil),
                         layout=layout)


def _inputs(case, dt, seed):
    n, c, h, w, k, r, s, st, pad, dil = case
    p, q = conv_out(h, r, st, pad, dil), conv_out(w, s, st, pad, dil)
    g = rng(seed)
    x = host_input(g.standard_normal((n, c, h, w)), dt)
    wt = host_input(g.standard_normal((k, c, r, s)) / math.sqrt(c * r * s), dt)
    b = f32(g.standard_normal(k) * 0.1)
    dy = host_input(g.standard_normal((n, k, p, q)), dt)
    return x, wt, b, dy


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", CONV, ids=lambda c: "n{}c{}h{}w{}k{}r{}s{}st{}p{}d{}".format(*c))
def test_conv(ops, oracle, dt, case):
    d = _desc(ops, case)
    x, w, b, dy = _inputs(case, dt, sum(case))
    y = ops.conv2d_fwd(dev(x, dt), dev(w, dt), dev(b), d)
    dx = ops.conv2d_bwd_data(dev(dy, dt), dev(w, dt), d)
    dw, db = ops.conv2d_bwd_weight(dev(x, dt), dev(dy, dt), d, need_db=True)
    torch.cuda.synchronize()
    check(host(y), oracle.conv2d_fwd(d, x, w, b), dt, "conv y")
    check(host(dx), oracle.conv2d_bwd_data(d, dy, w), dt, "conv dx")
    rdw, rdb = oracle.conv2d_bwd_weight(d, x, dy)
    check(host(dw), rdw, dt, "conv dw")
    check(host(db), rdb, dt, "conv db")


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", [CONV[0], CONV[1], CONV[2], CONV[6]], ids=lambda c: "n{}c{}h{}w{}k{}".format(*c[:5]))
def test_conv_nhwc(ops, oracle, dt, case):
    """Channels-last layout (the reference's ChannelsLast mode) gives the same numbers."""
    d = _desc(ops, case, layout=1)
    dn = _desc(ops, case, layout=0)
    x, w, b, dy = _inputs(case, dt, 7 + sum(case))
    nhwc = lambda a: np.ascontiguousarray(a.transpose(0, 2, 3, 1))
    y = ops.conv2d_fwd(dev(nhwc(x), dt), dev(w, dt), dev(b), d)
    dx = ops.conv2d_bwd_data(dev(nhwc(dy), dt), dev(w, dt), d)
    dw, db = ops.conv2d_bwd_weight(dev(nhwc(x), dt), dev(nhwc(dy), dt), d, need_db=True)
    torch.cuda.synchronize()
    check(host(y), nhwc(oracle.conv2d_fwd(dn, x, w, b)), dt, "nhwc y")
    check(host(dx), nhwc(oracle.conv2d_bwd_data(dn, dy, w)), dt, "nhwc dx")
    rdw, rdb = oracle.conv2d_bwd_weight(dn, x, dy)
    check(host(dw), rdw, dt, "nhwc dw")
    check(host(db), rdb, dt, "nhwc db")


@pytest.mark.parametrize("name", ["conv3x3_s1p1_bias", "conv3x3_s2p1", "conv7x7_s2p3", "conv1x1_s2",
                                  "conv3x3_dil2_rect"])
def test_conv_golden(ops, name):
    """The HIP path against vectors written by the reference's own Conv2d module."""
    z = np.load(os.path.join(GOLD, name + ".npz"))
    n, c, h, w, k, r, s, sh, sw, ph, pw, dh, dw_ = (int(v) for v in z["desc"])
    d = ops.conv_desc((n, c, h, w), (k, c, r, s), stride=(sh, sw), padding=(ph, pw), dilation=(dh, dw_))
    b = dev(f32(z["b"])) if "b" in z else None
    y = ops.conv2d_fwd(dev(f32(z["x"])), dev(f32(z["w"])), b, d)
    dx = ops.conv2d_bwd_data(dev(f32(z["dy"])), dev(f32(z["w"])), d)
    dwt, dbt = ops.conv2d_bwd_weight(dev(f32(z["x"])), dev(f32(z["dy"])), d, need_db="db" in z)
    torch.cuda.synchronize()
    check(host(y), z["y"], what=f"{name} y")
    check(host(dx), z["dx"], what=f"{name} dx")
    check(host(dwt), z["dw"], what=f"{name} dw")
    if "db" in z:
        check(host(dbt), z["db"], what=f"{name} db")


def test_conv_accumulate(ops, oracle):
    case = CONV[0]
    d = _desc(ops, case)
    x, w, b, dy = _inputs(case, "f32", 99)
    g = rng(5)
    dw0, db0 = f32(g.standard_normal(w.shape)), f32(g.standard_normal(w.shape[0]))
    dwd, dbd = dev(dw0), dev(db0)
    ops.conv2d_bwd_weight(dev(x), dev(dy), d, dw=dwd, db=dbd, accumulate=True)
    torch.cuda.synchronize()
    rdw, rdb = oracle.conv2d_bwd_weight(d, x, dy)
    check(host(dwd), dw0 + rdw, what="accumulated dw")
    check(host(dbd), db0 + rdb, what="accumulated db")


def test_conv_rejects_bad_descriptors(ops):
    from thot_amd._abi import NottInvalidArgument
    x = torch.zeros((1, 2, 5, 5), device="cuda")
    w = torch.zeros((3, 2, 3, 3), device="cuda")
    d = ops.conv_desc((1, 2, 5, 5), (3, 2, 3, 3), padding=(1, 1))
    d.groups = 2
    with pytest.raises(NottInvalidArgument):
        ops.conv2d_fwd(x, w, None, d)
    d = ops.conv_desc((1, 2, 5, 5), (3, 2, 3, 3), stride=(0, 1))
    with pytest.raises((NottInvalidArgument, ZeroDivisionError)):
        ops.conv2d_fwd(x, w, None, d)


@pytest.mark.parametrize("dt", DTYPES)
def test_conv_bwd_full_size_config(ops, oracle, dt):
    """configs[1] at full size (N=128, 64->128, 56x56, 3x3 s1 p1).

    dgrad: images 0 and 127 against the oracle (dgrad is per image).
    wgrad: against torch's fp32 convolution backward on the same (rounded)
    inputs, plus the adjoint identity <dy, conv(x, w)> = <w, wgrad(x, dy)>
    = <x, dgrad(dy, w)> in float64."""
    N, C, K, H = 128, 64, 128, 56
    d = ops.conv_desc((N, C, H, H), (K, C, 3, 3), padding=(1, 1))
    gen = torch.Generator(device="cuda").manual_seed(0)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    x = torch.randn((N, C, H, H), generator=gen, device="cuda").to(tdt)
    w = (torch.randn((K, C, 3, 3), generator=gen, device="cuda") / math.sqrt(C * 9)).to(tdt)
    dy = torch.randn((N, K, H, H), generator=gen, device="cuda").to(tdt)
    dx = ops.conv2d_bwd_data(dy, w, d)
    dw, _ = ops.conv2d_bwd_weight(x, dy, d)
    torch.cuda.synchronize()
    d1 = ops.conv_desc((1, C, H, H), (K, C, 3, 3), padding=(1, 1))
    wh = host(w)
    for i in (0, N - 1):
        check(host(dx[i:i + 1]), oracle.conv2d_bwd_data(d1, host(dy[i:i + 1]), wh), dt, f"dx image {i}")
    # torch fp32 reference for the batch-summed weight gradient
    xf, dyf = x.float(), dy.float()
    ref_dw = torch.nn.grad.conv2d_weight(xf, (K, C, 3, 3), dyf, padding=1)
    check(host(dw), host(ref_dw), dt, "dw vs torch fp32")
    # adjoint identities in float64
    xd, wd, dyd = x.double(), w.double(), dy.double()
    y = torch.nn.functional.conv2d(xd, wd, padding=1)
    lhs = float((y * dyd).sum())
    via_w = float((wd * dw.double()).sum())
    via_x = float((xd * dx.double()).sum())
    scale = float(torch.sqrt((y * y).sum() * (dyd * dyd).sum()))
    tol = 1e-6 if dt == "f32" else 2e-3
    assert abs(via_w - lhs) <= tol * scale, (via_w, lhs)
    assert abs(via_x - lhs) <= tol * scale, (via_x, lhs)
    # every image of dx, and the forward, against torch's fp32 convolution
    ref_dx = torch.nn.grad.conv2d_input((N, C, H, H), w.float(), dyf, padding=1)
    check(host(dx), host(ref_dx), dt, "dx vs torch fp32")
    b = torch.randn((K,), generator=gen, device="cuda")
    yk = ops.conv2d_fwd(x, w, b, d)
    check(host(yk), host(torch.nn.functional.conv2d(xf, w.float(), b, padding=1)), dt, "y vs torch fp32")


# Large bf16 3x3 grids: several rounds of workgroups, pixel tiles across
# image boundaries, row widths 8..64, 1..8 output-channel blocks.
# (n, c, h, w, k)
BIG3X3 = [
    (42, 64, 56, 56, 64),
    (33, 64, 32, 32, 256),     # tiles spanning images
    (5, 64, 64, 64, 512),      # widest row, 8 channel blocks
    (1030, 32, 8, 8, 256),     # 4 images per tile, one channel chunk
    (130, 64, 16, 16, 256),
    (34, 256, 32, 32, 64),     # dgrad: cin 64 -> 256 output channels
]


@pytest.mark.parametrize("case", BIG3X3)
def test_conv3x3_large_grids(ops, case):
    """bf16 forward and dgrad of 3x3 s1 p1 convs at sizes the CPU oracle is
    too slow for, against torch's fp32 convolution on the same rounded inputs
    (the same kernels meet the oracle at the small sizes above)."""
    n, c, h, w_, k = case
    d = ops.conv_desc((n, c, h, w_), (k, c, 3, 3), padding=(1, 1))
    gen = torch.Generator(device="cuda").manual_seed(sum(case))
    x = torch.randn((n, c, h, w_), generator=gen, device="cuda").to(torch.bfloat16)
    w = (torch.randn((k, c, 3, 3), generator=gen, device="cuda") / math.sqrt(c * 9)).to(torch.bfloat16)
    b = torch.randn((k,), generator=gen, device="cuda")
    dy = torch.randn((n, k, h, w_), generator=gen, device="cuda").to(torch.bfloat16)
    y = ops.conv2d_fwd(x, w, b, d)
    dx = ops.conv2d_bwd_data(dy, w, d)
    torch.cuda.synchronize()
    ref_y = torch.nn.functional.conv2d(x.float(), w.float(), b, padding=1)
    ref_dx = torch.nn.grad.conv2d_input((n, c, h, w_), w.float(), dy.float(), padding=1)
    check(host(y), host(ref_y), "bf16", "y vs torch fp32")
    check(host(dx), host(ref_dx), "bf16", "dx vs torch fp32")


# bf16 3x3 passes on the direct-to-LDS kernel (conv3x3_dma.hip: row widths
# dividing 112, 32-channel multiples): ragged last row bands (h not a
# multiple of the 448-pixel tile's rows), loaded pixel ranges that start off
# a 16-byte boundary (w = 28), several output-channel blocks and input
# chunks, 28-row tiles (w = 16) and 4-row tiles (w = 112), workgroups that
# walk several tiles.
# (n, c, h, w, k)
DMA3X3 = [
    (2, 32, 30, 56, 96),
    (3, 96, 14, 28, 64),
    (2, 64, 9, 16, 32),
    (4, 32, 8, 8, 64),
    (3, 32, 21, 16, 64),
    (1, 32, 5, 112, 64),
    (8, 32, 30, 56, 512),      # 16 output blocks: workgroups walk two tiles each, across images
]


@pytest.mark.parametrize("case", DMA3X3, ids=lambda c: "n{}c{}h{}w{}k{}".format(*c))
def test_conv3x3_dma_vs_oracle(ops, oracle, case):
    """bf16 forward (with bias, with and without the fused ReLU) and data
    gradient of the DMA kernel against the oracle."""
    n, c, h, w_, k = case
    cc = (n, c, h, w_, k, 3, 3, 1, 1, 1)
    d = _desc(ops, cc)
    x, w, b, dy = _inputs(cc, "bf16", 11 + sum(case))
    y = ops.conv2d_fwd(dev(x, "bf16"), dev(w, "bf16"), dev(b), d)
    yr = ops.conv2d_fwd(dev(x, "bf16"), dev(w, "bf16"), dev(b), d, relu=True)
    dx = ops.conv2d_bwd_data(dev(dy, "bf16"), dev(w, "bf16"), d)
    torch.cuda.synchronize()
    ry = oracle.conv2d_fwd(d, x, w, b)
    check(host(y), ry, "bf16", "conv y")
    check(host(yr), np.maximum(ry, 0), "bf16", "conv relu(y)")
    assert torch.equal(yr, torch.relu(y))
    check(host(dx), oracle.conv2d_bwd_data(d, dy, w), "bf16", "conv dx")


# bf16 3x3 weight gradients on the direct-to-LDS band kernel
# (conv3x3_dma.hip: rows of a multiple of 8 pixels dividing 224, 64-channel
# dy blocks): ragged last bands, a partial last x-channel block, two dy
# blocks, 7-, 14- and 28-row bands, several bands per split.  (n, c, h, w, k)
WDMA3X3 = [
    (2, 48, 30, 56, 64),
    (3, 64, 13, 32, 128),
    (2, 16, 20, 16, 64),
    (5, 32, 9, 8, 64),
    (6, 96, 56, 56, 64),
]


@pytest.mark.parametrize("case", WDMA3X3, ids=lambda c: "n{}c{}h{}w{}k{}".format(*c))
def test_conv3x3_wgrad_dma_vs_oracle(ops, oracle, case):
    """bf16 weight gradient (and bias gradient) of the band kernel against
    the oracle, set and accumulated."""
    n, c, h, w_, k = case
    cc = (n, c, h, w_, k, 3, 3, 1, 1, 1)
    d = _desc(ops, cc)
    x, w, b, dy = _inputs(cc, "bf16", 17 + sum(case))
    dw, db = ops.conv2d_bwd_weight(dev(x, "bf16"), dev(dy, "bf16"), d, need_db=True)
    dw0 = f32(rng(5).standard_normal((k, c, 3, 3)))
    dwa = dev(dw0)
    ops.conv2d_bwd_weight(dev(x, "bf16"), dev(dy, "bf16"), d, dw=dwa, accumulate=True)
    torch.cuda.synchronize()
    rdw, rdb = oracle.conv2d_bwd_weight(d, x, dy)
    check(host(dw), rdw, "bf16", "conv dw")
    check(host(db), rdb, "bf16", "conv db")
    check(host(dwa), dw0 + rdw, "bf16", "conv dw accumulated")


# bf16 3x3 weight gradients of images at most 15 wide that the band kernel
# does not take: the images are stacked vertically with a zero row after
# each, in bands of 256 slots (slot pitch 8 / 16: 32 / 16 rows), so bands
# start and end inside images and hold several of them.  Odd widths read
# their 2-byte-aligned rows with realigning 16-byte loads (8-element chunks
# with a fifth dword at w = 9, 11, 15), element by element in the band that
# holds the tensor's last row.  The 20- and 28-wide cases keep one image per
# band.
STACK3X3 = [
    (3, 32, 7, 7, 64),
    (16, 256, 7, 7, 128),
    (4, 64, 14, 14, 64),
    (7, 48, 5, 6, 64),
    (5, 64, 11, 12, 64),
    (1, 128, 3, 3, 64),
    (4, 32, 9, 9, 64),
    (5, 16, 13, 11, 64),
    (2, 64, 15, 15, 64),
    (2, 16, 28, 28, 128),
    (3, 24, 20, 20, 64),
]


@pytest.mark.parametrize("case", STACK3X3, ids=lambda c: "n{}c{}h{}w{}k{}".format(*c))
def test_conv3x3_wgrad_stacked_vs_oracle(ops, oracle, case):
    """bf16 weight gradient (and bias gradient) over stacked-image bands
    against the oracle, set and accumulated."""
    n, c, h, w_, k = case
    cc = (n, c, h, w_, k, 3, 3, 1, 1, 1)
    d = _desc(ops, cc)
    x, w, b, dy = _inputs(cc, "bf16", 29 + sum(case))
    dw, db = ops.conv2d_bwd_weight(dev(x, "bf16"), dev(dy, "bf16"), d, need_db=True)
    dw0 = f32(rng(7).standard_normal((k, c, 3, 3)))
    dwa = dev(dw0)
    ops.conv2d_bwd_weight(dev(x, "bf16"), dev(dy, "bf16"), d, dw=dwa, accumulate=True)
    torch.cuda.synchronize()
    rdw, rdb = oracle.conv2d_bwd_weight(d, x, dy)
    check(host(dw), rdw, "bf16", "conv dw")
    check(host(db), rdb, "bf16", "conv db")
    check(host(dwa), dw0 + rdw, "bf16", "conv dw accumulated")


# fp32 3x3 grids of a little more than one round of workgroup slots (512 on
# 256 CUs) with one output-channel block: the last tiles are split over their
# channel chunks in the same launch (4 pieces each for 64 input channels, 8
# for 128) and summed by the split reduce; the last tile is partial.
TAIL3X3 = [
    (42, 64, 56, 56, 64),      # forward and dgrad: 515 tiles, 3 split 4 ways
    (43, 64, 56, 56, 128),     # dgrad (128 -> 64 channels): 527 tiles, 15 split 8 ways
]


@pytest.mark.parametrize("case", TAIL3X3)
def test_conv3x3_tail_split_fp32(ops, case):
    """fp32 forward (with bias) and dgrad whose last partial round of tiles is
    split, against torch's fp32 convolution; images in the split tail and
    before it are both checked."""
    n, c, h, w_, k = case
    d = ops.conv_desc((n, c, h, w_), (k, c, 3, 3), padding=(1, 1))
    gen = torch.Generator(device="cuda").manual_seed(sum(case))
    x = torch.randn((n, c, h, w_), generator=gen, device="cuda")
    w = torch.randn((k, c, 3, 3), generator=gen, device="cuda") / math.sqrt(c * 9)
    b = torch.randn((k,), generator=gen, device="cuda")
    dy = torch.randn((n, k, h, w_), generator=gen, device="cuda")
    y = ops.conv2d_fwd(x, w, b, d)
    dx = ops.conv2d_bwd_data(dy, w, d)
    torch.cuda.synchronize()
    ref_y = torch.nn.functional.conv2d(x, w, b, padding=1)
    ref_dx = torch.nn.grad.conv2d_input((n, c, h, w_), w, dy, padding=1)
    check(host(y), host(ref_y), "f32", "y vs torch fp32")
    check(host(dx), host(ref_dx), "f32", "dx vs torch fp32")
    # the last images (the split tail) on their own
    check(host(dx[-3:]), host(ref_dx[-3:]), "f32", "dx tail images")


TAIL3X3_BF16 = [
    (42, 256, 56, 56, 64),     # forward over 256 channels (8 bf16 chunks): 515 tiles, 3 split 8 ways
    (42, 64, 56, 56, 256),     # dgrad over dy's 256 channels: the same split
]


@pytest.mark.parametrize("case", TAIL3X3_BF16)
def test_conv3x3_tail_split_bf16(ops, case):
    """bf16 forward and dgrad whose tail tiles are split (the fp32 split
    partials and their reduce, with bf16 stores) against torch's fp32
    convolution of the same bf16-rounded operands."""
    n, c, h, w_, k = case
    d = ops.conv_desc((n, c, h, w_), (k, c, 3, 3), padding=(1, 1))
    gen = torch.Generator(device="cuda").manual_seed(sum(case) + 1)
    x = torch.randn((n, c, h, w_), generator=gen, device="cuda").to(torch.bfloat16)
    w = (torch.randn((k, c, 3, 3), generator=gen, device="cuda") / math.sqrt(c * 9)).to(torch.bfloat16)
    dy = torch.randn((n, k, h, w_), generator=gen, device="cuda").to(torch.bfloat16)
    y = ops.conv2d_fwd(x, w, None, d)
    dx = ops.conv2d_bwd_data(dy, w, d)
    torch.cuda.synchronize()
    ref_y = torch.nn.functional.conv2d(x.float(), w.float(), None, padding=1)
    ref_dx = torch.nn.grad.conv2d_input((n, c, h, w_), w.float(), dy.float(), padding=1)
    check(host(y), host(ref_y), "bf16", "y vs torch fp32")
    check(host(dx), host(ref_dx), "bf16", "dx vs torch fp32")
    check(host(y[-3:]), host(ref_y[-3:]), "bf16", "y tail images")
    check(host(dx[-3:]), host(ref_dx[-3:]), "bf16", "dx tail images")


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", [CONV[5], CONV[6], CONV[2], CONV[3], (2, 32, 10, 10, 64, 3, 3, 1, 1, 1)],
                         ids=lambda c: "n{}c{}h{}w{}k{}r{}s{}st{}".format(*c[:8]))
def test_conv_fwd_relu_fused(ops, dt, case):
    """nott_conv2d_fwd_act(relu=1) equals the ReLU of the plain forward, bit
    for bit, on every forward path (single channel, 3×3 MFMA with and without
    split-K, column path, generic GEMM + separate ReLU)."""
    d = _desc(ops, case)
    x, w, b, _ = _inputs(case, dt, 3 + sum(case))
    xd, wd, bd = dev(x, dt), dev(w, dt), dev(b)
    y = ops.conv2d_fwd(xd, wd, bd, d)
    yr = ops.conv2d_fwd(xd, wd, bd, d, relu=True)
    torch.cuda.synchronize()
    assert torch.equal(yr, torch.relu(y))


PREP_CASES = [
    (2, 64, 14, 14, 64),     # one 64-channel block each way
    (2, 32, 9, 7, 96),       # a partial last block of output channels
    (4, 128, 7, 7, 256),     # channel splits (small grid)
    (1, 64, 28, 28, 128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("case", PREP_CASES)
def test_conv_prepared_dgrad_weights(ops, dt, case):
    """nott_conv2d_fwd_prep writes the data gradient's weight layout from the
    forward's own weight prep; its output and the prepared data gradient equal
    nott_conv2d_fwd_act / nott_conv2d_bwd_data bit for bit."""
    import ctypes as C
    from thot_amd import _abi
    n, c, h, w, k = case
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    code = _abi.NOTT_F32 if dt == "f32" else _abi.NOTT_BF16
    g = torch.Generator(device="cuda").manual_seed(n * 1000 + c + k)
    x = torch.randn((n, c, h, w), generator=g, device="cuda").to(tdt)
    wt = (torch.randn((k, c, 3, 3), generator=g, device="cuda") / math.sqrt(9 * c)).to(tdt)
    b = torch.randn((k,), generator=g, device="cuda")
    dy = torch.randn((n, k, h, w), generator=g, device="cuda").to(tdt)
    d = ops.conv_desc((n, c, h, w), (k, c, 3, 3), padding=(1, 1))
    nb = C.c_int64()
    assert ops.context(0).lib.nott_conv2d_dgrad_prep_bytes(C.byref(d), code, C.byref(nb)) == 0
    assert nb.value > 0
    wd = torch.empty((nb.value,), dtype=torch.uint8, device="cuda")
    P = lambda t: C.c_void_p(t.data_ptr())
    fb = C.cast(b.data_ptr(), C.POINTER(C.c_float))
    ctx = ops.context(0)
    for relu in (0, 1):
        y0, y1 = torch.empty((n, k, h, w), dtype=tdt, device="cuda"), torch.empty((n, k, h, w), dtype=tdt, device="cuda")
        ctx.call("nott_conv2d_fwd_act", C.byref(d), code, P(x), P(wt), fb, relu, P(y0))
        ctx.call("nott_conv2d_fwd_prep", C.byref(d), code, P(x), P(wt), fb, relu, P(y1), P(wd))
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), relu
    dx0, dx1 = torch.empty_like(x), torch.empty_like(x)
    ctx.call("nott_conv2d_bwd_data", C.byref(d), code, P(dy), P(wt), P(dx0))
    ctx.call("nott_conv2d_bwd_data_prepped", C.byref(d), code, P(dy), P(wd), P(dx1))
    torch.cuda.synchronize()
    assert torch.equal(dx0, dx1)


@pytest.mark.gpu
def test_conv_prepared_dgrad_weights_other_shapes(ops):
    """Convolutions outside the 3x3 stride-1 kernels report no prepared
    layout, and the prepared entry points refuse them."""
    import ctypes as C
    from thot_amd import _abi
    nb = C.c_int64()
    for xs, ws, st, pd in (((2, 64, 14, 14), (64, 64, 3, 3), (2, 2), (1, 1)),
                           ((2, 64, 14, 14), (128, 64, 1, 1), (1, 1), (0, 0)),
                           ((2, 3, 32, 32), (64, 3, 7, 7), (2, 2), (3, 3))):
        d = ops.conv_desc(xs, ws, stride=st, padding=pd)
        assert ops.context(0).lib.nott_conv2d_dgrad_prep_bytes(C.byref(d), _abi.NOTT_BF16, C.byref(nb)) == 0
        assert nb.value == 0, (xs, ws)
        x = torch.zeros(xs, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(_abi.NottInvalidArgument):
            ops.context(0).call("nott_conv2d_bwd_data_prepped", C.byref(d), _abi.NOTT_BF16, C.c_void_p(x.data_ptr()),
                                C.c_void_p(x.data_ptr()), C.c_void_p(x.data_ptr()))
