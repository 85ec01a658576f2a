"""Writes the golden fixtures in tests/golden/*.npz from the reference itself.

The reference (Nott) is C++ over libtorch; oracle/ref/nott_ref.cpp drives its
own modules (build_registered_layer for Conv2d / FC / MaxPool2d /
AdaptiveAvgPool2d / BatchNorm2d, Activation::Details::apply, Loss::Details::compute,
Optimizer::Details::Adam/AdamW, ScaledDotProductKernel, MultiHeadAttention)
on the CPU.  Build it with `make -C oracle ref` (needs /root/reference), then:

    python tests/golden/make_golden.py

Each fixture holds the seeded inputs, the options and the reference's outputs.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from oracle_lib import Ref, f32, rng  # noqa: E402
from thot_amd._abi import AttnDesc, Conv2dDesc, Pool2dDesc  # noqa: E402

CONV_CASES = [
    # name, n, c, h, w, k, r, s, stride, pad, dil, bias
    ("conv3x3_s1p1_bias", 2, 3, 9, 9, 4, 3, 3, (1, 1), (1, 1), (1, 1), True),
    ("conv3x3_s2p1", 2, 3, 9, 8, 4, 3, 3, (2, 2), (1, 1), (1, 1), False),
    ("conv7x7_s2p3", 1, 3, 12, 12, 5, 7, 7, (2, 2), (3, 3), (1, 1), False),
    ("conv1x1_s2", 2, 4, 7, 7, 6, 1, 1, (2, 2), (0, 0), (1, 1), False),
    ("conv3x3_dil2_rect", 1, 2, 10, 7, 3, 3, 2, (1, 2), (2, 1), (2, 1), True),
]

POOL_CASES = [
    # name, n, c, h, w, k, stride, pad, dil, ceil
    ("maxpool2x2_s2_relu_ties", 2, 3, 8, 8, (2, 2), (2, 2), (0, 0), (1, 1), False),
    ("maxpool3x3_s2p1_overlap", 2, 2, 9, 9, (3, 3), (2, 2), (1, 1), (1, 1), False),
    ("maxpool3x3_s2_ceil", 1, 2, 8, 8, (3, 3), (2, 2), (0, 0), (1, 1), True),
    ("maxpool2x2_dil2", 1, 2, 7, 7, (2, 2), (1, 1), (0, 0), (2, 2), False),
]


NONFINITE_POOL_CASES = [
    # name, n, c, h, w, k, stride, pad
    ("maxpool3x3_s2p1_nan_inf", 1, 5, 9, 9, (3, 3), (2, 2), (1, 1)),   # the ResNet-18 stem pool's window
    ("maxpool2x2_s2_nan_inf", 2, 3, 6, 6, (2, 2), (2, 2), (0, 0)),     # the small CNN's
]


def nonfinite_pool_input(g, n, c, h, w):
    """Planes of non-finite windows: 0 all -inf; 1 all NaN; 2 normal values
    with single NaNs, two NaNs in one window, a NaN beside +inf, and +inf;
    3 whole windows (and the padded corner window) of -inf among normal
    values, with equal maxima; 4 post-ReLU zeros with -inf and NaN mixed."""
    x = g.standard_normal((n, c, h, w)).astype(np.float32)
    x[:, 0] = -np.inf
    if c > 1:
        x[:, 1] = np.nan
    if c > 2:
        p = x[:, 2]
        p[:, 0, 0] = np.nan                       # first element of a window
        p[:, 2, 3] = np.nan                       # two NaNs in one window (the last wins)
        p[:, 3, 3] = np.nan
        p[:, h - 1, w - 1] = np.nan               # last element of the image
        p[:, 4, 1] = np.inf
        p[:, 4, 0] = np.nan                       # NaN beside +inf
        p[:, 1, 4] = np.inf
    if c > 3:
        p = x[:, 3]
        p[:, 0:2, 0:2] = -np.inf                  # the window at the padded corner
        p[:, 2:4, 2:4] = -np.inf
        p[:, 3:6, 3:6] = -np.inf
        p[:, h - 2:, 0:3] = 0.75                  # equal maxima
    if c > 4:
        p = np.maximum(x[:, 4], 0.0)
        p[:, ::3, ::2] = -np.inf
        p[:, 1::4, 1::3] = np.nan
        x[:, 4] = p
    return x


def save(name: str, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **{k: np.asarray(v) for k, v in arrays.items()})
    print("wrote", os.path.relpath(path))


def main():
    ref = Ref()
    ref.set_threads(1)

    for i, (name, n, c, h, w, k, r, s, st, pd, dl, bias) in enumerate(CONV_CASES):
        g = rng(100 + i)
        d = Conv2dDesc(n, c, h, w, k, r, s, st[0], st[1], pd[0], pd[1], dl[0], dl[1], 1, 0, 0)
        x = f32(g.standard_normal((n, c, h, w)))
        wt = f32(g.standard_normal((k, c, r, s)) / np.sqrt(c * r * s))
        b = f32(g.standard_normal(k)) if bias else None
        p_ = (h + 2 * pd[0] - dl[0] * (r - 1) - 1) // st[0] + 1
        q_ = (w + 2 * pd[1] - dl[1] * (s - 1) - 1) // st[1] + 1
        dy = f32(g.standard_normal((n, k, p_, q_)))
        y, dx, dw, db = ref.conv2d(d, x, wt, b, dy)
        extra = {"b": b, "db": db} if bias else {}
        save(name, desc=np.array([n, c, h, w, k, r, s, st[0], st[1], pd[0], pd[1], dl[0], dl[1]], np.int64),
             x=x, w=wt, dy=dy, y=y, dx=dx, dw=dw, **extra)

    g = rng(200)
    x = f32(g.standard_normal((5, 7)))
    wt = f32(g.standard_normal((3, 7)) * 0.3)
    b = f32(g.standard_normal(3))
    dy = f32(g.standard_normal((5, 3)))
    y, dx, dw, db = ref.linear(x, wt, b, dy)
    save("linear", x=x, w=wt, b=b, dy=dy, y=y, dx=dx, dw=dw, db=db)

    g = rng(201)
    x = f32(g.standard_normal(64))
    x[::7] = 0.0
    x[3] = -0.0
    x[5] = np.nan
    dy = f32(g.standard_normal(64))
    y, dx = ref.relu(x, dy)
    save("relu", x=x, dy=dy, y=y, dx=dx)

    for i, (name, n, c, h, w, kk, st, pd, dl, ceil) in enumerate(POOL_CASES):
        g = rng(300 + i)
        d = Pool2dDesc(n, c, h, w, kk[0], kk[1], st[0], st[1], pd[0], pd[1], dl[0], dl[1], int(ceil), 0)
        x = f32(g.standard_normal((n, c, h, w)))
        if "relu_ties" in name:
            x = np.maximum(x, 0.0).astype(np.float32)  # post-ReLU: many exact-zero ties
            x[0, 0, 0:2, 0:2] = 0.0
        if "overlap" in name:
            x[0, 0, 0, :] = 1.5  # equal maxima inside overlapping windows
            x[0, 1, 2, 2] = np.nan
            x[1, 0, 4:7, 4:7] = -np.inf
        oh = (h + 2 * pd[0] - dl[0] * (kk[0] - 1) - 1 + (st[0] - 1 if ceil else 0)) // st[0] + 1
        ow = (w + 2 * pd[1] - dl[1] * (kk[1] - 1) - 1 + (st[1] - 1 if ceil else 0)) // st[1] + 1
        if ceil and (oh - 1) * st[0] >= h + pd[0]:
            oh -= 1
        if ceil and (ow - 1) * st[1] >= w + pd[1]:
            ow -= 1
        dy = f32(g.standard_normal((n, c, oh, ow)))
        y, idx, dx = ref.maxpool2d(d, x, dy)
        save(name, desc=np.array([n, c, h, w, kk[0], kk[1], st[0], st[1], pd[0], pd[1], dl[0], dl[1], int(ceil)],
                                 np.int64), x=x, dy=dy, y=y, argmax=idx, dx=dx)

    # Non-finite windows (pooling.hpp:144, ATen's max_pool2d rule: a NaN
    # always takes the window, so the last NaN wins; a window of -inf only
    # keeps its first in-image element).
    for i, (name, n, c, h, w, kk, st, pd) in enumerate(NONFINITE_POOL_CASES):
        g = rng(350 + i)
        d = Pool2dDesc(n, c, h, w, kk[0], kk[1], st[0], st[1], pd[0], pd[1], 1, 1, 0, 0)
        x = nonfinite_pool_input(g, n, c, h, w)
        oh = (h + 2 * pd[0] - (kk[0] - 1) - 1) // st[0] + 1
        ow = (w + 2 * pd[1] - (kk[1] - 1) - 1) // st[1] + 1
        dy = f32(g.standard_normal((n, c, oh, ow)))
        y, idx, dx = ref.maxpool2d(d, x, dy)
        save(name, desc=np.array([n, c, h, w, kk[0], kk[1], st[0], st[1], pd[0], pd[1], 1, 1, 0], np.int64),
             x=x, dy=dy, y=y, argmax=idx, dx=dx)

    g = rng(400)
    x = f32(g.standard_normal((2, 3, 5, 5)))
    dy = f32(g.standard_normal((2, 3, 1, 1)))
    y, dx = ref.avgpool_global(x, dy)
    save("avgpool_global", x=x, dy=dy, y=y, dx=dx)

    g = rng(401)
    x = f32(g.standard_normal((3, 4, 5, 5)) * 2.0 + 0.5)
    gamma = f32(1.0 + 0.1 * g.standard_normal(4))
    beta = f32(0.1 * g.standard_normal(4))
    dy = f32(g.standard_normal((3, 4, 5, 5)))
    rm = f32(0.1 * g.standard_normal(4))
    rv = f32(1.0 + 0.1 * np.abs(g.standard_normal(4)))
    y, dx, dg, db, rm2, rv2 = ref.batchnorm2d(x, gamma, beta, dy, 1e-5, 0.1, rm, rv)
    save("batchnorm2d", x=x, gamma=gamma, beta=beta, dy=dy, running_mean=rm, running_var=rv, y=y, dx=dx, dgamma=dg,
         dbeta=db, running_mean_out=rm2, running_var_out=rv2)

    g = rng(402)
    x = f32(g.standard_normal((6, 16)))
    gamma = f32(1.0 + 0.1 * g.standard_normal(16))
    beta = f32(0.1 * g.standard_normal(16))
    dy = f32(g.standard_normal((6, 16)))
    y, dx, dg, db = ref.layernorm(x, gamma, beta, dy)
    save("layernorm", x=x, gamma=gamma, beta=beta, dy=dy, y=y, dx=dx, dgamma=dg, dbeta=db)

    for i, (name, eps, ignore) in enumerate((("xent", 0.0, False), ("xent_smooth_ignore", 0.1, True))):
        g = rng(500 + i)
        logits = f32(g.standard_normal((8, 10)) * 2.0)
        labels = g.integers(0, 10, 8).astype(np.int64)
        if ignore:
            labels[[1, 5]] = -100
        dl, loss = ref.cross_entropy(logits, labels, eps)
        save(name, logits=logits, labels=labels, label_smoothing=np.array(eps), dlogits=dl, loss=np.array(loss))

    for i, (name, dec, wd, step) in enumerate((("adam_step1", 0, 0.0, 1), ("adam_l2_step10", 0, 0.01, 10),
                                                ("adamw_step10", 1, 0.01, 10), ("adamw_step1_nowd", 1, 0.0, 1))):
        g = rng(600 + i)
        n = 64
        p = f32(g.standard_normal(n) * 0.02)
        gr = f32(g.standard_normal(n) * 1e-3)
        m = f32(g.standard_normal(n) * 1e-4) if step > 1 else np.zeros(n, np.float32)
        v = f32(np.abs(g.standard_normal(n)) * 1e-7) if step > 1 else np.zeros(n, np.float32)
        lr, b1, b2, ep = 3e-4, 0.9, 0.999, 1e-8
        p2, m2, v2 = ref.adam_step(dec, p, gr, m, v, lr, b1, b2, ep, wd, step)
        save(name, decoupled=np.array(dec), p=p, g=gr, m=m, v=v,
             hyper=np.array([lr, b1, b2, ep, wd, step], np.float64), p_out=p2, m_out=m2, v_out=v2)

    for i, (name, causal) in enumerate((("attention_causal", 1), ("attention_full", 0))):
        g = rng(700 + i)
        d = AttnDesc(1, 2, 5, 5, 4, causal, 0, 0.5)
        q, k, v, dO = (f32(g.standard_normal((1, 2, 5, 4))) for _ in range(4))
        o, dq, dk, dv = ref.attention(d, q, k, v, dO)
        save(name, causal=np.array(causal), q=q, k=k, v=v, dO=dO, o=o, dq=dq, dk=dk, dv=dv)

    g = rng(800)
    b, t, e, heads = 2, 5, 8, 2
    x = f32(g.standard_normal((b, t, e)))
    ws = [f32(g.standard_normal((e, e)) * 0.3) for _ in range(4)]
    bs = [f32(g.standard_normal(e) * 0.1) for _ in range(4)]
    dy = f32(g.standard_normal((b, t, e)))
    outs = ref.mha(x, *ws, *bs, dy, heads, True)
    save("mha_causal", x=x, wq=ws[0], wk=ws[1], wv=ws[2], wo=ws[3], bq=bs[0], bk=bs[1], bv=bs[2], bo=bs[3], dy=dy,
         heads=np.array(heads), **outs)


if __name__ == "__main__":
    main()
