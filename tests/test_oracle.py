"""Pins the CPU oracle (oracle/oracle.c).

1. Golden vectors written by the reference's own modules (tests/golden/*.npz,
   from oracle/_ref via tests/golden/make_golden.py): every oracle function
   must reproduce them (fp32 rel 1e-4 / abs 1e-5, indices bit-exact).
2. Mathematical checks independent of the oracle's formulas: adjoint
   identities, finite differences, conservation invariants, closed forms.
3. When oracle/_ref is built here, randomised cases against the reference.
"""
import glob
import os

import numpy as np
import pytest

from oracle_lib import conv_out, f32, rng, round_bf16
from thot_amd._abi import AttnDesc, Conv2dDesc, Pool2dDesc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RTOL, ATOL = 1e-4, 1e-5


def close(a, b, rtol=RTOL, atol=ATOL):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    nan_a, nan_b = np.isnan(a), np.isnan(b)
    assert np.array_equal(nan_a, nan_b), "NaN positions differ"
    a, b = a[~nan_a], b[~nan_b]
    inf = np.isinf(a) | np.isinf(b)
    assert np.array_equal(a[inf], b[inf]), "infinities differ"
    a, b = a[~inf], b[~inf]
    err = np.abs(a - b) - (atol + rtol * np.abs(b))
    assert (err <= 0).all(), f"max excess {err.max():.3e}"


def load(name):
    return np.load(os.path.join(GOLD, name + ".npz"))


def conv_from(desc):
    n, c, h, w, k, r, s, sh, sw, ph, pw, dh, dw = (int(v) for v in desc)
    return Conv2dDesc(n, c, h, w, k, r, s, sh, sw, ph, pw, dh, dw, 1, 0, 0)


def pool_from(desc):
    n, c, h, w, kh, kw, sh, sw, ph, pw, dh, dw, ceil = (int(v) for v in desc)
    return Pool2dDesc(n, c, h, w, kh, kw, sh, sw, ph, pw, dh, dw, ceil, 0)


def test_golden_set_is_complete():
    names = {os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLD, "*.npz"))}
    for need in ("linear", "relu", "avgpool_global", "batchnorm2d", "layernorm", "xent", "xent_smooth_ignore",
                 "adam_step1", "adamw_step10", "attention_causal", "mha_causal"):
        assert need in names


# ------------------------------------------------------------------- golden
@pytest.mark.parametrize("name", ["conv3x3_s1p1_bias", "conv3x3_s2p1", "conv7x7_s2p3", "conv1x1_s2",
                                  "conv3x3_dil2_rect"])
def test_conv_golden(oracle, name):
    g = load(name)
    d = conv_from(g["desc"])
    b = g["b"] if "b" in g else None
    close(oracle.conv2d_fwd(d, g["x"], g["w"], b), g["y"])
    close(oracle.conv2d_bwd_data(d, g["dy"], g["w"]), g["dx"])
    dw, db = oracle.conv2d_bwd_weight(d, g["x"], g["dy"], with_db=True)
    close(dw, g["dw"])
    if b is not None:
        close(db, g["db"])


def test_linear_golden(oracle):
    g = load("linear")
    close(oracle.linear_fwd(g["x"], g["w"], g["b"]), g["y"])
    dx, dw, db = oracle.linear_bwd(g["dy"], g["x"], g["w"])
    close(dx, g["dx"])
    close(dw, g["dw"])
    close(db, g["db"])


def test_relu_golden(oracle):
    g = load("relu")
    close(oracle.relu_fwd(g["x"]), g["y"])
    y = oracle.relu_fwd(g["x"])
    close(oracle.relu_bwd(y, g["dy"]), g["dx"])


@pytest.mark.parametrize("name", ["maxpool2x2_s2_relu_ties", "maxpool3x3_s2p1_overlap", "maxpool3x3_s2_ceil",
                                  "maxpool2x2_dil2", "maxpool3x3_s2p1_nan_inf", "maxpool2x2_s2_nan_inf"])
def test_maxpool_golden(oracle, name):
    g = load(name)
    d = pool_from(g["desc"])
    y, idx = oracle.maxpool2d_fwd(d, g["x"])
    assert np.array_equal(idx, g["argmax"]), "argmax routing differs from the reference"
    close(y, g["y"])
    close(oracle.maxpool2d_bwd(d, idx, g["dy"]), g["dx"])


def test_avgpool_golden(oracle):
    g = load("avgpool_global")
    close(oracle.avgpool_global_fwd(g["x"]), g["y"])
    close(oracle.avgpool_global_bwd(g["dy"], g["x"].shape[2:]), g["dx"])


def test_batchnorm_golden(oracle):
    g = load("batchnorm2d")
    y, mean, rstd, rm, rv = oracle.batchnorm2d_fwd(g["x"], g["gamma"], g["beta"], 1e-5, 0.1, g["running_mean"],
                                                   g["running_var"])
    close(y, g["y"])
    close(rm, g["running_mean_out"])
    close(rv, g["running_var_out"])
    dx, dg, db = oracle.batchnorm2d_bwd(g["x"], g["dy"], mean, rstd, g["gamma"])
    close(dx, g["dx"])
    close(dg, g["dgamma"])
    close(db, g["dbeta"])


def test_layernorm_golden(oracle):
    g = load("layernorm")
    y, mean, rstd = oracle.layernorm_fwd(g["x"], g["gamma"], g["beta"])
    close(y, g["y"])
    dx, dg, db = oracle.layernorm_bwd(g["x"], g["dy"], mean, rstd, g["gamma"])
    close(dx, g["dx"])
    close(dg, g["dgamma"])
    close(db, g["dbeta"])


@pytest.mark.parametrize("name", ["xent", "xent_smooth_ignore"])
def test_xent_golden(oracle, name):
    g = load(name)
    dl, loss = oracle.softmax_xent(g["logits"], g["labels"], float(g["label_smoothing"]))
    close(dl, g["dlogits"])
    close(loss, g["loss"])


@pytest.mark.parametrize("name", ["adam_step1", "adam_l2_step10", "adamw_step10", "adamw_step1_nowd"])
def test_adam_golden(oracle, name):
    g = load(name)
    lr, b1, b2, eps, wd, step = g["hyper"]
    p, m, v = oracle.adam_step(int(g["decoupled"]), g["p"], g["g"], g["m"], g["v"], lr, b1, b2, eps, wd, int(step))
    close(p, g["p_out"], rtol=1e-6, atol=1e-9)
    close(m, g["m_out"], rtol=1e-6, atol=1e-12)
    close(v, g["v_out"], rtol=1e-6, atol=1e-15)


@pytest.mark.parametrize("name", ["attention_causal", "attention_full"])
def test_attention_golden(oracle, name):
    g = load(name)
    q = g["q"]
    d = AttnDesc(q.shape[0], q.shape[1], q.shape[2], g["k"].shape[2], q.shape[3], int(g["causal"]), 0,
                 1.0 / np.sqrt(q.shape[3]))
    o, _ = oracle.attention_fwd(d, q, g["k"], g["v"])
    close(o, g["o"])
    dq, dk, dv = oracle.attention_bwd(d, q, g["k"], g["v"], o, g["dO"])
    close(dq, g["dq"])
    close(dk, g["dk"])
    close(dv, g["dv"])


def test_mha_golden_composition(oracle):
    """MultiHeadAttention = 4 Linear + SDPA: the oracle's pieces composed must
    reproduce the reference module's output and every gradient."""
    g = load("mha_causal")
    x, dy = g["x"], g["dy"]
    b, t, e = x.shape
    heads = int(g["heads"])
    dh = e // heads
    x2 = x.reshape(b * t, e)
    proj = {}
    for n in "qkv":
        proj[n] = oracle.linear_fwd(x2, g["w" + n], g["b" + n])
    to_heads = lambda a: np.ascontiguousarray(a.reshape(b, t, heads, dh).transpose(0, 2, 1, 3))
    from_heads = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3).reshape(b * t, e))
    d = AttnDesc(b, heads, t, t, dh, 1, 0, 1.0 / np.sqrt(dh))
    qh, kh, vh = (to_heads(proj[n]) for n in "qkv")
    o, _ = oracle.attention_fwd(d, qh, kh, vh)
    a = from_heads(o)
    y = oracle.linear_fwd(a, g["wo"], g["bo"])
    close(y.reshape(b, t, e), g["y"])
    da, dwo, dbo = oracle.linear_bwd(dy.reshape(b * t, e), a, g["wo"])
    close(dwo, g["dwo"])
    close(dbo, g["dbo"])
    dq, dk, dv = oracle.attention_bwd(d, qh, kh, vh, o, to_heads(da))
    dx = np.zeros((b * t, e), np.float64)
    for n, dd in zip("qkv", (dq, dk, dv)):
        dxn, dwn, dbn = oracle.linear_bwd(from_heads(dd), x2, g["w" + n])
        close(dwn, g["dw" + n])
        close(dbn, g["db" + n])
        dx += dxn
    close(dx.reshape(b, t, e), g["dx"])


# -------------------------------------------------- independent math checks
def test_conv_adjoint_identities(oracle):
    """<conv(x,w), dy> = <x, dgrad(dy,w)> = <w, wgrad(x,dy)> for strided,
    padded, dilated shapes: fixes the index maps of both backward passes."""
    g = rng(11)
    for (n, c, h, w, k, r, s, st, pd, dl) in ((2, 3, 8, 9, 4, 3, 3, (1, 1), (1, 1), (1, 1)),
                                              (1, 2, 11, 10, 3, 5, 3, (2, 3), (2, 1), (1, 2)),
                                              (2, 2, 7, 7, 2, 1, 1, (2, 2), (0, 0), (1, 1))):
        d = Conv2dDesc(n, c, h, w, k, r, s, st[0], st[1], pd[0], pd[1], dl[0], dl[1], 1, 0, 0)
        x = f32(g.standard_normal((n, c, h, w)))
        wt = f32(g.standard_normal((k, c, r, s)))
        y = oracle.conv2d_fwd(d, x, wt)
        dy = f32(g.standard_normal(y.shape))
        lhs = np.dot(y.ravel().astype(np.float64), dy.ravel())
        dx = oracle.conv2d_bwd_data(d, dy, wt)
        dw, db = oracle.conv2d_bwd_weight(d, x, dy)
        assert abs(lhs - np.dot(x.ravel().astype(np.float64), dx.ravel())) <= 1e-4 * (abs(lhs) + 1)
        assert abs(lhs - np.dot(wt.ravel().astype(np.float64), dw.ravel())) <= 1e-4 * (abs(lhs) + 1)
        close(db, dy.sum(axis=(0, 2, 3)), rtol=1e-5, atol=1e-5)


def test_conv_forward_matches_sliding_window(oracle):
    """Forward against an independent numpy sliding-window correlation."""
    g = rng(12)
    n, c, h, w, k = 2, 3, 7, 6, 4
    d = Conv2dDesc(n, c, h, w, k, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0, 0)
    x = f32(g.standard_normal((n, c, h, w)))
    wt = f32(g.standard_normal((k, c, 3, 3)))
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    win = np.lib.stride_tricks.sliding_window_view(xp, (3, 3), axis=(2, 3))  # n c h w 3 3
    ref = np.einsum("nchwrs,kcrs->nkhw", win, wt.astype(np.float64))
    close(oracle.conv2d_fwd(d, x, wt), ref)


def test_linear_matches_matmul(oracle):
    g = rng(13)
    x, w, dy = (f32(g.standard_normal(s)) for s in ((6, 5), (4, 5), (6, 4)))
    dx, dw, db = oracle.linear_bwd(dy, x, w)
    close(dx, dy.astype(np.float64) @ w)
    close(dw, dy.T.astype(np.float64) @ x)
    close(db, dy.sum(0))


def test_batchnorm_invariants(oracle):
    g = rng(14)
    x = f32(g.standard_normal((4, 3, 6, 6)) * 3 + 1)
    gamma, beta = f32(g.standard_normal(3)), f32(g.standard_normal(3))
    y, mean, rstd, _, _ = oracle.batchnorm2d_fwd(x, gamma, beta)
    yn = (y - beta[None, :, None, None]) / gamma[None, :, None, None]
    close(yn.mean(axis=(0, 2, 3)), np.zeros(3), atol=1e-5)
    close(yn.var(axis=(0, 2, 3)), np.ones(3), rtol=1e-3)
    dy = f32(g.standard_normal(x.shape))
    dx, dg, db = oracle.batchnorm2d_bwd(x, dy, mean, rstd, gamma)
    xh = (x - mean[None, :, None, None]) * rstd[None, :, None, None]
    close(dx.sum(axis=(0, 2, 3)), np.zeros(3), atol=1e-4)
    close((dx * xh).sum(axis=(0, 2, 3)), np.zeros(3), atol=1e-3)
    close(db, dy.sum(axis=(0, 2, 3)), atol=1e-5)


def test_layernorm_invariants_and_fd(oracle):
    g = rng(15)
    x = f32(g.standard_normal((3, 12)))
    gamma, beta = f32(1 + 0.2 * g.standard_normal(12)), f32(g.standard_normal(12))
    dy = f32(g.standard_normal(x.shape))
    y, mean, rstd = oracle.layernorm_fwd(x, gamma, beta)
    dx, dg, db = oracle.layernorm_bwd(x, dy, mean, rstd, gamma)
    close(dx.sum(1), np.zeros(3), atol=1e-5)
    # central finite difference of L = <LN(x), dy> in float64
    def L(xx):
        xx = xx.astype(np.float64)
        mu = xx.mean(1, keepdims=True)
        var = ((xx - mu) ** 2).mean(1, keepdims=True)
        return (((xx - mu) / np.sqrt(var + 1e-5) * gamma + beta) * dy).sum()
    h = 1e-4
    for (i, j) in ((0, 0), (1, 5), (2, 11)):
        xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
        xp[i, j] += h
        xm[i, j] -= h
        assert abs((L(xp) - L(xm)) / (2 * h) - dx[i, j]) < 2e-3


def test_xent_invariants_and_fd(oracle):
    g = rng(16)
    z = f32(g.standard_normal((5, 7)) * 2)
    y = np.array([0, 6, 3, -100, 2], np.int64)
    for eps in (0.0, 0.2):
        dz, loss = oracle.softmax_xent(z, y, eps)
        close(dz.sum(1), np.zeros(5), atol=1e-6)
        assert np.all(dz[3] == 0)  # ignored row
        def L(zz):
            zz = zz.astype(np.float64)
            lse = np.log(np.exp(zz - zz.max(1, keepdims=True)).sum(1)) + zz.max(1)
            logp = zz - lse[:, None]
            valid = y != -100
            nll = -logp[valid, y[valid]]
            smooth = -logp[valid].sum(1)
            return ((1 - eps) * nll + eps / zz.shape[1] * smooth).sum() / valid.sum()
        assert abs(L(z) - loss) < 1e-5
        h = 1e-4
        for (i, j) in ((0, 0), (1, 6), (4, 3)):
            zp, zm = z.astype(np.float64).copy(), z.astype(np.float64).copy()
            zp[i, j] += h
            zm[i, j] -= h
            assert abs((L(zp) - L(zm)) / (2 * h) - dz[i, j]) < 1e-5


def test_adam_step1_closed_form(oracle):
    """At t = 1 with zero moments m̂ = g and v̂ = g², so Adam moves every
    parameter by lr·g/(|g| + eps) (Kingma & Ba, Alg. 1)."""
    g = rng(17)
    p = f32(g.standard_normal(100))
    gr = f32(g.standard_normal(100) * 1e-2)
    z = np.zeros(100, np.float32)
    lr, eps = 1e-3, 1e-8
    p2, m2, v2 = oracle.adam_step(0, p, gr, z, z, lr, 0.9, 0.999, eps, 0.0, 1)
    close(p2, p - lr * gr / (np.abs(gr) + eps), rtol=1e-5, atol=1e-7)
    close(m2, 0.1 * gr, rtol=1e-6, atol=0)
    # AdamW with wd: p first shrinks by (1 - lr*wd), then the same move.
    p3, _, _ = oracle.adam_step(1, p, gr, z, z, lr, 0.9, 0.999, eps, 0.1, 1)
    close(p3, p * (1 - lr * 0.1) - lr * gr / (np.abs(gr) + eps), rtol=1e-5, atol=1e-7)


def test_attention_fd_and_causal_row0(oracle):
    g = rng(18)
    d = AttnDesc(1, 1, 4, 4, 3, 1, 0, 1 / np.sqrt(3))
    q, k, v, dO = (f32(g.standard_normal((1, 1, 4, 3))) for _ in range(4))
    o, lse = oracle.attention_fwd(d, q, k, v)
    close(o[0, 0, 0], v[0, 0, 0])  # first query only sees key 0
    dq, dk, dv = oracle.attention_bwd(d, q, k, v, o, dO)
    def L(qq, kk, vv):
        s = (qq[0, 0].astype(np.float64) @ kk[0, 0].T.astype(np.float64)) / np.sqrt(3)
        s = np.where(np.triu(np.ones((4, 4)), 1) > 0, -np.inf, s)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        return ((p @ vv[0, 0].astype(np.float64)) * dO[0, 0]).sum()
    h = 1e-4
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        for idx in ((0, 0, 1, 2), (0, 0, 3, 0)):
            ap, am = arr.astype(np.float64).copy(), arr.astype(np.float64).copy()
            ap[idx] += h
            am[idx] -= h
            args_p = [ap if a is arr else a for a in (q, k, v)]
            args_m = [am if a is arr else a for a in (q, k, v)]
            assert abs((L(*args_p) - L(*args_m)) / (2 * h) - grad[idx]) < 1e-4


def test_maxpool_argmax_points_at_max(oracle):
    g = rng(19)
    x = f32(np.round(g.standard_normal((2, 3, 9, 9)), 1))  # rounding creates ties
    d = Pool2dDesc(2, 3, 9, 9, 3, 3, 2, 2, 1, 1, 1, 1, 0, 0)
    y, idx = oracle.maxpool2d_fwd(d, x)
    flat = x.reshape(6, 81)
    assert np.array_equal(np.take_along_axis(flat, idx.reshape(6, -1), 1).reshape(y.shape), y)
    dy = f32(g.standard_normal(y.shape))
    dx = oracle.maxpool2d_bwd(d, idx, dy)
    close(dx.sum(), dy.sum(), rtol=1e-5)  # routing conserves the total gradient


# ------------------------------------------------ against the reference build
def test_random_cases_against_reference(oracle, ref):
    g = rng(21)
    d = Conv2dDesc(2, 5, 10, 9, 6, 3, 3, 2, 1, 1, 1, 1, 1, 1, 0, 0)
    x = f32(g.standard_normal((2, 5, 10, 9)))
    w = f32(g.standard_normal((6, 5, 3, 3)))
    b = f32(g.standard_normal(6))
    y0 = oracle.conv2d_fwd(d, x, w, b)
    dy = f32(g.standard_normal(y0.shape))
    y, dx, dw, db = ref.conv2d(d, x, w, b, dy)
    close(y0, y)
    close(oracle.conv2d_bwd_data(d, dy, w), dx)
    dw0, db0 = oracle.conv2d_bwd_weight(d, x, dy)
    close(dw0, dw)
    close(db0, db)
    z = f32(g.standard_normal((16, 33)) * 3)
    lab = g.integers(0, 33, 16).astype(np.int64)
    dl, loss = ref.cross_entropy(z, lab, 0.05)
    dl0, loss0 = oracle.softmax_xent(z, lab, 0.05)
    close(dl0, dl)
    close(loss0, loss)


# ------------------------------------------------- bf16 rounding, pinned
def _bf16_specials():
    """Random values over the whole fp32 range plus the cases rounding gets
    wrong: exact ties (even and odd lower halves), values just above and below
    a tie, ±0, ±inf, quiet and signalling NaNs of both signs, fp32 subnormals,
    the largest finite values (which round to inf) and carries into the
    exponent."""
    g = rng(404)
    u = g.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    base = g.integers(0, 2 ** 16, 2000, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001, base | 0xFFFF, base | 0x0001])
    special = np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001,
                        0xFF800001, 0x7FBFFFFF, 0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF, 0x00008000,
                        0x00018000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x3F7FFFFF, 0x3F7F8000,
                        0x3F808000, 0x3F818000], np.uint32)
    return np.concatenate([u, ties, special]).view(np.float32)


def test_round_bf16_matches_torch(oracle):
    """round_bf16 (tests) and oracle_round_bf16 (oracle.c), which give the
    oracle the values a bf16 path computes with, agree bit for bit with
    torch's CPU float32 -> bfloat16 conversion (round to nearest even) on
    every finite value and infinity, and keep NaN as NaN of the same sign."""
    import torch
    x = _bf16_specials()
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).to(torch.float32).numpy()
    got_py = round_bf16(x)
    got_c = oracle.round_bf16(x)
    for got in (got_py, got_c):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
        assert np.array_equal(np.signbit(got[nan]), np.signbit(x[nan]))
