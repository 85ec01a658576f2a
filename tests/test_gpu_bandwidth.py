"""GPU parity of the bandwidth-bound kernels against the CPU oracle, through
the C ABI (thot_amd.ops -> libnott_hip.so).  Same seeded inputs on both sides;
bf16 inputs are rounded once and the oracle sees the rounded values."""
import numpy as np
import pytest
import torch

from gpu_util import check, dev, host, host_input
from oracle_lib import f32, rng

pytestmark = pytest.mark.gpu

DTYPES = ["f32", "bf16"]


@pytest.fixture(scope="module")
def ops():
    from thot_amd import ops as _ops
    assert torch.cuda.is_available()
    return _ops


# ------------------------------------------------------------------ adam
@pytest.mark.parametrize("decoupled,wd,step", [(1, 0.01, 10), (0, 0.0, 1), (0, 0.01, 3), (1, 0.0, 2)])
@pytest.mark.parametrize("n", [1, 7, 4096 + 3, 1 << 20])
def test_adam_fp32_bit_exact(ops, oracle, decoupled, wd, step, n):
    g = rng(1000 + n + step)
    p = f32(g.standard_normal(n) * 0.02)
    gr = f32(g.standard_normal(n) * 1e-3)
    m = f32(g.standard_normal(n) * 1e-4) if step > 1 else np.zeros(n, np.float32)
    v = f32(np.abs(g.standard_normal(n)) * 1e-7) if step > 1 else np.zeros(n, np.float32)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=wd)
    pd, gd, md, vd = dev(p), dev(gr), dev(m), dev(v)
    ops.adam_step(pd, gd, md, vd, step=step, decoupled=bool(decoupled), **hp)
    pe, me, ve = oracle.adam_step(decoupled, p, gr, m, v, hp["lr"], hp["beta1"], hp["beta2"], hp["eps"], wd, step)
    # identical fp32 operation order: bit-exact
    assert np.array_equal(host(pd).view(np.int32), pe.view(np.int32))
    assert np.array_equal(host(md).view(np.int32), me.view(np.int32))
    assert np.array_equal(host(vd).view(np.int32), ve.view(np.int32))


def test_adam_unaligned_and_zero_grad(ops, oracle):
    g = rng(5)
    n = 1001
    base = [torch.zeros(n + 1, device="cuda") for _ in range(4)]
    p, gr, m, v = (b[1:] for b in base)  # 4-byte offset: scalar path
    p.copy_(dev(f32(g.standard_normal(n))))
    gr.copy_(dev(f32(g.standard_normal(n) * 1e-2)))
    pe, me, ve = oracle.adam_step(1, host(p), host(gr), host(m), host(v), 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
    ops.adam_step(p, gr, m, v, lr=1e-3, weight_decay=0.01, step=1, decoupled=True, zero_grad=True)
    assert np.array_equal(host(p), pe) and np.array_equal(host(m), me) and np.array_equal(host(v), ve)
    assert torch.count_nonzero(gr).item() == 0


def test_adam_bf16_params(ops, oracle):
    g = rng(6)
    n = 100003
    p = host_input(g.standard_normal(n) * 0.02, "bf16")
    gr = host_input(g.standard_normal(n) * 1e-3, "bf16")
    m = f32(g.standard_normal(n) * 1e-4)
    v = f32(np.abs(g.standard_normal(n)) * 1e-7)
    pd, gd, md, vd = dev(p, "bf16"), dev(gr, "bf16"), dev(m), dev(v)
    ops.adam_step(pd, gd, md, vd, lr=3e-4, weight_decay=0.01, step=10, decoupled=True)
    pe, me, ve = oracle.adam_step(1, p, gr, m, v, 3e-4, 0.9, 0.999, 1e-8, 0.01, 10)
    # moments are fp32 and see exactly the same inputs: bit-exact
    assert np.array_equal(host(md), me) and np.array_equal(host(vd), ve)
    # p is rounded to bf16 once at the end
    assert np.array_equal(host(pd), host_input(pe, "bf16"))


def test_adam_rejects_bad_arguments(ops):
    from thot_amd._abi import NottInvalidArgument
    p = torch.zeros(8, device="cuda")
    with pytest.raises(NottInvalidArgument):
        ops.adam_step(p, p.clone(), p.clone(), p.clone(), lr=1e-3, step=0, decoupled=True)
    with pytest.raises(NottInvalidArgument):
        ops.adam_step(p, p.clone(), p.clone(), p.clone(), lr=1e-3, beta1=1.0, step=1, decoupled=True)


# ------------------------------------------------------------------ relu
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1, 5, 64 * 1000 + 3])
def test_relu(ops, oracle, dt, n):
    g = rng(n)
    x = host_input(g.standard_normal(n), dt)
    x[:: 5] = 0.0
    if n > 4:
        x[3] = np.nan
    dy = host_input(g.standard_normal(n), dt)
    y = ops.relu_fwd(dev(x, dt))
    ye = oracle.relu_fwd(x)
    assert np.array_equal(np.isnan(host(y)), np.isnan(ye))
    check(host(y), ye, dt, "relu y", rtol=0, atol=0)
    dx = ops.relu_bwd(y, dev(dy, dt))
    check(host(dx), oracle.relu_bwd(ye, dy), dt, "relu dx", rtol=0, atol=0)


@pytest.mark.parametrize("dt", DTYPES)
def test_add_cast_zero(ops, dt):
    g = rng(9)
    a, b = host_input(g.standard_normal(1003), dt), host_input(g.standard_normal(1003), dt)
    out = ops.add(dev(a, dt), dev(b, dt))
    check(host(out), host_input(a + b, dt), dt, "add", rtol=0, atol=0)
    x = f32(g.standard_normal(999))
    xb = ops.cast(dev(x), torch.bfloat16)
    assert np.array_equal(host(xb), host_input(x, "bf16"))
    t = dev(x)
    ops.zero_(t)
    assert torch.count_nonzero(t).item() == 0


# ----------------------------------------------------------------- pools
POOLS = [
    # n, c, h, w, k, stride, pad, dil, ceil
    (64, 32, 28, 28, (2, 2), (2, 2), (0, 0), (1, 1), False),   # small CNN pool 1
    (64, 64, 14, 14, (2, 2), (2, 2), (0, 0), (1, 1), False),   # small CNN pool 2
    (4, 64, 112, 112, (3, 3), (2, 2), (1, 1), (1, 1), False),  # ResNet-18 stem pool (batch slice)
    (2, 3, 9, 8, (3, 3), (2, 2), (0, 0), (1, 1), True),
    (2, 3, 9, 9, (2, 2), (1, 1), (0, 0), (2, 2), False),
    (2, 3, 17, 23, (3, 3), (2, 2), (1, 1), (1, 1), True),     # row bands cut mid-window, ceil mode
    (1, 2, 40, 33, (5, 4), (3, 2), (2, 1), (1, 2), False),    # dilation with padding
    (3, 5, 70, 19, (3, 3), (1, 1), (1, 1), (1, 1), False),    # stride 1: several bands per plane
    # rows of whole 4-element groups (the 4-wide path)
    (2, 3, 24, 16, (3, 3), (1, 1), (1, 1), (1, 1), False),
    (3, 4, 16, 16, (2, 2), (2, 2), (0, 0), (1, 1), False),
    (2, 5, 40, 64, (3, 3), (2, 2), (1, 1), (1, 1), False),
    # stride-2 kernels: odd height (last window cut by the image edge), several
    # 32-row bands, 2x2 windows over several bands, wide rows
    (2, 3, 35, 8, (3, 3), (2, 2), (1, 1), (1, 1), False),
    (1, 2, 66, 24, (2, 2), (2, 2), (0, 0), (1, 1), False),
    (1, 3, 23, 256, (3, 3), (2, 2), (1, 1), (1, 1), False),
]


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", POOLS)
def test_maxpool(ops, oracle, dt, case):
    n, c, h, w, k, st, pd, dl, ceil = case
    g = rng(h * w + c)
    x = g.standard_normal((n, c, h, w))
    x = np.maximum(x, 0.0)  # post-ReLU ties, as in the reference's small CNN
    x = host_input(x, dt)
    d = ops.pool_desc((n, c, h, w), k, st, pd, dl, ceil)
    y, idx = ops.maxpool2d_fwd(dev(x, dt), d)
    ye, idxe = oracle.maxpool2d_fwd(d, x)
    assert np.array_equal(host(idx).astype(np.int64) if idx.dtype != torch.int64 else idx.cpu().numpy(), idxe), \
        "argmax routing must be bit-exact"
    check(host(y), ye, dt, "maxpool y", rtol=0, atol=0)
    dy = host_input(g.standard_normal(ye.shape), dt)
    dx = ops.maxpool2d_bwd(idx, dev(dy, dt), d)
    check(host(dx), oracle.maxpool2d_bwd(d, idxe, dy), dt, "maxpool dx")


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", POOLS)
def test_maxpool_tap(ops, oracle, dt, case):
    """The one-byte window-tap argmax (nott_maxpool2d_*_tap) names the same
    inputs as the int64 flat index, and y / dx are bit-identical to the int64
    pair's, NaN and -inf windows included."""
    n, c, h, w, k, st, pd, dl, ceil = case
    g = rng(h * w + c + 1)
    x = np.maximum(g.standard_normal((n, c, h, w)), 0.0)
    flat = x.reshape(-1)
    flat[g.integers(0, flat.size, max(1, flat.size // 97))] = np.nan
    flat[g.integers(0, flat.size, max(1, flat.size // 89))] = -np.inf
    x = host_input(x, dt)
    d = ops.pool_desc((n, c, h, w), k, st, pd, dl, ceil)
    y, idx = ops.maxpool2d_fwd(dev(x, dt), d)
    yt, tap = ops.maxpool2d_fwd_tap(dev(x, dt), d)
    assert tap.dtype == torch.uint8
    ye, idxe = oracle.maxpool2d_fwd(d, x)
    assert np.array_equal(idx.cpu().numpy(), idxe), "argmax routing must be bit-exact (NaN / -inf windows)"
    assert np.array_equal(host(y), ye, equal_nan=True)
    assert torch.equal(y.view(torch.int16 if dt == "bf16" else torch.int32),
                       yt.view(torch.int16 if dt == "bf16" else torch.int32))
    oh, ow = y.shape[2], y.shape[3]
    t = tap.cpu().numpy().astype(np.int64)
    ohg = np.arange(oh).reshape(1, 1, oh, 1)
    owg = np.arange(ow).reshape(1, 1, 1, ow)
    decoded = (ohg * st[0] - pd[0] + (t // k[1]) * dl[0]) * w + (owg * st[1] - pd[1] + (t % k[1]) * dl[1])
    assert np.array_equal(decoded, idx.cpu().numpy()), "tap and flat index must name the same input"
    dy = dev(host_input(g.standard_normal(y.shape), dt), dt)
    dx = ops.maxpool2d_bwd(idx, dy, d)
    dxt = ops.maxpool2d_bwd_tap(tap, dy, d)
    check(host(dx), oracle.maxpool2d_bwd(d, idxe, host(dy)), dt, "maxpool dx")
    assert torch.equal(dx.view(torch.int16 if dt == "bf16" else torch.int32),
                       dxt.view(torch.int16 if dt == "bf16" else torch.int32))
    # through the ReLU that produced the pool's input (zeros, NaN and -inf
    # included): bit-identical to the pool backward then the ReLU backward
    xd = dev(x, dt)
    dxr = ops.maxpool2d_bwd_tap(tap, dy, d, relu_y=xd)
    ref = ops.relu_bwd(xd, dxt)
    assert torch.equal(dxr.view(torch.int16 if dt == "bf16" else torch.int32),
                       ref.view(torch.int16 if dt == "bf16" else torch.int32))


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n,offset", [(64 * 64 * 56 * 56, 0), (1000003, 0), (4099, 1)])
def test_add_relu_bwd(ops, dt, n, offset):
    """The fork gradient of a ReLU output, (y <= 0) ? 0 : a + b, against the
    two passes, bit for bit (zeros, NaN and -inf in y; an odd length and an
    unaligned start take the tail and two-pass paths)."""
    g = rng(n % 1000 + offset)
    mk = lambda: dev(host_input(g.standard_normal(n + offset), dt), dt)[offset:]
    a, b, y = mk(), mk(), ops.relu_fwd(mk())
    yh = y.view(-1)
    yh[::97] = float("nan")
    yh[::89] = float("-inf")
    iv = torch.int16 if dt == "bf16" else torch.int32
    dz = ops.add_relu_bwd(a, b, y)
    ref = ops.relu_bwd(y, ops.add(a, b))
    assert torch.equal(dz.view(iv), ref.view(iv))


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", [(4, 64, 112, 112, 3, 1), (3, 16, 30, 24, 3, 1), (2, 8, 17, 20, 2, 0)])
def test_batchnorm_relu_maxpool_fused(ops, dt, case):
    """The stem's BatchNorm + ReLU + max-pool with the BatchNorm's output never
    stored: pooled values, taps, mean, rstd and running stats bit-identical
    to the fused-ReLU BatchNorm followed by the pool."""
    n, c, h, w, k, pd = case
    g = rng(n * c + h + w)
    x = dev(host_input(g.standard_normal((n, c, h, w)) * 2 + 0.5, dt), dt)
    gamma = dev(f32(g.standard_normal(c)))
    beta = dev(f32(g.standard_normal(c)))
    d = ops.pool_desc((n, c, h, w), (k, k), (2, 2), (pd, pd), (1, 1), False)
    rm1, rv1 = torch.zeros(c, device="cuda"), torch.ones(c, device="cuda")
    rm2, rv2 = rm1.clone(), rv1.clone()
    yb, m1, r1 = ops.batchnorm2d_fwd(x, gamma, beta, running_mean=rm1, running_var=rv1, relu=True)
    yp, tap = ops.maxpool2d_fwd_tap(yb, d)
    y2, tap2, m2, r2 = ops.batchnorm2d_relu_maxpool2d_fwd(x, gamma, beta, d, running_mean=rm2, running_var=rv2)
    iv = torch.int16 if dt == "bf16" else torch.int32
    assert torch.equal(yp.view(iv), y2.view(iv))
    assert torch.equal(tap, tap2)
    for u, v in ((m1, m2), (r1, r2), (rm1, rm2), (rv1, rv2)):
        assert torch.equal(u, v)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("case", [(4, 64, 112, 112, 3, 1), (3, 16, 30, 24, 3, 1), (5, 8, 12, 16, 2, 0),
                                  (2, 8, 17, 20, 2, 0)])
def test_batchnorm_relu_maxpool_bwd_fused(ops, dt, case):
    """The stem's backward with the routed gradient never stored, against the
    pool's backward followed by the BatchNorm + ReLU backward.  The fused
    sums take each routed term before it is rounded, so dγ and dβ agree to
    2^-7 (bf16) or 1e-5 (fp32) of Σ|term| and dx to the same fraction of its
    largest magnitude; shapes outside the stride-2 kernels (the last case:
    10-wide output rows) run the two calls and match bit for bit."""
    n, c, h, w, k, pd = case
    g = rng(n * c + h + w + 7)
    x = dev(host_input(g.standard_normal((n, c, h, w)) * 2 + 0.5, dt), dt)
    gamma = dev(f32(g.standard_normal(c)))
    beta = dev(f32(g.standard_normal(c)))
    d = ops.pool_desc((n, c, h, w), (k, k), (2, 2), (pd, pd), (1, 1), False)
    y, tap, mean, rstd = ops.batchnorm2d_relu_maxpool2d_fwd(x, gamma, beta, d)
    dy = dev(host_input(g.standard_normal(tuple(y.shape)), dt), dt)
    dz = ops.maxpool2d_bwd_tap(tap, dy, d)
    dx1, dg1, db1 = ops.batchnorm2d_bwd(x, dz, mean, rstd, gamma, beta=beta, relu=True)
    dx2, dg2, db2 = ops.batchnorm2d_relu_maxpool2d_bwd(x, tap, dy, d, mean, rstd, gamma, beta)
    _, dg3, db3 = ops.batchnorm2d_relu_maxpool2d_bwd(x, tap, dy, d, mean, rstd, gamma, beta, need_dx=False)
    assert torch.equal(dg2, dg3) and torch.equal(db2, db3)
    fused = (w % 4 == 0) and ((w + 2 * pd - k) // 2 + 1) % 4 == 0
    if not fused:
        iv = torch.int16 if dt == "bf16" else torch.int32
        assert torch.equal(dx1.view(iv), dx2.view(iv))
        assert torch.equal(dg1, dg2) and torch.equal(db1, db2)
    else:
        tol = 2.0 ** -7 if dt == "bf16" else 1e-5
        gz = dz.float() * ((x.float() * (gamma * rstd).view(1, c, 1, 1)
                            + (beta - mean * gamma * rstd).view(1, c, 1, 1)) > 0)
        xh = (x.float() - mean.view(1, c, 1, 1)) * rstd.view(1, c, 1, 1)
        sb = gz.abs().sum((0, 2, 3))
        sg = (gz * xh).abs().sum((0, 2, 3))
        assert ((db1 - db2).abs() <= tol * sb + 1e-6).all()
        assert ((dg1 - dg2).abs() <= tol * sg + 1e-6).all()
        scale = dx1.float().abs().max()
        assert ((dx1.float() - dx2.float()).abs() <= tol * scale).all()
    # accumulate adds into the given buffers
    dg4, db4 = dg2.clone(), db2.clone()
    ops.batchnorm2d_relu_maxpool2d_bwd(x, tap, dy, d, mean, rstd, gamma, beta, dgamma=dg4, dbeta=db4, accumulate=True)
    torch.testing.assert_close(dg4, 2 * dg2, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(db4, 2 * db2, rtol=1e-6, atol=1e-6)


MAXPOOL_GOLDEN = ["maxpool2x2_s2_relu_ties", "maxpool3x3_s2p1_overlap", "maxpool3x3_s2_ceil", "maxpool2x2_dil2",
                  "maxpool3x3_s2p1_nan_inf", "maxpool2x2_s2_nan_inf"]


@pytest.mark.parametrize("name", MAXPOOL_GOLDEN)
def test_maxpool_golden(ops, name):
    """Both GPU max-pool paths (int64 flat index and one-byte tap) against the
    fixtures the reference's MaxPool2d wrote (pooling.hpp:132-149), all-NaN,
    all--inf and mixed non-finite windows included: argmax and y bit-exact,
    dx within fp32 tolerance."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name + ".npz"))
    n, c, h, w, kh, kw, sh, sw, ph, pw, dh, dw, ceil = (int(v) for v in z["desc"])
    d = ops.pool_desc((n, c, h, w), (kh, kw), (sh, sw), (ph, pw), (dh, dw), bool(ceil))
    x = dev(z["x"])
    y, idx = ops.maxpool2d_fwd(x, d)
    yt, tap = ops.maxpool2d_fwd_tap(x, d)
    assert np.array_equal(idx.cpu().numpy(), z["argmax"]), "argmax routing differs from the reference's"
    assert np.array_equal(host(y), z["y"], equal_nan=True)
    assert torch.equal(y.view(torch.int32), yt.view(torch.int32))
    dy = dev(z["dy"])
    dx = ops.maxpool2d_bwd(idx, dy, d)
    dxt = ops.maxpool2d_bwd_tap(tap, dy, d)
    check(host(dx), z["dx"], "f32", "golden maxpool dx")
    assert torch.equal(dx.view(torch.int32), dxt.view(torch.int32))


def test_maxpool_tap_rejects_large_windows(ops):
    d = ops.pool_desc((1, 1, 40, 40), (17, 17), (1, 1), (0, 0), (1, 1), False)
    with pytest.raises(RuntimeError, match="256 taps"):
        ops.maxpool2d_fwd_tap(torch.zeros((1, 1, 40, 40), device="cuda"), d)


@pytest.mark.parametrize("dt", DTYPES)
def test_avgpool_global(ops, oracle, dt):
    g = rng(77)
    x = host_input(g.standard_normal((64, 512, 7, 7)), dt)
    y = ops.avgpool_global_fwd(dev(x, dt))
    check(host(y), oracle.avgpool_global_fwd(x), dt, "avgpool y")
    dy = host_input(g.standard_normal((64, 512, 1, 1)), dt)
    dx = ops.avgpool_global_bwd(dev(dy, dt), (7, 7))
    check(host(dx), oracle.avgpool_global_bwd(dy, (7, 7)), dt, "avgpool dx")


# -------------------------------------------------------------- batchnorm
BN_SHAPES = [(64, 64, 56, 56), (64, 512, 7, 7), (3, 5, 4, 3)]


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", BN_SHAPES)
def test_batchnorm(ops, oracle, dt, shape):
    n, c, h, w = shape
    g = rng(n * c + h)
    x = host_input(g.standard_normal(shape) * 1.5 + 0.3, dt)
    gamma = f32(1 + 0.1 * g.standard_normal(c))
    beta = f32(0.1 * g.standard_normal(c))
    rm, rv = f32(np.zeros(c)), f32(np.ones(c))
    rmd, rvd = dev(rm), dev(rv)
    y, mean, rstd = ops.batchnorm2d_fwd(dev(x, dt), dev(gamma), dev(beta), 1e-5, 0.1, rmd, rvd)
    ye, me, re_, rme, rve = oracle.batchnorm2d_fwd(x, gamma, beta, 1e-5, 0.1, rm, rv)
    check(host(mean), me, "f32", "bn mean", atol=1e-5)
    check(host(rstd), re_, "f32", "bn rstd")
    check(host(y), ye, dt, "bn y")
    check(host(rmd), rme, "f32", "bn running_mean", atol=1e-5)
    check(host(rvd), rve, "f32", "bn running_var")
    dy = host_input(g.standard_normal(shape), dt)
    dx, dg, db = ops.batchnorm2d_bwd(dev(x, dt), dev(dy, dt), mean, rstd, dev(gamma))
    dxe, dge, dbe = oracle.batchnorm2d_bwd(x, dy, host(mean), host(rstd), gamma)
    check(host(dx), dxe, dt, "bn dx")
    check(host(dg), dge, "f32", "bn dgamma")
    check(host(db), dbe, "f32", "bn dbeta")


@pytest.mark.parametrize("dt", DTYPES)
def test_batchnorm_bwd_params_only(ops, dt):
    """With no dx requested the backward still writes dgamma / dbeta (its own
    finalize pass), bit-identical to the full backward's, and accumulates."""
    from thot_amd.ops import _ctx_for, _ptr, nott_dtype
    n, c, h, w = 8, 24, 9, 12
    g = rng(321)
    x = dev(host_input(g.standard_normal((n, c, h, w)), dt), dt)
    dy = dev(host_input(g.standard_normal((n, c, h, w)), dt), dt)
    gamma = dev(f32(1 + 0.1 * g.standard_normal(c)))
    _, mean, rstd = ops.batchnorm2d_fwd(x, gamma, dev(f32(np.zeros(c))), 1e-5, 0.1)
    _, dg, db = ops.batchnorm2d_bwd(x, dy, mean, rstd, gamma)
    dg2 = torch.full((c,), 0.5, device="cuda")
    db2 = torch.full((c,), -0.25, device="cuda")
    _ctx_for(x).call("nott_batchnorm2d_bwd", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(dy), _ptr(mean),
                     _ptr(rstd), _ptr(gamma), None, _ptr(dg2), _ptr(db2), 1)
    assert torch.equal(dg2, dg + 0.5) and torch.equal(db2, db - 0.25)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", BN_SHAPES)
@pytest.mark.parametrize("with_res", [False, True])
def test_batchnorm_act(ops, oracle, dt, shape, with_res):
    """nott_batchnorm2d_fwd_act / _bwd_act against the composition the
    reference runs: BatchNorm2d, then (+ skip) ReLU (residual.hpp:94-96,
    130-132); the backward through the ReLU masks dy where BN(x) <= 0."""
    n, c, h, w = shape
    g = rng(n * c + h + 7)
    x = host_input(g.standard_normal(shape) * 1.5 + 0.3, dt)
    gamma = f32(1 + 0.1 * g.standard_normal(c))
    beta = f32(0.1 * g.standard_normal(c))
    res = host_input(g.standard_normal(shape), dt) if with_res else None
    y, mean, rstd = ops.batchnorm2d_fwd(dev(x, dt), dev(gamma), dev(beta), 1e-5, 0.1,
                                        residual=dev(res, dt) if with_res else None, relu=True)
    ye, me, re_, _, _ = oracle.batchnorm2d_fwd(x, gamma, beta, 1e-5, 0.1, f32(np.zeros(c)), f32(np.ones(c)))
    check(host(mean), me, "f32", "bn mean", atol=1e-5)
    ya = ye + (res if with_res else 0.0)
    check(host(y), np.maximum(ya, 0.0), dt, "bn+relu y")
    if with_res:
        return                       # the residual block's backward goes through relu_bwd + BN backward
    dy = host_input(g.standard_normal(shape), dt)
    dx, dg, db = ops.batchnorm2d_bwd(dev(x, dt), dev(dy, dt), mean, rstd, dev(gamma), beta=dev(beta), relu=True)
    # mask from this run's statistics (a flip needs |BN(x)| below fp32 rounding)
    mh, rh = host(mean).astype(np.float64), host(rstd).astype(np.float64)
    z = (x.astype(np.float64) - mh[None, :, None, None]) * rh[None, :, None, None] * gamma[None, :, None, None] \
        + beta[None, :, None, None]
    dym = np.where(z > 0, dy, 0.0).astype(np.float32)
    dxe, dge, dbe = oracle.batchnorm2d_bwd(x, dym, host(mean), host(rstd), gamma)
    check(host(dx), dxe, dt, "bn+relu dx")
    check(host(dg), dge, "f32", "bn+relu dgamma")
    check(host(db), dbe, "f32", "bn+relu dbeta")


# -------------------------------------------------------------- layernorm
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("rows,d", [(2048, 1024), (37, 256), (5, 1000), (3, 3000), (64, 4), (4099, 512), (257, 2048),
                                    (1029, 64)])
def test_layernorm(ops, oracle, dt, rows, d):
    g = rng(rows + d)
    x = host_input(g.standard_normal((rows, d)), dt)
    gamma = host_input(1 + 0.1 * g.standard_normal(d), dt)
    beta = host_input(0.1 * g.standard_normal(d), dt)
    y, mean, rstd = ops.layernorm_fwd(dev(x, dt), dev(gamma, dt), dev(beta, dt))
    ye, me, re_ = oracle.layernorm_fwd(x, gamma, beta)
    check(host(mean), me, "f32", "ln mean")
    check(host(rstd), re_, "f32", "ln rstd")
    check(host(y), ye, dt, "ln y")
    dy = host_input(g.standard_normal((rows, d)), dt)
    dx, dg, db = ops.layernorm_bwd(dev(x, dt), dev(dy, dt), mean, rstd, dev(gamma, dt))
    dxe, dge, dbe = oracle.layernorm_bwd(x, dy, host(mean), host(rstd), gamma)
    check(host(dx), dxe, dt, "ln dx")
    check(host(dg), dge, "f32", "ln dgamma")
    check(host(db), dbe, "f32", "ln dbeta")
    # accumulate into existing grads
    dg2, db2 = dg.clone(), db.clone()
    ops.layernorm_bwd(dev(x, dt), dev(dy, dt), mean, rstd, dev(gamma, dt), dg2, db2, accumulate=True)
    check(host(dg2), 2 * dge, "f32", "ln dgamma accumulate")


def test_layernorm_full_size_invariants(ops):
    """C3a shape 16384 x 1024: per-row Σdx = 0 and Σdx·x̂ = 0 (exact in reals)."""
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(16384, 1024, device="cuda", generator=g)
    gamma = 1 + 0.1 * torch.randn(1024, device="cuda", generator=g)
    beta = torch.zeros(1024, device="cuda")
    dy = torch.randn(16384, 1024, device="cuda", generator=g)
    y, mean, rstd = ops.layernorm_fwd(x, gamma, beta)
    dx, dg, db = ops.layernorm_bwd(x, dy, mean, rstd, gamma)
    xh = (x - mean[:, None]) * rstd[:, None]
    scale = dx.abs().mean().item() * 1024
    assert dx.sum(1).abs().max().item() < 1e-4 * scale
    assert (dx * xh).sum(1).abs().max().item() < 1e-3 * scale
    torch.testing.assert_close(db, dy.sum(0), rtol=1e-4, atol=1e-3)
    torch.testing.assert_close(dg, (dy * xh).sum(0), rtol=1e-4, atol=1e-3)


# ---------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n,c,eps,ignore", [(64, 10, 0.0, False), (64, 1000, 0.0, False), (33, 1001, 0.1, True),
                                            (256, 32000, 0.0, False), (8, 40000, 0.05, True), (5, 7, 0.0, False),
                                            # more rows than resident workgroups: each takes several rows
                                            (2000, 5000, 0.1, True), (600, 32000, 0.0, True), (5000, 1000, 0.0, True),
                                            # single-workgroup path (c <= 64, n <= 4096) at its limits
                                            (4096, 64, 0.1, True), (3000, 33, 0.05, True), (1, 3, 0.0, False)])
def test_softmax_xent(ops, oracle, dt, n, c, eps, ignore):
    g = rng(n + c)
    z = host_input(g.standard_normal((n, c)) * 2.0, dt)
    y = g.integers(0, c, n).astype(np.int64)
    if ignore:
        y[:: 4] = -100
    dl, loss = ops.softmax_xent_bwd(dev(z, dt), torch.from_numpy(y).cuda(), label_smoothing=eps)
    dle, losse = oracle.softmax_xent(z, y, eps)
    check(host(dl), dle, dt, "xent dlogits")
    check(loss.item(), losse, "f32", "xent loss", rtol=1e-5)
    # label gather is exact: the target column carries the −(1−ε)/n term
    # (negative without smoothing; with it a label of probability above
    # 1 − ε + ε/c has a positive gradient)
    rows = np.nonzero(y != -100)[0]
    if eps == 0.0:
        assert (host(dl)[rows, y[rows]] < 0).all()


@pytest.mark.parametrize("dt", DTYPES)
def test_softmax_xent_full_size_config(ops, oracle, dt):
    """configs[2]b at its benched size, 16384 x 32000, logits ~ N(0, 2),
    labels uniform (reference ce.hpp:36): every row's gradient sums to zero
    (in float64), the label column is the only negative entry of its row,
    the loss matches a float64 log-sum-exp, and 64 rows spread over the
    batch match the oracle run on those rows (its mean over 64 rows rescaled
    by 64/16384, a power of two, so the rescale is exact)."""
    n, c = 16384, 32000
    gen = torch.Generator(device="cuda").manual_seed(2)
    z = (2 * torch.randn((n, c), generator=gen, device="cuda")).to(torch.bfloat16 if dt == "bf16" else torch.float32)
    y = torch.randint(0, c, (n,), generator=gen, device="cuda")
    dz, loss = ops.softmax_xent_bwd(z, y)
    torch.cuda.synchronize()
    # Σ_j dz_ij = (Σ_j p_ij − 1)/n = 0 in reals.  fp32: the row's softmax
    # denominator is one fp32 sum of 32000 terms, common to the row, so Σp
    # is 1 within ~1e-6 (bound 1e-5 of Σ|dz|, where a missing label term
    # would give 0.5); bf16: each stored element is rounded once more, at
    # most 2^-9 of itself.
    row_sum = dz.double().sum(1)
    row_abs = dz.double().abs().sum(1)
    tol = 1e-5 if dt == "f32" else 2.0 ** -8
    assert (row_sum.abs() <= tol * row_abs).all().item(), "rows must sum to zero"
    at_label = dz.gather(1, y[:, None]).squeeze(1)
    assert (at_label < 0).all().item(), "label column must carry the -1/n term"
    neg = (dz < 0).sum(1)
    assert (neg == 1).all().item(), "only the label column is negative"
    zd = z.double()
    want_loss = (torch.logsumexp(zd, 1) - zd.gather(1, y[:, None]).squeeze(1)).mean().item()
    assert abs(loss.item() - want_loss) <= 1e-5 * abs(want_loss)
    rows = np.linspace(0, n - 1, 64).astype(np.int64)
    zr = host(z[rows])
    yr = y[rows].cpu().numpy()
    dle, _ = oracle.softmax_xent(zr, yr, 0.0)
    check(host(dz[rows]), dle * np.float32(64.0 / n), dt, "xent dlogits rows at full size")
    del z, dz, zd


@pytest.mark.parametrize("dt", DTYPES)
def test_adamw_full_size_config(ops, oracle, dt):
    """configs[2]c at its benched size: AdamW over one flat 1e8-parameter
    buffer, params ~ N(0, 0.02), grads ~ N(0, 1e-3), m = v = 0, lr 3e-4,
    wd 0.01, step 10 (reference adam.hpp:159-250).  Every element is compared
    with the oracle: fp32 bit-exact; bf16 moments bit-exact and parameters
    equal to the oracle's fp32 result rounded once to bf16."""
    n = 100_000_000
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    gen = torch.Generator(device="cuda").manual_seed(3)
    p = (0.02 * torch.randn(n, generator=gen, device="cuda")).to(tdt)
    gr = (1e-3 * torch.randn(n, generator=gen, device="cuda")).to(tdt)
    m = torch.zeros(n, device="cuda")
    v = torch.zeros(n, device="cuda")
    ph, gh = host(p), host(gr)
    ops.adam_step(p, gr, m, v, lr=3e-4, weight_decay=0.01, step=10, decoupled=True)
    pe, me, ve = oracle.adam_step(1, ph, gh, np.zeros(n, np.float32), np.zeros(n, np.float32), 3e-4, 0.9, 0.999,
                                  1e-8, 0.01, 10)
    assert np.array_equal(host(m).view(np.int32), me.view(np.int32))
    assert np.array_equal(host(v).view(np.int32), ve.view(np.int32))
    if dt == "f32":
        assert np.array_equal(host(p).view(np.int32), pe.view(np.int32))
    else:
        assert np.array_equal(host(p), host_input(pe, "bf16"))


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("c", [37, 40])
def test_softmax_xent_small_path_matches_general_path(ops, dt, c):
    """4096 rows of c classes take the single-workgroup kernel; the same rows
    plus one ignored row (4097 rows, same valid count) take the three-launch
    path.  With c = 37 that path is the element kernel, whose summation order
    the small kernel keeps: gradients and loss agree bit for bit.  With c = 40
    it is the vector kernel (16-byte groups summed first): within rounding."""
    g = rng(41)
    z = host_input(g.standard_normal((4097, c)) * 2.0, dt)
    y = g.integers(0, c, 4097).astype(np.int64)
    y[::7] = -100
    y[-1] = -100
    zd, yd = dev(z, dt), torch.from_numpy(y).cuda()
    dl_small, loss_small = ops.softmax_xent_bwd(zd[:4096].contiguous(), yd[:4096].contiguous(), label_smoothing=0.1)
    dl_gen, loss_gen = ops.softmax_xent_bwd(zd, yd, label_smoothing=0.1)
    torch.cuda.synchronize()
    if c % 4 != 0:
        assert torch.equal(dl_small, dl_gen[:4096])
        assert torch.equal(loss_small, loss_gen)
    else:
        check(host(dl_small), host(dl_gen[:4096]), dt, "small vs vector path dlogits")
        check(loss_small.item(), loss_gen.item(), "f32", "small vs vector path loss", rtol=1e-6)


def test_softmax_xent_bad_label_is_reported(ops):
    z = torch.randn(4, 10, device="cuda")
    y = torch.tensor([1, 2, 10, -5], device="cuda")
    ctx = ops.context()
    ctx.device_errors()
    dl, _ = ops.softmax_xent_bwd(z, y)
    assert ctx.device_errors() == 2
    assert torch.count_nonzero(dl[2:]).item() == 0


def test_cast_matches_torch_bf16_conversion(ops):
    """nott_cast fp32 -> bf16 (the mixed-precision weight copies and input
    cast) against torch's CPU conversion, bit for bit, on random values over
    the whole range, exact ties, ±0, ±inf, NaNs, subnormals and overflow to
    inf; NaN stays NaN with its sign."""
    from test_oracle import _bf16_specials
    x = _bf16_specials()
    got = host(ops.cast(torch.from_numpy(x.copy()).cuda(), torch.bfloat16))
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).to(torch.float32).numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.array_equal(np.signbit(got[nan]), np.signbit(x[nan]))
