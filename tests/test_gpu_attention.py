"""GPU parity of the flash-style attention kernels (forward, dq/dk/dv) and of
the multi-head attention module built from them, against the CPU oracle and
the reference's own golden vectors, through the C ABI.

configs[3] (B=8, H=16, T=1024, dh=64, causal, bf16) is checked at full size
against a float32 torch reference of the same attention on the GPU (scores
materialised, as the reference module does)."""
import math
import os

import numpy as np
import pytest
import torch

from gpu_util import check, dev, host, host_input
from oracle_lib import f32, rng

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ops():
    from thot_amd import ops as _ops
    assert torch.cuda.is_available()
    return _ops


@pytest.mark.parametrize("name", ["attention_causal", "attention_full"])
def test_attention_golden(ops, name):
    """The HIP path against vectors written by the reference's ScaledDotProductKernel."""
    z = np.load(os.path.join(GOLD, name + ".npz"))
    q, k, v, dO = (f32(z[n]) for n in ("q", "k", "v", "dO"))
    b, h, t, dh = q.shape
    d = ops.attn_desc(b, h, t, k.shape[2], dh, bool(z["causal"]))
    o, lse = ops.attention_fwd(dev(q), dev(k), dev(v), d)
    dq, dk, dv = ops.attention_bwd(dev(q), dev(k), dev(v), o, dev(dO), lse, d)
    torch.cuda.synchronize()
    check(host(o), z["o"], what="o")
    check(host(dq), z["dq"], what="dq")
    check(host(dk), z["dk"], what="dk")
    check(host(dv), z["dv"], what="dv")


CASES = [
    (1, 2, 5, 5, 4, True),
    (2, 3, 70, 70, 16, True),
    (1, 2, 64, 64, 64, False),
    (2, 2, 130, 130, 32, True),
    (1, 1, 100, 77, 8, False),
    (1, 2, 33, 100, 64, True),
    (1, 1, 192, 192, 24, True),
    # head dim 64 (the bf16 a64 kernels): ragged ends over several 128-row
    # blocks, causal and full, t < s and t > s
    (1, 2, 300, 300, 64, True),
    (1, 2, 200, 330, 64, False),
    (2, 1, 257, 129, 64, True),
]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "b{}h{}t{}s{}d{}c{}".format(*c))
def test_attention_vs_oracle(ops, oracle, dt, case):
    b, h, t, s, dh, causal = case
    g = rng(sum(case) + len(dt))
    q = host_input(g.standard_normal((b, h, t, dh)), dt)
    k = host_input(g.standard_normal((b, h, s, dh)), dt)
    v = host_input(g.standard_normal((b, h, s, dh)), dt)
    dO = host_input(g.standard_normal((b, h, t, dh)), dt)
    d = ops.attn_desc(b, h, t, s, dh, causal)
    o, lse = ops.attention_fwd(dev(q, dt), dev(k, dt), dev(v, dt), d)
    ro, rlse = oracle.attention_fwd(d, q, k, v)
    torch.cuda.synchronize()
    check(host(o), ro, dt, "o")
    check(host(lse), rlse, "f32" if dt == "f32" else dt, "lse")
    # backward from the oracle's o (rounded like the GPU's) so both sides see the same inputs
    o_in = host_input(ro, dt)
    dq, dk, dv = ops.attention_bwd(dev(q, dt), dev(k, dt), dev(v, dt), dev(o_in, dt), dev(dO, dt), lse, d)
    rdq, rdk, rdv = oracle.attention_bwd(d, q, k, v, o_in, dO)
    torch.cuda.synchronize()
    check(host(dq), rdq, dt, "dq")
    check(host(dk), rdk, dt, "dk")
    check(host(dv), rdv, dt, "dv")


def _torch_attention_fp32(q, k, v, dO, causal, scale):
    """float32 reference with materialised scores (the reference module's math)."""
    q, k, v = (x.float().detach().clone().requires_grad_(True) for x in (q, k, v))
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if causal:
        t, sl = s.shape[-2], s.shape[-1]
        mask = torch.triu(torch.ones(t, sl, dtype=torch.bool, device=s.device), 1)
        s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, v)
    o.backward(dO.float())
    return o.detach(), q.grad, k.grad, v.grad


def test_attention_config4_full_size(ops):
    """B=8, H=16, T=1024, dh=64, causal, bf16 (checked on 2 of the 8 batches)."""
    B, H, T, Dh = 8, 16, 1024, 64
    gen = torch.Generator(device="cuda").manual_seed(4)
    mk = lambda: torch.randn((B, H, T, Dh), generator=gen, device="cuda").to(torch.bfloat16)
    q, k, v, dO = mk(), mk(), mk(), mk()
    d = ops.attn_desc(B, H, T, T, Dh, True)
    o, lse = ops.attention_fwd(q, k, v, d)
    dq, dk, dv = ops.attention_bwd(q, k, v, o, dO, lse, d)
    torch.cuda.synchronize()
    for bsl in (slice(0, 1), slice(B - 1, B)):
        ro, rdq, rdk, rdv = _torch_attention_fp32(q[bsl], k[bsl], v[bsl], dO[bsl], True, 1 / math.sqrt(Dh))
        check(host(o[bsl]), host(ro), "bf16", "o")
        check(host(dq[bsl]), host(rdq), "bf16", "dq")
        check(host(dk[bsl]), host(rdk), "bf16", "dk")
        check(host(dv[bsl]), host(rdv), "bf16", "dv")


def test_attention_rejects_bad_descriptors(ops):
    from thot_amd._abi import NottInvalidArgument
    q = torch.zeros((1, 1, 4, 200), device="cuda")
    d = ops.attn_desc(1, 1, 4, 4, 200, False)
    with pytest.raises(NottInvalidArgument):
        ops.attention_fwd(q, q, q, d)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,h,t,dh,causal", [(2, 3, 100, 64, True), (1, 4, 77, 40, False), (2, 2, 130, 32, True)])
def test_attention_token_major(ops, dt, b, h, t, dh, causal):
    """Token-major views (q, k, v packed per token as a [b·t, 3·h·dh]
    projection output, o / dO as [b·t, h·dh]; dq, dk, dv written into a packed
    buffer) give the head-major results bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(b * 100 + t + dh)
    E = h * dh
    qkv = torch.randn((b, t, 3, h, dh), generator=g, device="cuda").to(dt)
    dO_tm = torch.randn((b, t, h, dh), generator=g, device="cuda").to(dt)
    hm = lambda x: x.permute(0, 2, 1, 3).contiguous()
    q, k, v = (hm(qkv[:, :, i]) for i in range(3))
    d = ops.attn_desc(b, h, t, t, dh, causal)
    o, lse = ops.attention_fwd(q, k, v, d)
    dq, dk, dv = ops.attention_bwd(q, k, v, o, hm(dO_tm), lse, d)

    flat = qkv.view(b, t, 3 * E)
    qt, kt, vt = (flat[:, :, i * E:(i + 1) * E].view(b, t, h, dh) for i in range(3))
    dtm = ops.attn_desc(b, h, t, t, dh, causal, token_major=True, ld_qkv=3 * E)
    o_tm, lse_tm = ops.attention_fwd(qt, kt, vt, dtm)
    dqkv = torch.full((b, t, 3 * E), 5.0, device="cuda").to(dt)
    outs = tuple(dqkv[:, :, i * E:(i + 1) * E].view(b, t, h, dh) for i in range(3))
    ops.attention_bwd(qt, kt, vt, o_tm, dO_tm, lse_tm, dtm, out=outs)
    torch.cuda.synchronize()
    assert torch.equal(o_tm.permute(0, 2, 1, 3), o)
    assert torch.equal(lse_tm, lse)
    for got, want in zip(outs, (dq, dk, dv)):
        assert torch.equal(got.permute(0, 2, 1, 3), want)


# ------------------------------------------------ composed MultiHeadAttention
def _mha_composed(ops, x2, w_in, b_in, wo, bo, dy2, b, t, heads, causal=True):
    """MultiHeadAttentionImpl (reference attention/details/head.hpp:47-83 +
    kernel.hpp:20-96) as the bench composes it: one packed q/k/v projection,
    token-major attention on views of its output (no head split or merge
    copies), the output projection; then the backward in reverse, with dq,
    dk, dv written into the packed gradient the input projection reads."""
    e = x2.shape[1]
    dh = e // heads
    qkv = ops.linear_fwd(x2, w_in, b_in)
    d = ops.attn_desc(b, heads, t, t, dh, causal, token_major=True, ld_qkv=3 * e)
    q, k, v = (qkv.view(b, t, 3 * e)[:, :, i * e:(i + 1) * e].view(b, t, heads, dh) for i in range(3))
    o, lse = ops.attention_fwd(q, k, v, d)
    a = o.view(b * t, e)
    y = ops.linear_fwd(a, wo, bo)
    da, dwo, dbo = ops.linear_bwd(dy2, a, wo)
    dqkv = torch.empty((b, t, 3 * e), dtype=x2.dtype, device="cuda")
    views = tuple(dqkv[:, :, i * e:(i + 1) * e].view(b, t, heads, dh) for i in range(3))
    ops.attention_bwd(q, k, v, o, da.view(b, t, heads, dh), lse, d, out=views)
    dx, dw_in, db_in = ops.linear_bwd(dqkv.view(b * t, 3 * e), x2, w_in)
    return y, dx, dw_in, db_in, dwo, dbo


def test_mha_module_golden(ops):
    """The composed module against the reference MultiHeadAttention's own
    output and gradients (tests/golden/mha_causal.npz, written by head.hpp's
    module through libtorch): fp32, causal, with biases."""
    z = np.load(os.path.join(GOLD, "mha_causal.npz"))
    x = f32(z["x"])
    b, t, e = x.shape
    heads = int(z["heads"])
    w_in = np.concatenate([z["wq"], z["wk"], z["wv"]], 0)
    b_in = np.concatenate([z["bq"], z["bk"], z["bv"]], 0)
    y, dx, dw_in, db_in, dwo, dbo = _mha_composed(ops, dev(x.reshape(b * t, e)), dev(w_in), dev(b_in), dev(z["wo"]),
                                                  dev(z["bo"]), dev(f32(z["dy"]).reshape(b * t, e)), b, t, heads)
    torch.cuda.synchronize()
    check(host(y).reshape(b, t, e), z["y"], what="mha y")
    check(host(dx).reshape(b, t, e), z["dx"], what="mha dx")
    dw = host(dw_in)
    db = host(db_in)
    for i, n in enumerate("qkv"):
        check(dw[i * e:(i + 1) * e], z["dw" + n], what=f"mha dw{n}")
        check(db[i * e:(i + 1) * e], z["db" + n], what=f"mha db{n}")
    check(host(dwo), z["dwo"], what="mha dwo")
    check(host(dbo), z["dbo"], what="mha dbo")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_mha_projection_shapes_config3(ops, oracle, dt):
    """configs[3]'s projection GEMMs at full size (8192 tokens, E = 1024: the
    packed 1024→3072 input projection and the 1024→1024 output projection),
    forward and backward, on the hand-written GEMMs.  Checked against the
    oracle on slices: 64 rows of y and dx (all columns), and 16 output rows
    of dW / db (sums over all 8192 tokens)."""
    g = rng(31)
    m, kin = 8192, 1024
    for nout in (3072, 1024):
        print(f"projection {m}x{kin}->{nout} {dt}", flush=True)
        x = host_input(g.standard_normal((m, kin)), dt)
        w = host_input(g.standard_normal((nout, kin)) * 0.02, dt)
        bias = f32(g.standard_normal(nout) * 0.1)
        dy = host_input(g.standard_normal((m, nout)), dt)
        xd, wd, dyd = dev(x, dt), dev(w, dt), dev(dy, dt)
        y = ops.linear_fwd(xd, wd, dev(bias))
        dx, dw, db = ops.linear_bwd(dyd, xd, wd)
        torch.cuda.synchronize()
        rows = np.r_[0:32, m - 32:m]
        check(host(y)[rows], oracle.linear_fwd(x[rows], w, bias), dt, "proj y rows")
        rdx, _, _ = oracle.linear_bwd(dy[rows], x[rows], w)
        check(host(dx)[rows], rdx, dt, "proj dx rows")
        outs = np.r_[0:8, nout - 8:nout]
        _, rdw, rdb = oracle.linear_bwd(np.ascontiguousarray(dy[:, outs]), x, np.ascontiguousarray(w[outs]))
        check(host(dw)[outs], rdw, "f32" if dt == "f32" else dt, "proj dw rows")
        check(host(db)[outs], rdb, "f32" if dt == "f32" else dt, "proj db rows")
