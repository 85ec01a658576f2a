"""Empty inputs through every entry point of the path, on the GPU.

A batch (or row set) of size zero is legal at the reference's boundary
(libtorch ops accept empty tensors): activation gradients come back empty and
parameter gradients are sums over nothing, i.e. zero, or left unchanged when
accumulating.  The mean cross-entropy over no valid row is NaN (0/0), as
torch's mean reduction gives.  Outputs are pre-filled with a sentinel so that
"zeroed" is distinguishable from "untouched"."""
import math

import pytest
import torch

from thot_amd import ops

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.bfloat16]
SENT = 7.0


def _filled(shape):
    return torch.full(shape, SENT, dtype=torch.float32, device="cuda")


@pytest.mark.parametrize("dt", DT)
def test_empty_conv(dt):
    d = ops.conv_desc((0, 8, 9, 9), (16, 8, 3, 3), padding=(1, 1))
    x = torch.empty((0, 8, 9, 9), dtype=dt, device="cuda")
    dy = torch.empty((0, 16, 9, 9), dtype=dt, device="cuda")
    w = torch.randn((16, 8, 3, 3), device="cuda").to(dt)
    assert ops.conv2d_fwd(x, w, None, d).shape == (0, 16, 9, 9)
    assert ops.conv2d_bwd_data(dy, w, d).shape == (0, 8, 9, 9)
    dw, db = _filled((16, 8, 3, 3)), _filled((16,))
    ops.conv2d_bwd_weight(x, dy, d, dw=dw, db=db)
    torch.cuda.synchronize()
    assert torch.count_nonzero(dw).item() == 0 and torch.count_nonzero(db).item() == 0
    dw2, db2 = _filled((16, 8, 3, 3)), _filled((16,))
    ops.conv2d_bwd_weight(x, dy, d, dw=dw2, db=db2, accumulate=True)
    torch.cuda.synchronize()
    assert bool((dw2 == SENT).all()) and bool((db2 == SENT).all())


@pytest.mark.parametrize("dt", DT)
def test_empty_linear(dt):
    x = torch.empty((0, 12), dtype=dt, device="cuda")
    dy = torch.empty((0, 5), dtype=dt, device="cuda")
    w = torch.randn((5, 12), device="cuda").to(dt)
    dw, db = _filled((5, 12)), _filled((5,))
    dx, _, _ = ops.linear_bwd(dy, x, w, dw=dw, db=db)
    torch.cuda.synchronize()
    assert dx.shape == (0, 12)
    assert torch.count_nonzero(dw).item() == 0 and torch.count_nonzero(db).item() == 0


@pytest.mark.parametrize("dt", DT)
def test_empty_layernorm(dt):
    x = torch.empty((0, 64), dtype=dt, device="cuda")
    gamma = torch.ones(64, device="cuda").to(dt)
    mean = torch.empty(0, device="cuda")
    rstd = torch.empty(0, device="cuda")
    dg, dbt = _filled((64,)), _filled((64,))
    dx, _, _ = ops.layernorm_bwd(x, x, mean, rstd, gamma, dgamma=dg, dbeta=dbt)
    torch.cuda.synchronize()
    assert dx.shape == (0, 64)
    assert torch.count_nonzero(dg).item() == 0 and torch.count_nonzero(dbt).item() == 0


@pytest.mark.parametrize("dt", DT)
def test_empty_and_all_ignored_xent(dt):
    z = torch.empty((0, 10), dtype=dt, device="cuda")
    y = torch.empty((0,), dtype=torch.int64, device="cuda")
    dl, loss = ops.softmax_xent_bwd(z, y)
    torch.cuda.synchronize()
    assert dl.shape == (0, 10) and math.isnan(loss.item())
    # every row ignored: zero gradient, NaN mean loss
    z = torch.randn((4, 10), device="cuda").to(dt)
    y = torch.full((4,), -100, dtype=torch.int64, device="cuda")
    dl, loss = ops.softmax_xent_bwd(z, y)
    torch.cuda.synchronize()
    assert torch.count_nonzero(dl).item() == 0 and math.isnan(loss.item())


def test_empty_adam():
    e = torch.empty(0, device="cuda")
    ops.adam_step(e, e.clone(), e.clone(), e.clone(), lr=1e-3, step=1, decoupled=True)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", DT)
def test_empty_maxpool(dt):
    d = ops.pool_desc((0, 3, 8, 8), (2, 2))
    x = torch.empty((0, 3, 8, 8), dtype=dt, device="cuda")
    y, idx = ops.maxpool2d_fwd(x, d)
    dx = ops.maxpool2d_bwd(idx, torch.empty_like(y), d)
    torch.cuda.synchronize()
    assert y.shape == (0, 3, 4, 4) and dx.shape == (0, 3, 8, 8)


@pytest.mark.parametrize("dt", DT)
def test_empty_attention(dt):
    # no (batch, head) pairs
    d = ops.attn_desc(0, 4, 16, 16, 64, True)
    q = torch.empty((0, 4, 16, 64), dtype=dt, device="cuda")
    o, lse = ops.attention_fwd(q, q, q, d)
    dq, dk, dv = ops.attention_bwd(q, q, q, o, o, lse, d)
    assert dq.shape == q.shape
    # no queries (non-causal): dk = dv = 0
    d = ops.attn_desc(2, 3, 0, 16, 64, False)
    q = torch.empty((2, 3, 0, 64), dtype=dt, device="cuda")
    k = torch.randn((2, 3, 16, 64), device="cuda").to(dt)
    lse = torch.empty((2, 3, 0), device="cuda")
    dq, dk, dv = ops.attention_bwd(q, k, k, q, q, lse, d)
    torch.cuda.synchronize()
    assert dq.shape == q.shape
    assert torch.count_nonzero(dk).item() == 0 and torch.count_nonzero(dv).item() == 0


@pytest.mark.parametrize("dt", DT)
def test_empty_elementwise(dt):
    e = torch.empty(0, dtype=dt, device="cuda")
    assert ops.relu_bwd(e, e).shape == (0,)
    assert ops.add(e, e).shape == (0,)
