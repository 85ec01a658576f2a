"""nott_layernorm_bwd_noalloc (the allocation-free LayerNorm backward)
against nott_layernorm_bwd, through the C ABI: two calls in a row on the same
GPU, the second smaller, bit-identical outputs (the same kernels), plus the
clear error for a problem larger than the static scratch."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import dev, host
from oracle_lib import f32, rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from thot_amd import ops as _ops
    assert torch.cuda.is_available()
    return _ops


def _inputs(g, rows, d, dt):
    x = f32(g.standard_normal((rows, d)))
    gamma = f32(1 + 0.1 * g.standard_normal(d))
    beta = np.zeros(d, np.float32)
    dy = f32(g.standard_normal((rows, d)))
    return x, gamma, beta, dy


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_noalloc_matches_layernorm_bwd(ops, dt):
    g = rng(123)
    ctx = ops.context()
    # each call smaller than the one before; the first at the vector path's
    # largest row width with a large row count (accepted: ≤ 4 MiB of partials)
    for rows, d in ((16384, 2048), (4096, 1024), (300, 200), (7, 33)):
        print(f"noalloc case rows={rows} d={d} dtype={dt}", flush=True)
        x, gamma, beta, dy = (dev(a, dt) for a in _inputs(g, rows, d, dt))
        y, mean, rstd = ops.layernorm_fwd(x, gamma, beta)
        outs = []
        for name in ("nott_layernorm_bwd", "nott_layernorm_bwd_noalloc"):
            dx = torch.empty_like(x)
            dg = torch.full((d,), 7.0, device="cuda")
            db = torch.full((d,), -3.0, device="cuda")
            ctx.call(name, ops.nott_dtype(x.dtype), rows, d, ops._ptr(x), ops._ptr(dy), ops._ptr(mean),
                     ops._ptr(rstd), ops._ptr(gamma), ops._ptr(dx), ops._ptr(dg), ops._ptr(db), 0)
            torch.cuda.synchronize()
            outs.append((host(dx), host(dg), host(db)))
        for a, b in zip(*outs):
            assert np.array_equal(a, b)
        # accumulate = 1 adds into the existing parameter gradients
        dg = torch.full((d,), 1.5, device="cuda")
        db = torch.full((d,), 2.5, device="cuda")
        dx = torch.empty_like(x)
        ctx.call("nott_layernorm_bwd_noalloc", ops.nott_dtype(x.dtype), rows, d, ops._ptr(x), ops._ptr(dy),
                 ops._ptr(mean), ops._ptr(rstd), ops._ptr(gamma), ops._ptr(dx), ops._ptr(dg), ops._ptr(db), 1)
        torch.cuda.synchronize()
        np.testing.assert_allclose(host(dg), outs[0][1] + 1.5, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(host(db), outs[0][2] + 2.5, rtol=1e-6, atol=1e-6)


def test_noalloc_rejects_oversized_problem(ops):
    """d = 8192 is above the vector path's 2048, so the generic path needs
    8·d·rows = 512 MiB of partials, more than the 16 MiB static scratch: a
    clear error, no launch."""
    from thot_amd._abi import NottInvalidArgument
    rows, d = 8192, 8192
    x = torch.zeros((rows, d), device="cuda")
    mean = torch.zeros((rows,), device="cuda")
    rstd = torch.ones((rows,), device="cuda")
    gamma = torch.ones((d,), device="cuda")
    dx = torch.empty_like(x)
    ctx = ops.context()
    with pytest.raises(NottInvalidArgument, match="static scratch"):
        ctx.call("nott_layernorm_bwd_noalloc", 0, rows, d, ops._ptr(x), ops._ptr(x), ops._ptr(mean), ops._ptr(rstd),
                 ops._ptr(gamma), ops._ptr(dx), None, None, 0)
