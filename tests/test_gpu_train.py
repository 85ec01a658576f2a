"""End-to-end training steps through the C++ host layer (include/nott_hip/host.hpp,
thot_amd/_nott_host): forward, mean cross-entropy, backward and the fused
Adam/AdamW update all run on libnott_hip.

configs[0] (small CNN + Adam) is checked step by step against the CPU oracle
composed layer by layer in the reference's order (core.hpp:3735-3827): loss,
every parameter gradient, and the updated parameters after two steps.
configs[4] (ResNet-18 + AdamW) is checked at batch 64 against the reference's
ResNet-18 on the CPU (oracle/_ref) on identical weights and inputs."""
import math

import numpy as np
import pytest
import torch

from gpu_util import check, host
from oracle_lib import f32, rng
from thot_amd._abi import Conv2dDesc, Pool2dDesc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def host_mod():
    assert torch.cuda.is_available()
    from thot_amd import _abi
    _abi.load()
    from thot_amd import _nott_host
    return _nott_host


def conv_desc(n, c, h, w, k, r, pad):
    return Conv2dDesc(n, c, h, w, k, r, r, 1, 1, pad, pad, 1, 1, 1, 0, 0)


def pool_desc(n, c, h, w):
    return Pool2dDesc(n, c, h, w, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0)


def small_cnn_oracle_step(orc, P, x, y):
    """One configs[0] step on the CPU oracle: returns loss and grads."""
    n = x.shape[0]
    d1 = conv_desc(n, 1, 28, 28, 32, 3, 1)
    a1 = orc.conv2d_fwd(d1, x, P["conv2d_0.weight"], P["conv2d_0.bias"])
    r1 = orc.relu_fwd(a1)
    p1d = pool_desc(n, 32, 28, 28)
    m1, i1 = orc.maxpool2d_fwd(p1d, r1)
    d2 = conv_desc(n, 32, 14, 14, 64, 3, 1)
    a2 = orc.conv2d_fwd(d2, m1, P["conv2d_2.weight"], P["conv2d_2.bias"])
    r2 = orc.relu_fwd(a2)
    p2d = pool_desc(n, 64, 14, 14)
    m2, i2 = orc.maxpool2d_fwd(p2d, r2)
    flat = m2.reshape(n, -1)
    a3 = orc.linear_fwd(flat, P["fc_5.weight"], P["fc_5.bias"])
    r3 = orc.relu_fwd(a3)
    z = orc.linear_fwd(r3, P["fc_6.weight"], P["fc_6.bias"])
    dz, loss = orc.softmax_xent(z, y)
    G = {}
    dr3, G["fc_6.weight"], G["fc_6.bias"] = orc.linear_bwd(dz, r3, P["fc_6.weight"])
    da3 = orc.relu_bwd(r3, dr3)
    dflat, G["fc_5.weight"], G["fc_5.bias"] = orc.linear_bwd(da3, flat, P["fc_5.weight"])
    dm2 = dflat.reshape(m2.shape)
    dr2 = orc.maxpool2d_bwd(p2d, i2, dm2)
    da2 = orc.relu_bwd(r2, dr2)
    G["conv2d_2.weight"], G["conv2d_2.bias"] = orc.conv2d_bwd_weight(d2, m1, da2)
    dm1 = orc.conv2d_bwd_data(d2, da2, P["conv2d_2.weight"])
    dr1 = orc.maxpool2d_bwd(p1d, i1, dm1)
    da1 = orc.relu_bwd(r1, dr1)
    G["conv2d_0.weight"], G["conv2d_0.bias"] = orc.conv2d_bwd_weight(d1, x, da1)
    return loss, G


def test_small_cnn_two_steps_vs_oracle(host_mod, oracle):
    """batch 64 x 1x28x28, Adam(1e-3), HeUniform weights, zero bias."""
    g = rng(2024)
    n = 64
    P = {
        "conv2d_0.weight": f32(g.uniform(-1, 1, (32, 1, 3, 3)) * math.sqrt(6 / 9)),
        "conv2d_0.bias": np.zeros(32, np.float32),
        "conv2d_2.weight": f32(g.uniform(-1, 1, (64, 32, 3, 3)) * math.sqrt(6 / 288)),
        "conv2d_2.bias": np.zeros(64, np.float32),
        "fc_5.weight": f32(g.uniform(-1, 1, (128, 3136)) * math.sqrt(6 / 3136)),
        "fc_5.bias": np.zeros(128, np.float32),
        "fc_6.weight": f32(g.uniform(-1, 1, (10, 128)) * math.sqrt(6 / 128)),
        "fc_6.bias": np.zeros(10, np.float32),
    }
    tr = host_mod.SmallCNNTrainer(0, 1, 1e-3)
    assert tr.num_params() == 421642
    tr.load({k: torch.from_numpy(v).cuda() for k, v in P.items()})
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    for step in (1, 2):
        x = f32(g.uniform(0, 1, (n, 1, 28, 28)))
        y = g.integers(0, 10, n).astype(np.int64)
        loss = tr.forward_backward(torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda())
        grads = {k: host(v) for k, v in tr.grads().items()}
        rloss, G = small_cnn_oracle_step(oracle, P, x, y)
        check(np.array([loss.item()]), np.array([rloss]), what=f"loss step {step}")
        for k in P:
            check(grads[k], G[k], what=f"grad {k} step {step}")
        tr.optimizer_step()
        for k in P:
            P[k], M[k], V[k] = oracle.adam_step(0, P[k], G[k], M[k], V[k], 1e-3, 0.9, 0.999, 1e-8, 0.0, step)
        params = {k: host(v) for k, v in tr.params().items()}
        for k in P:
            check(params[k], P[k], what=f"param {k} after step {step}")
        # zero_grad(set_to_none=false) after the step (core.hpp:3823)
        assert all(float(torch.count_nonzero(v)) == 0 for v in tr.grads().values())


# ------------------------------------------------------------- ResNet-18
def _strict(got, want, rtol, atol):
    """Elements of `got` outside |got − want| <= atol + rtol·|want| (count, worst excess ratio)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = atol + rtol * np.abs(want)
    err = np.abs(got - want)
    return int((err > bound).sum()), float((err / bound).max()) if err.size else 0.0


def _ref_inputs(tr, bf16):
    """The reference's initial tensors: the HIP model's parameters and float
    buffers by registration key (bf16: conv/linear weights as the bf16
    working copies the mixed-precision path computes with)."""
    vals = {k: host(v) for k, v in tr.params().items()}
    if bf16:
        from oracle_lib import round_bf16
        vals = {k: (round_bf16(v) if v.ndim > 1 else v) for k, v in vals.items()}
    for k, v in tr.buffers().items():
        if not k.endswith("num_batches_tracked"):
            vals[k] = host(v)
    return vals


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-300))


@pytest.mark.parametrize("bf16,seed", [(False, 17), (False, 1), (False, 3), (True, 17)],
                         ids=["fp32-seed17", "fp32-seed1", "fp32-seed3", "bf16-seed17"])
def test_resnet18_step_batch64_vs_reference(host_mod, bf16, seed):
    """configs[4] at its size: one full training step (forward, CE mean,
    backward, AdamW lr 1e-3 wd 1e-2) at batch 64 × 3×224×224 against the
    reference's ResNet-18 assembled from Nott's own layer factories and
    residual-block semantics (oracle/_ref, libtorch CPU), on identical weights
    (loaded by registration key) and inputs.

    fp32.  The loss, the logits, every parameter after AdamW and every
    BatchNorm running statistic must agree with the reference's fp32 step
    elementwise at |got − want| <= 1e-5 + 1e-4·|want|.  The gradients are
    judged against the exact result: the same reference step in float64.
    Through 20 ReLUs and 20 training-mode BatchNorms at batch 64, the
    reference's own fp32 gradients are not within that bound of the float64
    ones (BatchNorm's backward subtracts per-channel sums from each element,
    and an activation within rounding of zero takes the other ReLU branch in
    one precision and not the other).  Which tensors that hits differs
    between any two fp32 computations, so the HIP gradients are held to the
    reference's fp32 distance from float64 in aggregate: the sum over the 56
    tensors of the relative-norm distances within 2x the reference's, the
    number of elements outside the bound within 2.5x, and every tensor
    within a relative norm of 5e-3 (about twice the largest either
    implementation shows).  Three weight seeds are run.  All counts, and the
    ReLU flips at the nine observable ReLU outputs (stem, eight blocks), are
    printed.
    Parameters after AdamW are bit-exact against the oracle's AdamW on the
    step's own gradients, and every element that differs from the
    reference's updated parameter beyond the bound is one whose gradient has
    the other sign (step 1 moves a weight by about lr·sign(g)).
    bf16 mixed precision: the reference runs on the bf16-rounded weights and
    input, once in plain fp32 and once with every activation and activation
    gradient rounded to bf16 where this path stores them.  Loss within rel
    2e-2 of both.  Two bf16-storage computations that differ only in fp32
    summation order already diverge through 20 layers (values on either side
    of a bf16 rounding boundary, thousands of ReLU flips per block), so the
    gradients are judged by what bf16 storage costs: for every tensor the
    relative-norm distance of the HIP gradient from the fp32 reference must
    be within 1.5× that of the bf16-storage reference (+1e-3); elementwise
    counts at rel 2e-2 are printed.  The AdamW update is bit-exact against
    the oracle on the step's own gradients."""
    from oracle_lib import Ref, round_bf16
    if not Ref.available():
        pytest.skip("oracle/_ref not built")
    ref = Ref()
    n = 64
    g = rng(4242)
    x = f32(g.uniform(0, 1, (n, 3, 224, 224)))
    y = g.integers(0, 1000, n).astype(np.int64)
    tr = host_mod.ResNet18Trainer(0, seed, bf16, 1e-3, 1e-2, 1000)
    assert tr.num_params() == 11687720
    vals = _ref_inputs(tr, bf16)
    p0 = {k: host(v) for k, v in tr.params().items()}
    loss_t, outs = tr.forward_backward_recording(torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda())
    loss = loss_t.item()
    grads = {k: host(v) for k, v in tr.grads().items()}
    outs = [host(o) for o in outs]
    logits = outs.pop()
    tr.optimizer_step()
    after = {k: host(v) for k, v in tr.params().items()}
    bufs = {k: host(v) for k, v in tr.buffers().items()}
    assert all(float(torch.count_nonzero(v)) == 0 for v in tr.grads().values())
    xr = round_bf16(x) if bf16 else x
    rloss, rlogits, rgrads, rafter, rblocks = ref.resnet18_step(xr, y, vals, 1e-3, 1e-2, want_blocks=True)
    assert set(rgrads) == set(grads), sorted(set(rgrads) ^ set(grads))
    flips = [int(((a > 0) != (b > 0)).sum()) for a, b in zip(outs, rblocks)]
    report = {"loss": (loss, rloss), "relu_flips_vs_ref32": flips}
    if not bf16:
        dloss, _, dgrads, _, dblocks = ref.resnet18_step(x, y, vals, 1e-3, 1e-2, want_blocks=True, precision="f64")
        report["loss_f64"] = dloss
        report["relu_flips_hip_vs_f64"] = [int(((a > 0) != (b > 0)).sum()) for a, b in zip(outs, dblocks)]
        report["relu_flips_ref32_vs_f64"] = [int(((a > 0) != (b > 0)).sum()) for a, b in zip(rblocks, dblocks)]
        assert abs(loss - rloss) <= 1e-5 + 1e-4 * abs(rloss), report
        report["logits_out_of_tol"] = _strict(logits, rlogits, 1e-4, 1e-5)
        assert report["logits_out_of_tol"][0] == 0, report
        rows = {}
        for k in sorted(rgrads):
            rows[k] = {"hip_vs_ref32": _strict(grads[k], rgrads[k], 1e-4, 1e-5)[0],
                       "hip_vs_f64": _strict(grads[k], dgrads[k], 1e-4, 1e-5)[0],
                       "ref32_vs_f64": _strict(rgrads[k], dgrads[k], 1e-4, 1e-5)[0],
                       "relnorm_hip_f64": _rel(grads[k], dgrads[k]), "relnorm_ref32_f64": _rel(rgrads[k], dgrads[k])}
        tot = {c: sum(r[c] for r in rows.values()) for c in ("hip_vs_ref32", "hip_vs_f64", "ref32_vs_f64")}
        report["grad_elements"] = int(sum(v.size for v in grads.values()))
        report["out_of_tol_totals"] = tot
        # Parameters after AdamW: the update is bit-exact on the step's own
        # gradients.  Against the reference's step, step 1 moves each weight
        # by lr·g/(|g| + eps) ≈ lr·sign(g), so an element whose gradient is
        # within the fp32 noise of zero moves differently in the two steps;
        # every element out of tolerance must be explained by its two
        # gradients: |Δp| <= lr·|u(g_hip) − u(g_ref)| + tolerance.
        lr, eps = 1e-3, 1e-8
        unexplained, out_tol = 0, 0
        for k in p0:
            pe, _, _ = oracle_adam(p0[k], grads[k], 1)
            assert np.array_equal(after[k], pe), k
            gh, gr = grads[k].astype(np.float64), rgrads[k].astype(np.float64)
            tol = 1e-5 + 1e-4 * np.abs(rafter[k])
            dp = np.abs(after[k].astype(np.float64) - rafter[k])
            du = lr * np.abs(gh / (np.abs(gh) + eps) - gr / (np.abs(gr) + eps))
            out_tol += int((dp > tol).sum())
            unexplained += int((dp > du + tol).sum())
        report["params_out_of_tol"] = out_tol
        sum_hip = sum(r["relnorm_hip_f64"] for r in rows.values())
        sum_ref = sum(r["relnorm_ref32_f64"] for r in rows.values())
        report["relnorm_sums_hip_ref32"] = (sum_hip, sum_ref)
        assert unexplained == 0, (unexplained, report)
        print(f"resnet18 fp32 batch 64 seed {seed}:", report)
        for k, r in rows.items():
            print(f"  {k:42s} hip-ref32 {r['hip_vs_ref32']:7d}  hip-f64 {r['hip_vs_f64']:7d}  ref32-f64 "
                  f"{r['ref32_vs_f64']:7d}  |hip-f64| {r['relnorm_hip_f64']:.2e}  |ref32-f64| {r['relnorm_ref32_f64']:.2e}")
        # Both fp32 computations are as far from float64 as each other, in
        # sum: per tensor the distances swing both ways with the ReLU branches
        # an implementation happens to flip (measured over seeds 1-4 and 17:
        # HIP from 0.002x to 273x the reference's distance on single tensors,
        # their sums over the 56 tensors within 0.86-1.66x, the elementwise
        # counts within 0.9-2.0x, every tensor below 2.7e-3 in both).
        for k, r in rows.items():
            assert r["relnorm_hip_f64"] <= 5e-3, (k, r)
        assert sum_hip <= 2 * sum_ref, report
        assert tot["hip_vs_f64"] <= 2.5 * tot["ref32_vs_f64"] + 100, tot
        for k, v in bufs.items():
            if k.endswith("num_batches_tracked"):
                assert int(v) == 1, (k, v)
            else:
                c, w = _strict(v, rafter[k], 1e-4, 1e-5)
                assert c == 0, (k, c, w)
    else:
        # The same reference computation with bf16 storage where this path
        # stores bf16 (activations and activation gradients), fp32 arithmetic.
        eloss, _, egrads, _, eblocks = ref.resnet18_step(xr, y, vals, 1e-3, 1e-2, want_blocks=True,
                                                         precision="bf16_storage")
        report["loss_bf16_storage_ref"] = eloss
        report["relu_flips_vs_bf16_storage_ref"] = [int(((a > 0) != (b > 0)).sum()) for a, b in zip(outs, eblocks)]
        report["grad_relnorm_vs_ref32_max"] = max(_rel(grads[k], rgrads[k]) for k in rgrads)
        report["grad_relnorm_bf16ref_vs_ref32_max"] = max(_rel(egrads[k], rgrads[k]) for k in rgrads)
        report["grad_relnorm_vs_bf16_storage_ref"] = {k: round(_rel(grads[k], egrads[k]), 5) for k in sorted(egrads)}
        rows = {}
        for k in sorted(rgrads):
            rows[k] = (_rel(grads[k], rgrads[k]), _rel(egrads[k], rgrads[k]))
        report["grad_elements_out_of_rel2e-2_vs_ref32"] = int(sum(
            _strict(grads[k], rgrads[k], 2e-2, 2e-2 * float(np.sqrt(np.mean(rgrads[k].astype(np.float64) ** 2))))[0]
            for k in rgrads))
        print("resnet18 bf16 batch 64:", report)
        for k, (a, b) in rows.items():
            print(f"  {k:42s} |hip-ref32| {a:.3e}  |bf16ref-ref32| {b:.3e}")
        assert abs(loss - eloss) <= 2e-2 * abs(eloss), report
        assert abs(loss - rloss) <= 2e-2 * abs(rloss), report
        # What bf16 storage itself costs: the reference computation with the
        # same bf16 storage is as far from the fp32 reference.  The HIP path
        # may not add more than half as much again on any tensor.
        for k, (a, b) in rows.items():
            assert a <= 1.5 * b + 1e-3, (k, a, b)
        for k in p0:
            pe, _, _ = oracle_adam(p0[k], grads[k], 1)
            assert np.array_equal(after[k], pe), k


def oracle_adam(p, gr, step):
    from oracle_lib import Oracle
    z = np.zeros_like(p)
    return Oracle().adam_step(1, p, gr, z, z, 1e-3, 0.9, 0.999, 1e-8, 1e-2, step)


def test_resnet18_checkpoint_loads_into_reference(host_mod, tmp_path):
    """parameters.binary of the HIP ResNet-18 (every tensor under Nott's
    registration keys, residual_block_<i>.conv2d_0.weight ...) loads into the
    reference's ResNet-18, whose CPU forward then matches the GPU forward."""
    from oracle_lib import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built")
    tr = host_mod.ResNet18Trainer(0, 23, False, 1e-3, 1e-2, 1000)
    g = rng(77)
    x = f32(g.uniform(0, 1, (4, 3, 224, 224)))
    y = g.integers(0, 1000, 4).astype(np.int64)
    tr.step(torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda())
    path = str(tmp_path / "parameters.binary")
    tr.save(path)
    got = host(tr.forward(torch.from_numpy(x).cuda()))
    want = Ref().resnet18_forward_archive(path, x)
    check(got, want, "f32", "ResNet-18 logits after checkpoint round trip")


def test_resnet18_loss_decreases(host_mod):
    """A few AdamW steps on one fixed batch drive the loss down (bf16 mixed precision)."""
    tr = host_mod.ResNet18Trainer(0, 3, True, 1e-3, 1e-2, 1000)
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.rand((8, 3, 224, 224), generator=gen, device="cuda")
    y = torch.randint(0, 1000, (8,), generator=gen, device="cuda")
    losses = [tr.step(x, y).item() for _ in range(6)]
    assert all(math.isfinite(l) for l in losses)
    assert losses[-1] < losses[0], losses


@pytest.mark.parametrize("model", ["small_cnn", "resnet18_bf16"])
def test_graph_step_matches_eager(host_mod, model):
    """The HIP-graph step (forward + loss + backward captured once, replayed
    per step; fused AdamW eager) against the eager step on a twin trainer
    that does no warm-up: every replay, with eager work and synchronisations
    between replays, must give the same loss and, at the end, the same
    parameters and buffers (BatchNorm running statistics, batch counters) bit
    for bit — the capture's warm-up passes leave no trace in the model."""
    def make():
        if model == "small_cnn":
            return host_mod.SmallCNNTrainer(0, 11, 1e-3)
        return host_mod.ResNet18Trainer(0, 11, True, 1e-3, 1e-2, 1000)
    eager, graphed = make(), make()
    gen = torch.Generator(device="cuda").manual_seed(9)
    shape, classes = ((16, 1, 28, 28), 10) if model == "small_cnn" else ((4, 3, 224, 224), 1000)
    batches = [(torch.rand(shape, generator=gen, device="cuda"),
                torch.randint(0, classes, (shape[0],), generator=gen, device="cuda")) for _ in range(4)]
    x0, y0 = batches[0]
    graphed.capture(x0, y0, 2)
    for i, (x, y) in enumerate(batches):
        le = eager.step(x, y)
        lg = graphed.step_graph(x, y)
        torch.cuda.synchronize()
        assert torch.equal(le, lg), (i, le.item(), lg.item())
        _ = (x * 2).sum().item()          # unrelated eager work between replays
    pe, pg = eager.params(), graphed.params()
    be, bg = eager.buffers(), graphed.buffers()
    torch.cuda.synchronize()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k
    for k in be:
        assert torch.equal(be[k], bg[k]), k


@pytest.mark.parametrize("bf16", [False, True])
def test_side_stream_weight_gradients_match_one_stream(host_mod, bf16):
    """Trainers run the large convolution weight gradients on a side stream
    (their own context and workspace, joined after backward).  The same step
    with the side stream switched off gives bit-identical gradients, loss and
    updated parameters: the kernels and their summation orders do not depend
    on the stream."""
    gen = torch.Generator(device="cuda").manual_seed(77)
    x = torch.rand((8, 3, 224, 224), generator=gen, device="cuda")
    y = torch.randint(0, 1000, (8,), generator=gen, device="cuda")
    results = []
    try:
        for on in (True, False):
            host_mod.set_side_stream(on)
            tr = host_mod.ResNet18Trainer(0, 19, bf16, 1e-3, 1e-2, 1000)
            loss = tr.step(x, y)
            torch.cuda.synchronize()
            results.append((loss.clone(), {k: v.clone() for k, v in tr.params().items()}))
            tr2 = host_mod.ResNet18Trainer(0, 19, bf16, 1e-3, 1e-2, 1000)
            tr2.forward_backward(x, y)
            torch.cuda.synchronize()
            results[-1] += ({k: v.clone() for k, v in tr2.grads().items()},)
    finally:
        host_mod.set_side_stream(True)
    (l1, p1, g1), (l2, p2, g2) = results
    assert torch.equal(l1, l2), (l1.item(), l2.item())
    assert set(g1) == set(g2) and len(g1) > 0
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
    for k in p1:
        assert torch.equal(p1[k], p2[k]), k


def test_graph_replay_after_workspace_growth(host_mod):
    """A captured graph keeps the workspace pointers it was recorded with (the
    device context's and the weight-gradient side stream's).  An eager step at
    a larger batch on the same device afterwards must grow the workspace
    without freeing the captured one, so later replays still match an eager
    twin bit for bit."""
    eager = host_mod.ResNet18Trainer(0, 13, True, 1e-3, 1e-2, 1000)
    graphed = host_mod.ResNet18Trainer(0, 13, True, 1e-3, 1e-2, 1000)
    gen = torch.Generator(device="cuda").manual_seed(31)
    batches = [(torch.rand((2, 3, 224, 224), generator=gen, device="cuda"),
                torch.randint(0, 1000, (2,), generator=gen, device="cuda")) for _ in range(3)]
    graphed.capture(*batches[0], 1)
    before = host_mod.workspace_bytes(0)
    other = host_mod.ResNet18Trainer(0, 5, True, 1e-3, 1e-2, 1000)
    for b in (32, 64, 128, 256):   # the workspace is shared by the whole process: grow it past its current size
        other.step(torch.rand((b, 3, 224, 224), generator=gen, device="cuda"),
                   torch.randint(0, 1000, (b,), generator=gen, device="cuda"))
        torch.cuda.synchronize()
        if host_mod.workspace_bytes(0) > before:
            break
    assert host_mod.workspace_bytes(0) > before, (before, host_mod.workspace_bytes(0))
    del other
    for i, (x, y) in enumerate(batches):
        le = eager.step(x, y)
        lg = graphed.step_graph(x, y)
        torch.cuda.synchronize()
        assert torch.equal(le, lg), (i, le.item(), lg.item())
    pe, pg = eager.params(), graphed.params()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k


def test_checkpoint_loads_into_reference(host_mod, oracle, tmp_path):
    """parameters.binary written by the HIP trainer (torch::nn::Module::save
    layout, Nott's registration keys) loads into the configs[0] model built
    from the reference's own layer descriptors, whose CPU forward then
    matches the GPU forward (fp32)."""
    from oracle_lib import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built")
    tr = host_mod.SmallCNNTrainer(0, 21, 1e-3)
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.rand((8, 1, 28, 28), generator=gen, device="cuda")
    y = torch.randint(0, 10, (8,), generator=gen, device="cuda")
    tr.step(x, y)
    path = str(tmp_path / "parameters.binary")
    tr.save(path)
    got = tr.forward(x).float().cpu().numpy()
    want = Ref().small_cnn_forward_archive(path, x.cpu().numpy())
    check(got, want, "f32", "logits after checkpoint round trip")


def test_graph_optimizer_follows_scheduler(host_mod):
    """The optimizer step inside the captured graph reads its learning rate
    at replay time: a scheduler-style set_lr between replays (cosine-like
    sequence) gives the same parameters, bit for bit, as the eager twin that
    steps through torch::optim::Optimizer::step with the same writes; the
    per-parameter step counts advance with the replays."""
    eager = host_mod.SmallCNNTrainer(0, 41, 1e-3)
    graphed = host_mod.SmallCNNTrainer(0, 41, 1e-3)
    gen = torch.Generator(device="cuda").manual_seed(12)
    batches = [(torch.rand((32, 1, 28, 28), generator=gen, device="cuda"),
                torch.randint(0, 10, (32,), generator=gen, device="cuda")) for _ in range(5)]
    graphed.capture(*batches[0], 1)
    lrs = [1e-3, 8e-4, 5e-4, 2e-4, 5e-5]
    for (x, y), lr in zip(batches, lrs):
        eager.set_lr(lr)
        graphed.set_lr(lr)
        le = eager.step(x, y)
        lg = graphed.step_graph(x, y)
        torch.cuda.synchronize()
        assert torch.equal(le, lg), (lr, le.item(), lg.item())
    pe, pg = eager.params(), graphed.params()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k
    # an eager step after the replays continues the same step count
    x, y = batches[0]
    eager.step(x, y)
    graphed.step(x, y)
    lg = graphed.step_graph(x, y)
    le = eager.step(x, y)
    torch.cuda.synchronize()
    assert torch.equal(le, lg)
    pe, pg = eager.params(), graphed.params()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k


def test_graph_lr_change_between_queued_replays(host_mod):
    """Learning-rate writes between replays that are still queued on the GPU
    (no host synchronisation anywhere in the loop, the device held busy by
    matrix products first so the host runs ahead): each replay must use the
    lr set before it, as the eager twin does, bit for bit."""
    eager = host_mod.SmallCNNTrainer(0, 43, 1e-3)
    graphed = host_mod.SmallCNNTrainer(0, 43, 1e-3)
    gen = torch.Generator(device="cuda").manual_seed(13)
    batches = [(torch.rand((32, 1, 28, 28), generator=gen, device="cuda"),
                torch.randint(0, 10, (32,), generator=gen, device="cuda")) for _ in range(6)]
    graphed.capture(*batches[0], 1)
    lrs = [1e-3, 7e-4, 4e-4, 4e-4, 1e-4, 3e-5]
    torch.cuda.synchronize()
    a = torch.randn((4096, 4096), device="cuda")
    for _ in range(20):
        a = torch.tanh(a @ a)      # keeps the stream busy while the replays queue
    lg = []
    for (x, y), lr in zip(batches, lrs):
        graphed.set_lr(lr)
        lg.append(graphed.step_graph(x, y))
    torch.cuda.synchronize()
    for (x, y), lr, l in zip(batches, lrs, lg):
        eager.set_lr(lr)
        le = eager.step(x, y)
        torch.cuda.synchronize()
        assert torch.equal(le, l), (lr, le.item(), l.item())
    pe, pg = eager.params(), graphed.params()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k


@pytest.mark.parametrize("model", ["small_cnn", "resnet18_bf16"])
def test_train_epoch_prefetch_matches_steps(host_mod, model):
    """One epoch from pinned host memory (batch i+1 copied on a copy stream
    while step i replays; the loss summed on the device in float64 as
    Model::run_epochs accumulates it) against eager steps over the same
    batches: the same parameters bit for bit and the same mean loss."""
    def make():
        if model == "small_cnn":
            return host_mod.SmallCNNTrainer(0, 17, 1e-3)
        return host_mod.ResNet18Trainer(0, 17, True, 1e-3, 1e-2, 1000)
    eager, graphed = make(), make()
    b, nb = (32, 6) if model == "small_cnn" else (4, 3)
    shape, classes = ((1, 28, 28), 10) if model == "small_cnn" else ((3, 224, 224), 1000)
    g = torch.Generator().manual_seed(23)
    xs = torch.rand((b * nb, *shape), generator=g).pin_memory()
    ys = torch.randint(0, classes, (b * nb,), generator=g).pin_memory()
    graphed.capture(xs[:b].cuda(), ys[:b].cuda(), 1)
    mean = graphed.train_epoch(xs, ys)
    total = 0.0
    for i in range(nb):
        loss = eager.step(xs[i * b:(i + 1) * b].cuda(), ys[i * b:(i + 1) * b].cuda())
        total += float(loss.item()) * b
    torch.cuda.synchronize()
    assert mean == total / (b * nb), (mean, total / (b * nb))
    pe, pg = eager.params(), graphed.params()
    for k in pe:
        assert torch.equal(pe[k], pg[k]), k


@pytest.mark.parametrize("model", ["small_cnn", "resnet18"])
def test_reference_checkpoint_loads_into_hip_model(host_mod, tmp_path, model):
    """parameters.binary written by the reference's own model (its layer
    factories' initialisation, BatchNorm statistics after a training-mode
    forward) loads into the HIP model by registration key (Model::load,
    core.hpp:2140-2244): the HIP forward (fp32, training mode) matches the
    reference's forward on the same archive, and the BatchNorm buffers and
    batch counters come through unchanged."""
    from oracle_lib import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built")
    ref = Ref()
    path = str(tmp_path / "parameters.binary")
    ref.save_archive(model, 99, 4, path)
    if model == "small_cnn":
        tr = host_mod.SmallCNNTrainer(0, 1, 1e-3)
        x = f32(rng(8).uniform(0, 1, (4, 1, 28, 28)))
        want = ref.small_cnn_forward_archive(path, x)
    else:
        tr = host_mod.ResNet18Trainer(0, 1, False, 1e-3, 1e-2, 1000)
        x = f32(rng(8).uniform(0, 1, (4, 3, 224, 224)))
        want = ref.resnet18_forward_archive(path, x)
    tr.load_archive(path)
    if model == "resnet18":
        # Read before the forward: a training-mode forward counts one more batch.
        bufs = tr.buffers()
        assert int(bufs["batchnorm2d_1.num_batches_tracked"]) == 1
        assert float(bufs["batchnorm2d_1.running_var"].float().std()) > 0
    got = host(tr.forward(torch.from_numpy(x).cuda()))
    check(got, want, "f32", f"{model} logits from a reference checkpoint")
    if model == "resnet18":
        assert int(tr.buffers()["batchnorm2d_1.num_batches_tracked"]) == 2


@pytest.mark.parametrize("model", ["small_cnn", "resnet18"])
def test_model_directory_round_trip(host_mod, tmp_path, model):
    """Model::save's directory (core.hpp:2088-2137: <dir>/<name>/ with
    architecture.json and parameters.binary; an existing directory leads to
    <name>_1, the reference's default answer) loads back through
    Model::load's checks (core.hpp:2140-2244) into a fresh model: same
    parameters and buffers, same name; an architecture.json of another
    model is refused."""
    def make(seed):
        if model == "small_cnn":
            return host_mod.SmallCNNTrainer(0, seed, 1e-3)
        return host_mod.ResNet18Trainer(0, seed, False, 1e-3, 1e-2, 1000)
    a = make(3)
    if model == "small_cnn":
        x, y = torch.rand(8, 1, 28, 28).cuda(), torch.randint(0, 10, (8,)).cuda()
    else:
        x, y = torch.rand(2, 3, 224, 224).cuda(), torch.randint(0, 1000, (2,)).cuda()
    a.step(x, y)
    a.set_model_name("net")
    d1 = a.save_model(str(tmp_path))
    d2 = a.save_model(str(tmp_path))
    assert d1.endswith("/net") and d2.endswith("/net_1")
    with open(f"{d1}/architecture.json") as f:
        assert f.read() == a.architecture_json()
    b = make(4)
    b.load_model(d2)
    assert b.model_name() == "net"
    pa, pb = a.params(), b.params()
    for k in pa:
        assert torch.equal(pa[k], pb[k]), k
    ba, bb = a.buffers(), b.buffers()
    for k in ba:
        assert torch.equal(ba[k].cpu(), bb[k].cpu()), k
    other = "resnet18" if model == "small_cnn" else "small_cnn"
    with open(f"{d1}/architecture.json", "w") as f:
        f.write(host_mod.architecture_json(other))
    with pytest.raises(RuntimeError, match="describes another model"):
        b.load_model(d1)
