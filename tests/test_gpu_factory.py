"""configs[0] assembled from the reference's own descriptors through Nott's
layer factory on the HIP modules (include/nott_hip/registry.hpp), trained on
the GPU.

The model is built by the test module tests/factory/nott_factory.cpp
(compiled against the reference's headers; see test_factory.py) with the
reference's HeUniform initialisation after torch::manual_seed, moved to the
GPU and stepped as Model::run_training_step does: forward through the
RegisteredLayers and their activations, mean cross-entropy, backward,
Nott::HIP::FusedAdam held as a torch::optim::Optimizer, step and
zero_grad(false) (core.hpp:3735-3827).  Two steps are checked against the
CPU oracle composed in the reference's order (loss, every gradient, every
updated parameter), and against the fixed-topology configs[0] trainer fed
the same weights and batches, which must agree bit for bit."""
import numpy as np
import pytest
import torch

import factory_util
from gpu_util import check, host
from oracle_lib import f32, rng
from test_gpu_train import small_cnn_oracle_step

pytestmark = pytest.mark.gpu

F = factory_util.load()


@pytest.mark.skipif(F is None, reason="factory test module not built (needs the reference headers)")
def test_factory_small_cnn_two_steps_vs_oracle(oracle):
    assert torch.cuda.is_available()
    from thot_amd import _nott_host
    s = F.SmallCnnFactory(5)
    P = {k: v.numpy().copy() for k, v in s.params().items()}
    s.to_device(0, 1e-3)
    twin = _nott_host.SmallCNNTrainer(0, 1, 1e-3)
    twin.load({k: torch.from_numpy(v).cuda() for k, v in P.items()})
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    g = rng(77)
    n = 64
    for step in (1, 2):
        x = f32(g.uniform(0, 1, (n, 1, 28, 28)))
        y = g.integers(0, 10, n).astype(np.int64)
        xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
        loss = s.forward_backward(xd, yd).item()
        grads = {k: host(v) for k, v in s.grads().items()}
        twin_loss = twin.forward_backward(xd, yd).item()
        twin_grads = {k: host(v) for k, v in twin.grads().items()}
        rloss, G = small_cnn_oracle_step(oracle, P, x, y)
        check(np.array([loss]), np.array([rloss]), what=f"loss step {step}")
        assert loss == twin_loss
        for k in P:
            check(grads[k], G[k], what=f"grad {k} step {step}")
            assert np.array_equal(grads[k], twin_grads[k]), k
        s.optimizer_step()
        twin.optimizer_step()
        for k in P:
            P[k], M[k], V[k] = oracle.adam_step(0, P[k], G[k], M[k], V[k], 1e-3, 0.9, 0.999, 1e-8, 0.0, step)
        params = {k: host(v) for k, v in s.params().items()}
        twin_params = {k: host(v) for k, v in twin.params().items()}
        for k in P:
            check(params[k], P[k], what=f"param {k} after step {step}")
            assert np.array_equal(params[k], twin_params[k]), k
        assert all(float(torch.count_nonzero(v)) == 0 for v in s.grads().values())
