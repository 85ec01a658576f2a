"""Initial weights of the host models against the reference's (CPU only).

A Nott model built from descriptors with HeUniform initialisation draws its
weights from torch's CPU generator: each layer factory constructs the
torch::nn module (its constructor draws the default initialisation) and then
applies the descriptor's initialisation (reference
src/initialization/apply.hpp:45-51, conv.hpp:182, fc.hpp:38).  The trainers
initialise from a seed the same way (Nott::HIP::reference_init_); these tests
check the result bit for bit against the reference's own models built in
oracle/_ref right after torch::manual_seed(seed), for configs[0] and
configs[4], and the HeUniform bound against its closed form.
"""
import math

import numpy as np
import pytest
import torch

host = pytest.importorskip("thot_amd._nott_host")


@pytest.mark.parametrize("model,seed", [("small_cnn", 0), ("small_cnn", 1234), ("resnet18", 7)])
def test_initial_parameters_match_reference(ref, model, seed):
    mine = {k: v.numpy() for k, v in host.initial_parameters(model, seed).items()}
    want = ref.init_params(model, seed, {k: v.shape for k, v in mine.items()})
    assert set(mine) == set(want)
    for k in sorted(mine):
        assert np.array_equal(mine[k], want[k]), f"{model} seed {seed}: {k} differs from the reference's draw"


@pytest.mark.parametrize("model", ["small_cnn", "resnet18"])
def test_initial_parameters_follow_he_uniform(model):
    """Weights lie inside the HeUniform bound sqrt(6 / fan_in) and fill it
    (max |w| within 2% of the bound for every layer with ≥ 2000 weights);
    conv/FC biases are zero, BatchNorm weights one and biases zero; another
    seed gives other weights."""
    a = host.initial_parameters(model, 3)
    b = host.initial_parameters(model, 4)
    for k, t in a.items():
        x = t.numpy()
        if k.endswith("weight") and x.ndim >= 2:
            bound = math.sqrt(6.0 / (x.size // x.shape[0]))
            assert np.abs(x).max() <= bound * (1 + 1e-6), k
            if x.size >= 2000:
                assert np.abs(x).max() >= 0.98 * bound, k
            assert not torch.equal(t, b[k]), k
        elif k.endswith("weight"):
            assert np.all(x == 1.0), k       # BatchNorm gamma
        else:
            assert np.all(x == 0.0), k       # biases
