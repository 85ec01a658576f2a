"""Nott's layer factory on the HIP modules (include/nott_hip/registry.hpp), CPU part.

The test module (tests/factory/nott_factory.cpp) is compiled against the
reference's own headers: configs[0] is assembled from the reference's
descriptors through its std::variant dispatch of build_registered_layer
(src/layer/registry.hpp:193-200), with an owner opted in to the HIP
overloads.  These tests check what that build produces without running a
kernel: every layer is a Nott::HIP module under the reference's registration
key, ReLU is fused (the registered activation is Identity), the initial
weights are bit for bit those of the reference's own factory after the same
torch::manual_seed (oracle/_ref), and the option checks throw as the
reference's do, or say that the HIP path does not take the option."""
import numpy as np
import pytest

import factory_util

F = factory_util.load()
pytestmark = pytest.mark.skipif(F is None, reason="factory test module not built (needs the reference headers)")


def test_small_cnn_layers_are_hip_modules_under_reference_keys():
    s = F.SmallCnnFactory(0)
    assert s.modules() == [("conv2d_0", "hip.Conv2d"), ("maxpool2d_1", "hip.MaxPool2d"),
                           ("conv2d_2", "hip.Conv2d"), ("maxpool2d_3", "hip.MaxPool2d"),
                           ("flatten_4", "hip.Flatten"), ("fc_5", "hip.Linear"), ("fc_6", "hip.Linear")]
    # ReLU runs inside the HIP layers; Model::forward's activation dispatch is a no-op.
    assert s.activations() == ["identity"] * 7
    shapes = {k: tuple(v.shape) for k, v in s.params().items()}
    assert shapes == {"conv2d_0.weight": (32, 1, 3, 3), "conv2d_0.bias": (32,),
                      "conv2d_2.weight": (64, 32, 3, 3), "conv2d_2.bias": (64,),
                      "fc_5.weight": (128, 3136), "fc_5.bias": (128,),
                      "fc_6.weight": (10, 128), "fc_6.bias": (10,)}


@pytest.mark.parametrize("seed", [0, 99])
def test_initial_weights_equal_reference_factory(ref, seed):
    """Same seed, same descriptors: the HIP factory's weights are the
    reference factory's, bit for bit (the torch::nn constructor's default
    draws, then HeUniform and zero biases from apply_module_initialization)."""
    mine = {k: v.numpy() for k, v in F.SmallCnnFactory(seed).params().items()}
    want = ref.init_params("small_cnn", seed, {k: v.shape for k, v in mine.items()})
    for k in sorted(mine):
        assert np.array_equal(mine[k], want[k]), k


@pytest.mark.parametrize("case,want", [
    ("conv", "conv2d_0 hip.Conv2d 1 1 1 1 1 1"),
    ("conv_strided_rect", "conv2d_0 hip.Conv2d 2 1 0 1 1 1"),
    ("maxpool_3s2p1", "maxpool2d_0 hip.MaxPool2d 3 3 2 2 1 1 1 1 0"),
    # torch's MaxPool2dOptions: the stride defaults to the window
    ("maxpool_default_stride", "maxpool2d_0 hip.MaxPool2d 3 3 3 3 1 1 1 1 1"),
    ("bn", "batchnorm2d_0 hip.BatchNorm2d"),
    ("adaptive_avg_1x1", "adaptive_avgpool2d_0 hip.AdaptiveAvgPool2d"),
    ("flatten", "flatten_0 hip.Flatten"),
])
def test_layer_geometry_and_keys(case, want):
    assert F.build_one(case) == want


def test_other_layers_keep_the_reference_factory():
    """A descriptor with no HIP overload is built by the reference's own
    factory, unchanged."""
    assert F.build_one("dropout") == "hard_dropout_0 other:Nott::Layer::Details::HardDropoutImpl"


@pytest.mark.parametrize("case,exc,msg", [
    # the reference's own checks, same exception type and text
    ("conv_zero_channels", ValueError, "Conv2d layers require positive channel counts."),
    ("conv_bad_mode", ValueError, "Unsupported padding mode provided to Conv2d descriptor: mirror"),
    ("fc_zero", ValueError, "Fully connected layers require positive in/out features."),
    ("conv_three_kernel_values", RuntimeError, "Expected 2 values, but instead got 3"),
    # options the HIP kernels do not implement
    ("conv_groups", ValueError, "grouped convolution is not supported"),
    ("conv_reflect", ValueError, "padding mode 'reflect' is not supported"),
    ("bn_no_affine", ValueError, "only affine=true"),
    ("bn_no_stats", ValueError, "only affine=true"),
    ("avgpool2d", ValueError, "only MaxPool2d and AdaptiveAvgPool2d"),
    ("adaptive_max", ValueError, "only MaxPool2d and AdaptiveAvgPool2d"),
    ("adaptive_avg_2x2", ValueError, "only a 1x1 output"),
])
def test_option_errors(case, exc, msg):
    with pytest.raises(exc, match=msg.replace("(", r"\(").replace(")", r"\)").replace(".", r"\.")):
        F.build_one(case)
