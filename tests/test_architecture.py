"""architecture.json written by the HIP host (Nott::HIP::arch) for the
checkpointed models, read the way the reference's Model::load reads it.

Model::load (reference src/core.hpp:2140-2183) parses the file with Boost,
deserialises the module list (common/save_load.hpp:3159-3200; layers
2390-2525, residual blocks 2941-2956) and replays add(); the parameter
archive is then checked key by key and shape by shape (core.hpp:2196-2236).
Boost is absent from this image, so that reader cannot run here.  These
tests restate it: every field the deserialisers read must be present and
parse as the type they read it as, and the model the descriptors describe,
registered under the reference's keys (conv.hpp:177, batchnorm.hpp:50,
pooling.hpp:144,164, flatten.hpp:61, fc.hpp:40, core.hpp:580 for blocks),
must have exactly the parameters and buffers, with the shapes, that the
reference's own model of that configuration writes to parameters.binary
(oracle/_ref builds that model from the reference's layer factories).
"""
import json

import pytest
import torch

from oracle_lib import Ref

host = pytest.importorskip("thot_amd._nott_host")


def boolean(v, where):
    # ptree get<bool>: "true"/"false", then 1/0 (save_load.hpp:75-84)
    assert isinstance(v, str), where
    assert v in ("true", "false", "1", "0"), where
    return v in ("true", "1")


def integer(v, where):
    assert isinstance(v, str), where
    return int(v)


def number(v, where):
    assert isinstance(v, str), where
    return float(v)


def int_array(v, where):
    # Detail::read_array over the node's children (save_load.hpp:97-116)
    assert isinstance(v, list), where
    return [integer(e, where) for e in v]


def string(d, key, where):
    assert isinstance(d[key], str), f"{where}.{key}"
    return d[key]


def common(d, where, init=True):
    string(d["activation"], "type", where + ".activation")
    if init:
        string(d["initialization"], "type", where + ".initialization")
    loc = d["local"]
    assert isinstance(loc, dict), where
    # an empty regularization list is written by Boost as ""
    assert loc.get("regularization", "") in ("", []), where


def layer(d, where):
    """deserialize_layer_descriptor (save_load.hpp:2390-2525) for the layer
    types of the checkpointed models; returns (kind, parameter shapes)."""
    t = string(d, "type", where).lower()
    o = d["options"]
    if t == "conv2d":
        ci, co = integer(o["in_channels"], where), integer(o["out_channels"], where)
        k = int_array(o["kernel_size"], where)
        for f in ("stride", "padding", "dilation"):
            int_array(o[f], where)
        groups = integer(o["groups"], where)
        bias = boolean(o["bias"], where)
        string(o, "padding_mode", where)
        common(d, where)
        shapes = {"weight": (co, ci // groups, *k)}
        if bias:
            shapes["bias"] = (co,)
        return "conv2d", shapes
    if t == "fc":
        i, n = integer(o["in_features"], where), integer(o["out_features"], where)
        bias = boolean(o["bias"], where)
        common(d, where)
        shapes = {"weight": (n, i)}
        if bias:
            shapes["bias"] = (n,)
        return "fc", shapes
    if t == "batch_norm2d":
        c = integer(o["num_features"], where)
        number(o["eps"], where)
        number(o["momentum"], where)
        affine = boolean(o["affine"], where)
        track = boolean(o["track_running_stats"], where)
        common(d, where)
        shapes = {}
        if affine:
            shapes.update(weight=(c,), bias=(c,))
        if track:
            shapes.update(running_mean=(c,), running_var=(c,), num_batches_tracked=())
        return "batchnorm2d", shapes
    if t == "pooling":
        v = string(o, "variant", where).lower()
        common(d, where, init=False)
        if v == "max2d":
            for f in ("kernel_size", "stride", "padding", "dilation"):
                int_array(o[f], where)
            boolean(o["ceil_mode"], where)
            return "maxpool2d", {}
        if v == "adaptive_avg2d":
            int_array(o["output_size"], where)
            return "adaptive_avgpool2d", {}
        raise AssertionError(f"{where}: pooling variant {v}")
    if t == "flatten":
        integer(o["start_dim"], where)
        integer(o["end_dim"], where)
        common(d, where, init=False)
        return "flatten", {}
    raise AssertionError(f"{where}: layer type {t}")


def expected_state(arch):
    """Registration keys and shapes of the model the file describes: each
    module registered as <kind>_<index> in add() order (core.hpp:516-523),
    a residual block as residual_block_<index> holding its layers and then
    its projection under running indices (residual.hpp:49-62)."""
    assert isinstance(arch["name"], str)
    out = {}
    for i, m in enumerate(arch["modules"]):
        where = f"modules[{i}]"
        kind = m["kind"].lower()
        d = m["descriptor"]
        if kind == "layer":
            k, shapes = layer(d, where)
            for name, s in shapes.items():
                out[f"{k}_{i}.{name}"] = s
            continue
        assert kind == "block" and d["type"] == "residual", where
        integer(d["repeats"], where)
        number(d["output"]["dropout"], where)
        string(d["output"]["final_activation"], "type", where)
        sub = list(d["layers"])
        proj = d.get("skip", {}).get("projection")
        if proj is not None:
            sub.append(proj)
        for j, ld in enumerate(sub):
            k, shapes = layer(ld, f"{where}.layers[{j}]")
            for name, s in shapes.items():
                out[f"residual_block_{i}.{k}_{j}.{name}"] = s
    return out


@pytest.mark.parametrize("model", ["small_cnn", "resnet18"])
def test_architecture_describes_reference_archive(tmp_path, model):
    if not Ref.available():
        pytest.skip("oracle/_ref not built")
    text = host.architecture_json(model)
    arch = json.loads(text)
    want = expected_state(arch)
    path = str(tmp_path / "parameters.binary")
    Ref().save_archive(model, 5, 2, path)
    got = {k: tuple(v.shape) for k, v in torch.jit.load(path).state_dict().items()}
    assert want == got


def test_architecture_json_is_boost_form():
    """write_json's form: 4-space indentation, every scalar a quoted string,
    floats with 17 significant digits, empty nodes as "", a newline at the
    end (boost/property_tree/json_parser write_json_helper)."""
    text = host.architecture_json("resnet18", 10, "ResNet/18")
    assert text.endswith("}\n")
    assert '"name": "ResNet\\/18"' in text
    arch = json.loads(text)
    assert arch["name"] == "ResNet/18"

    def leaves(n):
        if isinstance(n, dict):
            for v in n.values():
                yield from leaves(v)
        elif isinstance(n, list):
            for v in n:
                yield from leaves(v)
        else:
            yield n

    assert all(isinstance(v, str) for v in leaves(arch))
    bn = arch["modules"][1]["descriptor"]["options"]
    assert bn["eps"] == "1.0000000000000001e-05" and bn["momentum"] == "0.10000000000000001"
    assert float(bn["eps"]) == 1e-5
    assert arch["modules"][-1]["descriptor"]["options"]["out_features"] == "10"
    assert arch["modules"][0]["descriptor"]["local"] == {"regularization": ""}
    lines = text.splitlines()
    assert lines[1] == '    "name": "ResNet\\/18",'
    assert lines[2] == '    "modules": ['


def test_block_shapes():
    """Down-sampling blocks carry a 1×1 stride-2 projection, the others none
    (residual.hpp:18-20, 99-104)."""
    arch = json.loads(host.architecture_json("resnet18"))
    blocks = [m["descriptor"] for m in arch["modules"] if m["kind"] == "block"]
    assert len(blocks) == 8
    proj = [b.get("skip", {}).get("projection") for b in blocks]
    assert [p is not None for p in proj] == [False, False, True, False, True, False, True, False]
    for p in proj:
        if p is not None:
            assert p["options"]["kernel_size"] == ["1", "1"] and p["options"]["stride"] == ["2", "2"]
