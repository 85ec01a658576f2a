"""CPU checks of the C ABI: the library loads without a GPU, exports every
function include/nott_hip.h declares, and the Python binding covers them."""
import os
import re
import subprocess

import pytest

from thot_amd import _abi

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "nott_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nott_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    for need in ("nott_conv2d_bwd_data", "nott_conv2d_bwd_weight", "nott_linear_bwd", "nott_relu_bwd",
                 "nott_maxpool2d_bwd", "nott_batchnorm2d_bwd", "nott_avgpool_global_bwd", "nott_layernorm_bwd",
                 "nott_softmax_xent_bwd", "nott_attention_bwd", "nott_adam_step"):
        assert need in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_abi.LIB_PATH), "build with python -m thot_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(nott_[a-z0-9_]+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(_abi.SIGNATURES) == declared_functions()


def test_load_without_gpu_and_error_paths():
    import ctypes as C
    lib = _abi.load()
    assert _abi.missing_symbols() == []
    assert lib.nott_abi_version() == 1
    assert lib.nott_status_string(_abi.NOTT_ERR_INVALID_ARG) == b"invalid argument"
    h = C.c_void_p()
    assert lib.nott_create(-1, C.byref(h)) == _abi.NOTT_ERR_INVALID_ARG
    assert lib.nott_create(0, None) == _abi.NOTT_ERR_INVALID_ARG
    # a null context is rejected by every entry point, before any launch
    assert lib.nott_adam_step(None, 1, 4, None, 0, None, 0, None, None, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0) == \
        _abi.NOTT_ERR_INVALID_ARG
    assert lib.nott_last_error(None) == b"null context"


def test_product_never_references_the_oracle():
    """The product path must not load or link the CPU checkers."""
    for root in (os.path.join(REPO, "thot_amd"), os.path.join(REPO, "include")):
        for dirpath, _, files in os.walk(root):
            for f in files:
                if f.endswith((".py", ".hip", ".hpp", ".h", ".cpp")):
                    text = open(os.path.join(dirpath, f), errors="ignore").read()
                    assert "liboracle" not in text and "nott_ref" not in text and "oracle_lib" not in text, f
