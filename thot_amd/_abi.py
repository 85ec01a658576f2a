"""ctypes binding of libnott_hip.so (the C ABI declared in include/nott_hip.h).

The library is loaded from the package directory.  There is no fallback:
if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libnott_hip.so")

NOTT_OK = 0
NOTT_ERR_INVALID_ARG = -1
NOTT_ERR_UNSUPPORTED = -2
NOTT_ERR_HIP = -3
NOTT_ERR_ALLOC = -4
NOTT_ERR_DEVICE = -5

NOTT_F32 = 0
NOTT_BF16 = 1
NOTT_NCHW = 0
NOTT_NHWC = 1

i64 = C.c_int64
i32 = C.c_int
f64 = C.c_double
vp = C.c_void_p
fp = C.c_void_p  # float*: passed as raw device addresses


class Conv2dDesc(C.Structure):
    _fields_ = [(n, i64) for n in ("n", "c", "h", "w", "k", "r", "s", "stride_h", "stride_w",
                                    "pad_h", "pad_w", "dil_h", "dil_w", "groups")] + \
               [("layout", C.c_int32), ("reserved", C.c_int32)]


class Pool2dDesc(C.Structure):
    _fields_ = [(n, i64) for n in ("n", "c", "h", "w", "kh", "kw", "stride_h", "stride_w",
                                    "pad_h", "pad_w", "dil_h", "dil_w")] + \
               [("ceil_mode", C.c_int32), ("layout", C.c_int32)]


NOTT_ATTN_HEAD_MAJOR, NOTT_ATTN_TOKEN_MAJOR = 0, 1


class AttnDesc(C.Structure):
    _fields_ = [(n, i64) for n in ("b", "h", "t", "s", "dh")] + \
               [("causal", C.c_int32), ("layout", C.c_int32), ("scale", f64), ("ld_qkv", i64), ("ld_o", i64)]


# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "nott_create": [i32, C.POINTER(vp)],
    "nott_destroy": [vp],
    "nott_set_stream": [vp, vp],
    "nott_get_stream": [vp],
    "nott_last_error": [vp],
    "nott_status_string": [i32],
    "nott_abi_version": [],
    "nott_device_errors": [vp, C.POINTER(i64)],
    "nott_workspace_bytes": [vp, C.POINTER(i64)],
    "nott_conv2d_fwd": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, fp, vp],
    "nott_conv2d_fwd_act": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, fp, i32, vp],
    "nott_conv2d_bwd_data": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, vp],
    "nott_conv2d_dgrad_prep_bytes": [C.POINTER(Conv2dDesc), i32, C.POINTER(i64)],
    "nott_conv2d_fwd_prep": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, fp, i32, vp, vp],
    "nott_conv2d_bwd_data_prepped": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, vp],
    "nott_conv2d_bwd_weight": [vp, C.POINTER(Conv2dDesc), i32, vp, vp, fp, fp, i32],
    "nott_linear_fwd": [vp, i32, i64, i64, i64, vp, vp, fp, vp],
    "nott_linear_bwd": [vp, i32, i64, i64, i64, vp, vp, vp, vp, fp, fp, i32],
    "nott_linear_fwd_act": [vp, i32, i64, i64, i64, vp, vp, fp, i32, vp],
    "nott_linear_bwd_act": [vp, i32, i64, i64, i64, vp, vp, vp, vp, fp, fp, i32, i32],
    "nott_relu_fwd": [vp, i32, i64, vp, vp],
    "nott_relu_bwd": [vp, i32, i64, vp, vp, vp],
    "nott_maxpool2d_fwd": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp],
    "nott_maxpool2d_bwd": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp],
    "nott_maxpool2d_fwd_tap": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp],
    "nott_maxpool2d_bwd_tap": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp],
    "nott_maxpool2d_bwd_tap_relu": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp, vp],
    "nott_maxpool2d_fwd_tap_bnrelu": [vp, C.POINTER(Pool2dDesc), i32, vp, fp, vp, vp],
    "nott_batchnorm2d_relu_maxpool2d_bwd": [vp, C.POINTER(Pool2dDesc), i32, vp, vp, vp, fp, fp, fp, fp, vp, fp, fp,
                                            i32],
    "nott_avgpool_global_fwd": [vp, i32, i64, i64, vp, vp],
    "nott_avgpool_global_bwd": [vp, i32, i64, i64, vp, vp],
    "nott_batchnorm2d_fwd": [vp, i32, i64, i64, i64, vp, fp, fp, f64, f64, fp, fp, vp, fp, fp],
    "nott_batchnorm2d_fwd_coef": [vp, i32, i64, i64, i64, vp, fp, fp, f64, f64, fp, fp, fp, fp, fp],
    "nott_batchnorm2d_bwd": [vp, i32, i64, i64, i64, vp, vp, fp, fp, fp, vp, fp, fp, i32],
    "nott_batchnorm2d_fwd_act": [vp, i32, i64, i64, i64, vp, fp, fp, f64, f64, fp, fp, vp, i32, vp, fp, fp],
    "nott_batchnorm2d_bwd_act": [vp, i32, i64, i64, i64, vp, vp, fp, fp, fp, fp, i32, vp, fp, fp, i32],
    "nott_layernorm_fwd": [vp, i32, i64, i64, vp, vp, vp, f64, vp, fp, fp],
    "nott_layernorm_bwd": [vp, i32, i64, i64, vp, vp, fp, fp, vp, vp, fp, fp, i32],
    "nott_layernorm_bwd_noalloc": [vp, i32, i64, i64, vp, vp, fp, fp, vp, vp, fp, fp, i32],
    "nott_softmax_xent_bwd": [vp, i32, i64, i64, vp, vp, f64, f64, vp, fp],
    "nott_attention_fwd": [vp, C.POINTER(AttnDesc), i32, vp, vp, vp, vp, fp],
    "nott_attention_bwd": [vp, C.POINTER(AttnDesc), i32, vp, vp, vp, vp, vp, fp, vp, vp, vp],
    "nott_adam_step": [vp, i32, i64, vp, i32, vp, i32, fp, fp, f64, f64, f64, f64, f64, i64, i32],
    "nott_adam_step_graph": [vp, i32, i64, vp, i32, vp, i32, fp, fp, vp, vp, i32, i32],
    "nott_loss_accumulate": [vp, fp, f64, vp],
    "nott_add": [vp, i32, i64, vp, vp, vp],
    "nott_add_relu_bwd": [vp, i32, i64, vp, vp, vp, vp],
    "nott_cast": [vp, i64, vp, i32, vp, i32],
    "nott_zero": [vp, i64, vp],
    "nott_scale": [vp, i32, i64, vp, fp, vp],
}

_RESTYPES = {
    "nott_get_stream": vp,
    "nott_last_error": C.c_char_p,
    "nott_status_string": C.c_char_p,
}

_lib: C.CDLL | None = None


class NottError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{msg} (status {status})")
        self.status = status


class NottInvalidArgument(NottError, ValueError):
    pass


def load() -> C.CDLL:
    """Loads libnott_hip.so (after torch, so one HIP runtime serves both)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libnott_hip.so not built at {LIB_PATH}; run `python -m thot_amd.build` "
            "(there is no CPU or PyTorch fallback)")
    import torch  # noqa: F401  (binds libamdhip64.so.7 from the torch wheel first)
    lib = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
    for name, args in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue  # reported by missing_symbols(); calling it raises AttributeError
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().nott_status_string(status).decode()


def missing_symbols() -> list[str]:
    lib = load()
    out = []
    for name in SIGNATURES:
        try:
            getattr(lib, name)
        except AttributeError:
            out.append(name)
    return out
