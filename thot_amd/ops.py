"""Functional host layer over the C ABI: torch tensors in, torch tensors out.

Each function checks shapes, dtypes, devices and contiguity on the host,
allocates outputs with torch (device memory and streams only) and calls one
libnott_hip entry point on the caller's current HIP stream.  There is no
fallback path: a missing library or a failing launch raises.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional

import torch

from . import _abi
from ._abi import AttnDesc, Conv2dDesc, Pool2dDesc

_DTYPES = {torch.float32: _abi.NOTT_F32, torch.bfloat16: _abi.NOTT_BF16}


def nott_dtype(t: torch.dtype) -> int:
    if t not in _DTYPES:
        raise TypeError(f"unsupported dtype {t}; expected float32 or bfloat16")
    return _DTYPES[t]


class Context:
    """One nott_ctx per device; launches go to torch's current stream."""

    def __init__(self, device: int = 0):
        self.lib = _abi.load()
        self.device = device
        h = C.c_void_p()
        rc = self.lib.nott_create(device, C.byref(h))
        if rc != 0:
            raise _abi.NottError(rc, f"nott_create({device}) failed: {_abi.status_string(rc)}")
        self.handle = h

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self.lib.nott_destroy(self.handle)
        except Exception:
            pass

    def call(self, name: str, *args):
        self.lib.nott_set_stream(self.handle, C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))
        rc = getattr(self.lib, name)(self.handle, *args)
        if rc != 0:
            msg = self.lib.nott_last_error(self.handle).decode()
            cls = _abi.NottInvalidArgument if rc in (_abi.NOTT_ERR_INVALID_ARG, _abi.NOTT_ERR_UNSUPPORTED) else _abi.NottError
            raise cls(rc, f"{name}: {msg}")
        return rc

    def device_errors(self) -> int:
        n = C.c_int64()
        self.call("nott_device_errors", C.byref(n))
        return n.value

    def workspace_bytes(self) -> int:
        n = C.c_int64()
        self.call("nott_workspace_bytes", C.byref(n))
        return n.value


_contexts: dict[int, Context] = {}


def context(device: Optional[int] = None) -> Context:
    if device is None:
        device = torch.cuda.current_device()
    if device not in _contexts:
        _contexts[device] = Context(device)
    return _contexts[device]


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _check(t: torch.Tensor, name: str, shape=None, dtype=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _ctx_for(t: torch.Tensor) -> Context:
    return context(t.device.index)


# --------------------------------------------------------------------- adam
def adam_step(p: torch.Tensor, g: torch.Tensor, m: torch.Tensor, v: torch.Tensor, *, lr: float,
              beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.0,
              step: int, decoupled: bool, zero_grad: bool = False) -> None:
    """In-place fused Adam (decoupled=False) / AdamW (decoupled=True) step on flat buffers."""
    n = p.numel()
    _check(p, "p")
    _check(g, "g", shape=p.shape, device=p.device)
    _check(m, "m", shape=p.shape, dtype=torch.float32, device=p.device)
    _check(v, "v", shape=p.shape, dtype=torch.float32, device=p.device)
    _ctx_for(p).call("nott_adam_step", int(decoupled), n, _ptr(p), nott_dtype(p.dtype), _ptr(g), nott_dtype(g.dtype),
                     _ptr(m), _ptr(v), float(lr), float(beta1), float(beta2), float(eps), float(weight_decay),
                     int(step), int(zero_grad))


# ---------------------------------------------------------------- elementwise
def relu_fwd(x: torch.Tensor) -> torch.Tensor:
    _check(x, "x")
    y = torch.empty_like(x)
    _ctx_for(x).call("nott_relu_fwd", nott_dtype(x.dtype), x.numel(), _ptr(x), _ptr(y))
    return y


def relu_bwd(y: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    _check(y, "y")
    _check(dy, "dy", shape=y.shape, dtype=y.dtype, device=y.device)
    dx = torch.empty_like(dy)
    _ctx_for(y).call("nott_relu_bwd", nott_dtype(y.dtype), y.numel(), _ptr(y), _ptr(dy), _ptr(dx))
    return dx


def add(a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _check(a, "a")
    _check(b, "b", shape=a.shape, dtype=a.dtype, device=a.device)
    out = torch.empty_like(a) if out is None else out
    _check(out, "out", shape=a.shape, dtype=a.dtype, device=a.device)
    _ctx_for(a).call("nott_add", nott_dtype(a.dtype), a.numel(), _ptr(a), _ptr(b), _ptr(out))
    return out


def add_relu_bwd(a: torch.Tensor, b: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """dz = (y <= 0) ? 0 : a + b (the gradient of a ReLU output used twice)."""
    _check(a, "a")
    _check(b, "b", shape=tuple(a.shape), dtype=a.dtype, device=a.device)
    _check(y, "y", shape=tuple(a.shape), dtype=a.dtype, device=a.device)
    dz = torch.empty_like(a)
    _ctx_for(a).call("nott_add_relu_bwd", nott_dtype(a.dtype), a.numel(), _ptr(a), _ptr(b), _ptr(y), _ptr(dz))
    return dz


def cast(src: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    _check(src, "src")
    dst = torch.empty(src.shape, dtype=dtype, device=src.device)
    _ctx_for(src).call("nott_cast", src.numel(), _ptr(src), nott_dtype(src.dtype), _ptr(dst), nott_dtype(dtype))
    return dst


def zero_(t: torch.Tensor) -> torch.Tensor:
    _check(t, "t")
    _ctx_for(t).call("nott_zero", t.numel() * t.element_size(), _ptr(t))
    return t


# --------------------------------------------------------------- cross-entropy
def softmax_xent_bwd(logits: torch.Tensor, labels: torch.Tensor, *, label_smoothing: float = 0.0,
                     grad_scale: float = 1.0, with_loss: bool = True, out: Optional[torch.Tensor] = None):
    """Returns (dlogits, loss) of mean softmax cross-entropy (ignore_index -100)."""
    _check(logits, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be [n, c]")
    n, c = logits.shape
    _check(labels, "labels", shape=(n,), dtype=torch.int64, device=logits.device)
    dl = torch.empty_like(logits) if out is None else out
    _check(dl, "out", shape=logits.shape, dtype=logits.dtype, device=logits.device)
    loss = torch.empty((), dtype=torch.float32, device=logits.device) if with_loss else None
    _ctx_for(logits).call("nott_softmax_xent_bwd", nott_dtype(logits.dtype), n, c, _ptr(logits), _ptr(labels),
                          float(label_smoothing), float(grad_scale), _ptr(dl), _ptr(loss))
    return dl, loss


# ------------------------------------------------------------------ layernorm
def layernorm_fwd(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-5):
    _check(x, "x")
    rows, d = x.reshape(-1, x.shape[-1]).shape
    _check(gamma, "gamma", shape=(d,), dtype=x.dtype, device=x.device)
    _check(beta, "beta", shape=(d,), dtype=x.dtype, device=x.device)
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    _ctx_for(x).call("nott_layernorm_fwd", nott_dtype(x.dtype), rows, d, _ptr(x), _ptr(gamma), _ptr(beta),
                     float(eps), _ptr(y), _ptr(mean), _ptr(rstd))
    return y, mean, rstd


def layernorm_bwd(x: torch.Tensor, dy: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor, gamma: torch.Tensor,
                  dgamma: Optional[torch.Tensor] = None, dbeta: Optional[torch.Tensor] = None,
                  accumulate: bool = False, out: Optional[torch.Tensor] = None):
    _check(x, "x")
    rows, d = x.reshape(-1, x.shape[-1]).shape
    _check(dy, "dy", shape=x.shape, dtype=x.dtype, device=x.device)
    _check(mean, "mean", shape=(rows,), dtype=torch.float32, device=x.device)
    _check(rstd, "rstd", shape=(rows,), dtype=torch.float32, device=x.device)
    _check(gamma, "gamma", shape=(d,), dtype=x.dtype, device=x.device)
    dx = torch.empty_like(x) if out is None else out
    _check(dx, "out", shape=x.shape, dtype=x.dtype, device=x.device)
    if dgamma is None:
        dgamma = torch.empty(d, dtype=torch.float32, device=x.device)
    if dbeta is None:
        dbeta = torch.empty(d, dtype=torch.float32, device=x.device)
    _check(dgamma, "dgamma", shape=(d,), dtype=torch.float32, device=x.device)
    _check(dbeta, "dbeta", shape=(d,), dtype=torch.float32, device=x.device)
    _ctx_for(x).call("nott_layernorm_bwd", nott_dtype(x.dtype), rows, d, _ptr(x), _ptr(dy), _ptr(mean), _ptr(rstd),
                     _ptr(gamma), _ptr(dx), _ptr(dgamma), _ptr(dbeta), int(accumulate))
    return dx, dgamma, dbeta


# ------------------------------------------------------------------ batchnorm
def batchnorm2d_fwd(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-5,
                    momentum: float = 0.1, running_mean: Optional[torch.Tensor] = None,
                    running_var: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
                    relu: bool = False):
    """Training-mode BatchNorm2d; with `residual` / `relu` the fused
    y = act(BN(x) [+ residual]) of nott_batchnorm2d_fwd_act."""
    _check(x, "x")
    if x.dim() != 4:
        raise ValueError("x must be [n, c, h, w]")
    n, c, h, w = x.shape
    for t, nm in ((gamma, "gamma"), (beta, "beta")):
        _check(t, nm, shape=(c,), dtype=torch.float32, device=x.device)
    if (running_mean is None) != (running_var is None):
        raise ValueError("running_mean and running_var go together")
    if running_mean is not None:
        _check(running_mean, "running_mean", shape=(c,), dtype=torch.float32, device=x.device)
        _check(running_var, "running_var", shape=(c,), dtype=torch.float32, device=x.device)
    y = torch.empty_like(x)
    mean = torch.empty(c, dtype=torch.float32, device=x.device)
    rstd = torch.empty(c, dtype=torch.float32, device=x.device)
    if residual is None and not relu:
        _ctx_for(x).call("nott_batchnorm2d_fwd", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(gamma), _ptr(beta),
                         float(eps), float(momentum), _ptr(running_mean), _ptr(running_var), _ptr(y), _ptr(mean),
                         _ptr(rstd))
    else:
        if residual is not None:
            _check(residual, "residual", shape=x.shape, dtype=x.dtype, device=x.device)
        _ctx_for(x).call("nott_batchnorm2d_fwd_act", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(gamma),
                         _ptr(beta), float(eps), float(momentum), _ptr(running_mean), _ptr(running_var),
                         _ptr(residual), int(relu), _ptr(y), _ptr(mean), _ptr(rstd))
    return y, mean, rstd


def batchnorm2d_bwd(x: torch.Tensor, dy: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor, gamma: torch.Tensor,
                    dgamma: Optional[torch.Tensor] = None, dbeta: Optional[torch.Tensor] = None,
                    accumulate: bool = False, beta: Optional[torch.Tensor] = None, relu: bool = False):
    """BatchNorm2d backward; with relu=True, dy is the gradient w.r.t.
    relu(BN(x)) and `beta` is required (nott_batchnorm2d_bwd_act)."""
    _check(x, "x")
    if x.dim() != 4:
        raise ValueError("x must be [n, c, h, w]")
    n, c, h, w = x.shape
    _check(dy, "dy", shape=x.shape, dtype=x.dtype, device=x.device)
    for t, nm in ((mean, "mean"), (rstd, "rstd"), (gamma, "gamma")):
        _check(t, nm, shape=(c,), dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    dgamma = torch.empty(c, dtype=torch.float32, device=x.device) if dgamma is None else dgamma
    dbeta = torch.empty(c, dtype=torch.float32, device=x.device) if dbeta is None else dbeta
    _check(dgamma, "dgamma", shape=(c,), dtype=torch.float32, device=x.device)
    _check(dbeta, "dbeta", shape=(c,), dtype=torch.float32, device=x.device)
    if not relu:
        _ctx_for(x).call("nott_batchnorm2d_bwd", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(dy), _ptr(mean),
                         _ptr(rstd), _ptr(gamma), _ptr(dx), _ptr(dgamma), _ptr(dbeta), int(accumulate))
    else:
        if beta is None:
            raise ValueError("relu=True needs beta")
        _check(beta, "beta", shape=(c,), dtype=torch.float32, device=x.device)
        _ctx_for(x).call("nott_batchnorm2d_bwd_act", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(dy), _ptr(mean),
                         _ptr(rstd), _ptr(gamma), _ptr(beta), 1, _ptr(dx), _ptr(dgamma), _ptr(dbeta),
                         int(accumulate))
    return dx, dgamma, dbeta


# ---------------------------------------------------------------------- pools
def pool_out(size: int, k: int, stride: int, pad: int, dil: int, ceil_mode: bool) -> int:
    num = size + 2 * pad - dil * (k - 1) - 1 + (stride - 1 if ceil_mode else 0)
    out = (num // stride) + 1
    if ceil_mode and (out - 1) * stride >= size + pad:
        out -= 1
    return out


def pool_desc(x_shape, kernel, stride=None, padding=(0, 0), dilation=(1, 1), ceil_mode=False) -> Pool2dDesc:
    n, c, h, w = x_shape
    stride = kernel if stride is None else stride
    return Pool2dDesc(n, c, h, w, kernel[0], kernel[1], stride[0], stride[1], padding[0], padding[1],
                      dilation[0], dilation[1], int(ceil_mode), _abi.NOTT_NCHW)


def maxpool2d_fwd(x: torch.Tensor, d: Pool2dDesc):
    _check(x, "x", shape=(d.n, d.c, d.h, d.w))
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    y = torch.empty((d.n, d.c, oh, ow), dtype=x.dtype, device=x.device)
    idx = torch.empty((d.n, d.c, oh, ow), dtype=torch.int64, device=x.device)
    _ctx_for(x).call("nott_maxpool2d_fwd", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(y), _ptr(idx))
    return y, idx


def maxpool2d_bwd(argmax: torch.Tensor, dy: torch.Tensor, d: Pool2dDesc) -> torch.Tensor:
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    _check(dy, "dy", shape=(d.n, d.c, oh, ow))
    _check(argmax, "argmax", shape=(d.n, d.c, oh, ow), dtype=torch.int64, device=dy.device)
    dx = torch.empty((d.n, d.c, d.h, d.w), dtype=dy.dtype, device=dy.device)
    _ctx_for(dy).call("nott_maxpool2d_bwd", C.byref(d), nott_dtype(dy.dtype), _ptr(argmax), _ptr(dy), _ptr(dx))
    return dx


def maxpool2d_fwd_tap(x: torch.Tensor, d: Pool2dDesc):
    """MaxPool2d forward keeping the argmax as the uint8 window tap
    ((ih − oh·sh + ph)/dh)·kw + (iw − ow·sw + pw)/dw (nott_maxpool2d_fwd_tap)."""
    _check(x, "x", shape=(d.n, d.c, d.h, d.w))
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    y = torch.empty((d.n, d.c, oh, ow), dtype=x.dtype, device=x.device)
    tap = torch.empty((d.n, d.c, oh, ow), dtype=torch.uint8, device=x.device)
    _ctx_for(x).call("nott_maxpool2d_fwd_tap", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(y), _ptr(tap))
    return y, tap


def batchnorm2d_relu_maxpool2d_fwd(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, d: Pool2dDesc,
                                   eps: float = 1e-5, momentum: float = 0.1,
                                   running_mean: Optional[torch.Tensor] = None,
                                   running_var: Optional[torch.Tensor] = None):
    """maxpool(relu(BN(x))) without the BatchNorm's output in memory
    (nott_batchnorm2d_fwd_coef, then nott_maxpool2d_fwd_tap_bnrelu):
    returns (y, tap, mean, rstd)."""
    _check(x, "x")
    n, c, h, w = x.shape
    mean = torch.empty(c, dtype=torch.float32, device=x.device)
    rstd = torch.empty(c, dtype=torch.float32, device=x.device)
    coef = torch.empty(2 * c, dtype=torch.float32, device=x.device)
    ctx = _ctx_for(x)
    ctx.call("nott_batchnorm2d_fwd_coef", nott_dtype(x.dtype), n, c, h * w, _ptr(x), _ptr(gamma), _ptr(beta),
             float(eps), float(momentum), _ptr(running_mean), _ptr(running_var), _ptr(mean), _ptr(rstd), _ptr(coef))
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    y = torch.empty((n, c, oh, ow), dtype=x.dtype, device=x.device)
    tap = torch.empty((n, c, oh, ow), dtype=torch.uint8, device=x.device)
    ctx.call("nott_maxpool2d_fwd_tap_bnrelu", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(coef), _ptr(y), _ptr(tap))
    return y, tap, mean, rstd


def batchnorm2d_relu_maxpool2d_bwd(x: torch.Tensor, tap: torch.Tensor, dy: torch.Tensor, d: Pool2dDesc,
                                   mean: torch.Tensor, rstd: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor,
                                   dgamma: Optional[torch.Tensor] = None, dbeta: Optional[torch.Tensor] = None,
                                   accumulate: bool = False, need_dx: bool = True):
    """Backward of batchnorm2d_relu_maxpool2d_fwd: (dx, dgamma, dbeta)
    (nott_batchnorm2d_relu_maxpool2d_bwd; dx None when need_dx is False)."""
    _check(x, "x")
    n, c, h, w = x.shape
    if (d.n, d.c, d.h, d.w) != (n, c, h, w):
        raise ValueError("descriptor does not match x")
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    _check(dy, "dy", shape=(n, c, oh, ow), dtype=x.dtype, device=x.device)
    _check(tap, "tap", shape=(n, c, oh, ow), dtype=torch.uint8, device=x.device)
    for t, nm in ((mean, "mean"), (rstd, "rstd"), (gamma, "gamma"), (beta, "beta")):
        _check(t, nm, shape=(c,), dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x) if need_dx else None
    dgamma = torch.empty(c, dtype=torch.float32, device=x.device) if dgamma is None else dgamma
    dbeta = torch.empty(c, dtype=torch.float32, device=x.device) if dbeta is None else dbeta
    _check(dgamma, "dgamma", shape=(c,), dtype=torch.float32, device=x.device)
    _check(dbeta, "dbeta", shape=(c,), dtype=torch.float32, device=x.device)
    _ctx_for(x).call("nott_batchnorm2d_relu_maxpool2d_bwd", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(tap),
                     _ptr(dy), _ptr(mean), _ptr(rstd), _ptr(gamma), _ptr(beta), _ptr(dx), _ptr(dgamma),
                     _ptr(dbeta), int(accumulate))
    return dx, dgamma, dbeta


def maxpool2d_bwd_tap(tap: torch.Tensor, dy: torch.Tensor, d: Pool2dDesc,
                      relu_y: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dx of the pool; with relu_y (the pool's input, a ReLU output) also the
    ReLU's backward: dx = 0 where relu_y <= 0."""
    oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, bool(d.ceil_mode))
    ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, bool(d.ceil_mode))
    _check(dy, "dy", shape=(d.n, d.c, oh, ow))
    _check(tap, "tap", shape=(d.n, d.c, oh, ow), dtype=torch.uint8, device=dy.device)
    dx = torch.empty((d.n, d.c, d.h, d.w), dtype=dy.dtype, device=dy.device)
    if relu_y is None:
        _ctx_for(dy).call("nott_maxpool2d_bwd_tap", C.byref(d), nott_dtype(dy.dtype), _ptr(tap), _ptr(dy), _ptr(dx))
    else:
        _check(relu_y, "relu_y", shape=(d.n, d.c, d.h, d.w), dtype=dy.dtype, device=dy.device)
        _ctx_for(dy).call("nott_maxpool2d_bwd_tap_relu", C.byref(d), nott_dtype(dy.dtype), _ptr(tap), _ptr(dy),
                          _ptr(relu_y), _ptr(dx))
    return dx


def avgpool_global_fwd(x: torch.Tensor) -> torch.Tensor:
    _check(x, "x")
    n, c, h, w = x.shape
    y = torch.empty((n, c, 1, 1), dtype=x.dtype, device=x.device)
    _ctx_for(x).call("nott_avgpool_global_fwd", nott_dtype(x.dtype), n * c, h * w, _ptr(x), _ptr(y))
    return y


def avgpool_global_bwd(dy: torch.Tensor, hw_shape) -> torch.Tensor:
    _check(dy, "dy")
    n, c = dy.shape[0], dy.shape[1]
    if dy.numel() != n * c:
        raise ValueError("dy must be [n, c, 1, 1] or [n, c]")
    h, w = hw_shape
    dx = torch.empty((n, c, h, w), dtype=dy.dtype, device=dy.device)
    _ctx_for(dy).call("nott_avgpool_global_bwd", nott_dtype(dy.dtype), n * c, h * w, _ptr(dy), _ptr(dx))
    return dx


# ---------------------------------------------------------------------- linear
def linear_fwd(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor] = None, relu: bool = False) -> torch.Tensor:
    _check(x, "x")
    m, kin = x.reshape(-1, x.shape[-1]).shape
    nout = w.shape[0]
    _check(w, "w", shape=(nout, kin), dtype=x.dtype, device=x.device)
    if b is not None:
        _check(b, "b", shape=(nout,), dtype=torch.float32, device=x.device)
    y = torch.empty((*x.shape[:-1], nout), dtype=x.dtype, device=x.device)
    if relu:
        _ctx_for(x).call("nott_linear_fwd_act", nott_dtype(x.dtype), m, kin, nout, _ptr(x), _ptr(w), _ptr(b), 1,
                         _ptr(y))
    else:
        _ctx_for(x).call("nott_linear_fwd", nott_dtype(x.dtype), m, kin, nout, _ptr(x), _ptr(w), _ptr(b), _ptr(y))
    return y


def linear_bwd(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, *, need_dx: bool = True, need_dw: bool = True,
               need_db: bool = True, dx: Optional[torch.Tensor] = None, dw: Optional[torch.Tensor] = None,
               db: Optional[torch.Tensor] = None, accumulate: bool = False, relu_input: bool = False):
    _check(x, "x")
    m, kin = x.reshape(-1, x.shape[-1]).shape
    nout = w.shape[0]
    _check(w, "w", shape=(nout, kin), dtype=x.dtype, device=x.device)
    _check(dy, "dy", shape=(*x.shape[:-1], nout), dtype=x.dtype, device=x.device)
    if need_dx and dx is None:
        dx = torch.empty_like(x)
    if need_dx:
        _check(dx, "dx", shape=tuple(x.shape), dtype=x.dtype, device=x.device)
    else:
        dx = None
    if need_dw and dw is None:
        dw = torch.empty((nout, kin), dtype=torch.float32, device=x.device)
    if need_db and db is None:
        db = torch.empty((nout,), dtype=torch.float32, device=x.device)
    if dw is not None:
        _check(dw, "dw", shape=(nout, kin), dtype=torch.float32, device=x.device)
    if db is not None:
        _check(db, "db", shape=(nout,), dtype=torch.float32, device=x.device)
    _ctx_for(x).call("nott_linear_bwd_act", nott_dtype(x.dtype), m, kin, nout, _ptr(dy), _ptr(x), _ptr(w), _ptr(dx),
                     _ptr(dw if need_dw else None), _ptr(db if need_db else None), int(accumulate), int(relu_input))
    return dx, (dw if need_dw else None), (db if need_db else None)


# ------------------------------------------------------------------------ conv
def conv_out(size: int, k: int, stride: int, pad: int, dil: int) -> int:
    return (size + 2 * pad - dil * (k - 1) - 1) // stride + 1


def conv_desc(x_shape, w_shape, stride=(1, 1), padding=(0, 0), dilation=(1, 1), layout=_abi.NOTT_NCHW) -> Conv2dDesc:
    """x_shape is the logical [n, c, h, w]; w_shape is [k, c, r, s]."""
    n, c, h, w = x_shape
    k, c2, r, s = w_shape
    if c2 != c:
        raise ValueError("weight channels do not match input channels")
    return Conv2dDesc(n, c, h, w, k, r, s, stride[0], stride[1], padding[0], padding[1], dilation[0], dilation[1], 1,
                      layout, 0)


def _conv_shapes(d: Conv2dDesc):
    p = conv_out(d.h, d.r, d.stride_h, d.pad_h, d.dil_h)
    q = conv_out(d.w, d.s, d.stride_w, d.pad_w, d.dil_w)
    if d.layout == _abi.NOTT_NCHW:
        return (d.n, d.c, d.h, d.w), (d.n, d.k, p, q)
    return (d.n, d.h, d.w, d.c), (d.n, p, q, d.k)


def conv2d_fwd(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], d: Conv2dDesc,
               relu: bool = False) -> torch.Tensor:
    """y = conv(x, w) + b, or relu of it with relu=True (fused where the kernel allows)."""
    xs, ys = _conv_shapes(d)
    _check(x, "x", shape=xs)
    _check(w, "w", shape=(d.k, d.c, d.r, d.s), dtype=x.dtype, device=x.device)
    if b is not None:
        _check(b, "b", shape=(d.k,), dtype=torch.float32, device=x.device)
    y = torch.empty(ys, dtype=x.dtype, device=x.device)
    _ctx_for(x).call("nott_conv2d_fwd_act", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(w), _ptr(b), int(relu),
                     _ptr(y))
    return y


def conv2d_bwd_data(dy: torch.Tensor, w: torch.Tensor, d: Conv2dDesc,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    xs, ys = _conv_shapes(d)
    _check(dy, "dy", shape=ys)
    _check(w, "w", shape=(d.k, d.c, d.r, d.s), dtype=dy.dtype, device=dy.device)
    dx = torch.empty(xs, dtype=dy.dtype, device=dy.device) if out is None else out
    _check(dx, "out", shape=xs, dtype=dy.dtype, device=dy.device)
    _ctx_for(dy).call("nott_conv2d_bwd_data", C.byref(d), nott_dtype(dy.dtype), _ptr(dy), _ptr(w), _ptr(dx))
    return dx


def conv2d_bwd_weight(x: torch.Tensor, dy: torch.Tensor, d: Conv2dDesc, *, need_db: bool = False,
                      dw: Optional[torch.Tensor] = None, db: Optional[torch.Tensor] = None,
                      accumulate: bool = False):
    xs, ys = _conv_shapes(d)
    _check(x, "x", shape=xs)
    _check(dy, "dy", shape=ys, dtype=x.dtype, device=x.device)
    dw = torch.empty((d.k, d.c, d.r, d.s), dtype=torch.float32, device=x.device) if dw is None else dw
    _check(dw, "dw", shape=(d.k, d.c, d.r, d.s), dtype=torch.float32, device=x.device)
    if need_db and db is None:
        db = torch.empty((d.k,), dtype=torch.float32, device=x.device)
    if db is not None:
        _check(db, "db", shape=(d.k,), dtype=torch.float32, device=x.device)
    _ctx_for(x).call("nott_conv2d_bwd_weight", C.byref(d), nott_dtype(x.dtype), _ptr(x), _ptr(dy), _ptr(dw), _ptr(db),
                     int(accumulate))
    return dw, db


# ------------------------------------------------------------------- attention
def attn_desc(b: int, h: int, t: int, s: int, dh: int, causal: bool, scale: Optional[float] = None, *,
              token_major: bool = False, ld_qkv: int = 0, ld_o: int = 0) -> AttnDesc:
    """Head-major ([b, h, rows, dh] contiguous) or token-major ([b, rows, h, dh]
    views with row strides ld_qkv for q/k/v and their gradients, ld_o for o/dO;
    0 = h·dh) attention descriptor."""
    layout = _abi.NOTT_ATTN_TOKEN_MAJOR if token_major else _abi.NOTT_ATTN_HEAD_MAJOR
    return AttnDesc(b, h, t, s, dh, int(causal), layout, 1.0 / math.sqrt(dh) if scale is None else float(scale),
                    int(ld_qkv), int(ld_o))


def _attn_ld(d: AttnDesc, which: str) -> int:
    ld = d.ld_qkv if which == "qkv" else d.ld_o
    return ld if ld else d.h * d.dh


def _check_attn(t: torch.Tensor, name: str, d: AttnDesc, rows: int, which: str, ref: Optional[torch.Tensor] = None):
    """Head-major: contiguous [b, h, rows, dh].  Token-major: [b, rows, h, dh]
    with strides (rows·ld, ld, dh, 1)."""
    if d.layout == _abi.NOTT_ATTN_HEAD_MAJOR:
        _check(t, name, shape=(d.b, d.h, rows, d.dh), dtype=None if ref is None else ref.dtype,
               device=None if ref is None else ref.device)
        return
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if tuple(t.shape) != (d.b, rows, d.h, d.dh):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {(d.b, rows, d.h, d.dh)}")
    ld = _attn_ld(d, which)
    want = (rows * ld, ld, d.dh, 1)
    if t.numel() and any(sz > 1 and st != w for sz, st, w in zip(t.shape, t.stride(), want)):
        raise ValueError(f"{name} has strides {t.stride()}, expected {want}")
    if ref is not None and (t.dtype != ref.dtype or t.device != ref.device):
        raise TypeError(f"{name} must match q's dtype and device")


def _attn_empty(d: AttnDesc, rows: int, which: str, like: torch.Tensor) -> torch.Tensor:
    if d.layout == _abi.NOTT_ATTN_HEAD_MAJOR:
        return torch.empty((d.b, d.h, rows, d.dh), dtype=like.dtype, device=like.device)
    if _attn_ld(d, which) != d.h * d.dh:
        raise ValueError("token-major outputs with a row stride other than h·dh must be passed in")
    return torch.empty((d.b, rows, d.h, d.dh), dtype=like.dtype, device=like.device)


def attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, d: AttnDesc, out: Optional[torch.Tensor] = None):
    _check_attn(q, "q", d, d.t, "qkv")
    _check_attn(k, "k", d, d.s, "qkv", q)
    _check_attn(v, "v", d, d.s, "qkv", q)
    o = _attn_empty(d, d.t, "o", q) if out is None else out
    _check_attn(o, "o", d, d.t, "o", q)
    lse = torch.empty((d.b, d.h, d.t), dtype=torch.float32, device=q.device)
    _ctx_for(q).call("nott_attention_fwd", C.byref(d), nott_dtype(q.dtype), _ptr(q), _ptr(k), _ptr(v), _ptr(o),
                     _ptr(lse))
    return o, lse


def attention_bwd(q, k, v, o, dO, lse, d: AttnDesc, out=None):
    """Returns (dq, dk, dv) in the descriptor's layout; `out` = three tensors
    to write them into (required for token-major row strides other than h·dh)."""
    _check_attn(q, "q", d, d.t, "qkv")
    for t, nm, rows, which in ((k, "k", d.s, "qkv"), (v, "v", d.s, "qkv"), (o, "o", d.t, "o"),
                               (dO, "dO", d.t, "o")):
        _check_attn(t, nm, d, rows, which, q)
    _check(lse, "lse", shape=(d.b, d.h, d.t), dtype=torch.float32, device=q.device)
    if out is None:
        dq, dk, dv = _attn_empty(d, d.t, "qkv", q), _attn_empty(d, d.s, "qkv", q), _attn_empty(d, d.s, "qkv", q)
    else:
        dq, dk, dv = out
    for t, nm, rows in ((dq, "dq", d.t), (dk, "dk", d.s), (dv, "dv", d.s)):
        _check_attn(t, nm, d, rows, "qkv", q)
    _ctx_for(q).call("nott_attention_bwd", C.byref(d), nott_dtype(q.dtype), _ptr(q), _ptr(k), _ptr(v), _ptr(o),
                     _ptr(dO), _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv))
    return dq, dk, dv
