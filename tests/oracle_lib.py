"""numpy wrappers over the CPU checkers (test infrastructure).

* `Oracle`  — oracle/liboracle.so, the plain-C restatement (always built).
* `Ref`     — oracle/_ref/libnott_ref.so, the reference's own modules compiled
              from its sources (present only where the reference was available
              at build time; tests that need it skip otherwise).

Inputs come from `rng(seed)` (numpy Philox), so the GPU path, the oracle and
the reference see identical buffers.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from thot_amd._abi import AttnDesc, Conv2dDesc, Pool2dDesc

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(REPO, "oracle", "liboracle.so")
REF_SO = os.path.join(REPO, "oracle", "_ref", "libnott_ref.so")

P = C.c_void_p
i64 = C.c_int64
f64 = C.c_double


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(seed))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(P)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (RNE), returned as fp32."""
    a = f32(a).copy()
    u = a.view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32)


def conv_out(size, k, stride, pad, dil):
    return (size + 2 * pad - dil * (k - 1) - 1) // stride + 1


def pool_out(size, k, stride, pad, dil, ceil_mode):
    num = size + 2 * pad - dil * (k - 1) - 1 + (stride - 1 if ceil_mode else 0)
    out = num // stride + 1
    if ceil_mode and (out - 1) * stride >= size + pad:
        out -= 1
    return out


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing; run `make -C oracle`")
        self.lib = C.CDLL(path)
        self.lib.oracle_conv_out.restype = i64
        self.lib.oracle_pool_out.restype = i64
        for name in ("oracle_conv_out", "oracle_pool_out"):
            getattr(self.lib, name).argtypes = None

    # conv -------------------------------------------------------------------
    def conv2d_fwd(self, d: Conv2dDesc, x, w, b=None):
        p_, q_ = conv_out(d.h, d.r, d.stride_h, d.pad_h, d.dil_h), conv_out(d.w, d.s, d.stride_w, d.pad_w, d.dil_w)
        y = np.empty((d.n, d.k, p_, q_), np.float32)
        self.lib.oracle_conv2d_fwd(C.byref(d), _p(f32(x)), _p(f32(w)), _p(None if b is None else f32(b)), _p(y))
        return y

    def conv2d_bwd_data(self, d: Conv2dDesc, dy, w):
        dx = np.empty((d.n, d.c, d.h, d.w), np.float32)
        self.lib.oracle_conv2d_bwd_data(C.byref(d), _p(f32(dy)), _p(f32(w)), _p(dx))
        return dx

    def conv2d_bwd_weight(self, d: Conv2dDesc, x, dy, with_db=True):
        dw = np.empty((d.k, d.c, d.r, d.s), np.float32)
        db = np.empty((d.k,), np.float32) if with_db else None
        self.lib.oracle_conv2d_bwd_weight(C.byref(d), _p(f32(x)), _p(f32(dy)), _p(dw), _p(db))
        return dw, db

    # linear -----------------------------------------------------------------
    def linear_fwd(self, x, w, b=None):
        m, kin = x.shape
        nout = w.shape[0]
        y = np.empty((m, nout), np.float32)
        self.lib.oracle_linear_fwd(i64(m), i64(kin), i64(nout), _p(f32(x)), _p(f32(w)),
                                   _p(None if b is None else f32(b)), _p(y))
        return y

    def linear_bwd(self, dy, x, w):
        m, kin = x.shape
        nout = w.shape[0]
        dx = np.empty((m, kin), np.float32)
        dw = np.empty((nout, kin), np.float32)
        db = np.empty((nout,), np.float32)
        self.lib.oracle_linear_bwd(i64(m), i64(kin), i64(nout), _p(f32(dy)), _p(f32(x)), _p(f32(w)), _p(dx), _p(dw),
                                   _p(db))
        return dx, dw, db

    # elementwise ------------------------------------------------------------
    def relu_fwd(self, x):
        x = f32(x)
        y = np.empty_like(x)
        self.lib.oracle_relu_fwd(i64(x.size), _p(x), _p(y))
        return y

    def relu_bwd(self, y, dy):
        y, dy = f32(y), f32(dy)
        dx = np.empty_like(dy)
        self.lib.oracle_relu_bwd(i64(y.size), _p(y), _p(dy), _p(dx))
        return dx

    # pools ------------------------------------------------------------------
    def maxpool2d_fwd(self, d: Pool2dDesc, x):
        oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, d.ceil_mode)
        ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, d.ceil_mode)
        y = np.empty((d.n, d.c, oh, ow), np.float32)
        idx = np.empty((d.n, d.c, oh, ow), np.int64)
        self.lib.oracle_maxpool2d_fwd(C.byref(d), _p(f32(x)), _p(y), _p(idx))
        return y, idx

    def maxpool2d_bwd(self, d: Pool2dDesc, argmax, dy):
        dx = np.empty((d.n, d.c, d.h, d.w), np.float32)
        self.lib.oracle_maxpool2d_bwd(C.byref(d), _p(np.ascontiguousarray(argmax, np.int64)), _p(f32(dy)), _p(dx))
        return dx

    def avgpool_global_fwd(self, x):
        n, c, h, w = x.shape
        y = np.empty((n, c, 1, 1), np.float32)
        self.lib.oracle_avgpool_global_fwd(i64(n * c), i64(h * w), _p(f32(x)), _p(y))
        return y

    def avgpool_global_bwd(self, dy, hw):
        n, c = dy.shape[:2]
        dx = np.empty((n, c, hw[0], hw[1]), np.float32)
        self.lib.oracle_avgpool_global_bwd(i64(n * c), i64(hw[0] * hw[1]), _p(f32(dy)), _p(dx))
        return dx

    # norms ------------------------------------------------------------------
    def batchnorm2d_fwd(self, x, gamma, beta, eps=1e-5, momentum=0.1, running_mean=None, running_var=None):
        n, c, h, w = x.shape
        y = np.empty_like(f32(x))
        mean = np.empty((c,), np.float32)
        rstd = np.empty((c,), np.float32)
        rm = None if running_mean is None else f32(running_mean).copy()
        rv = None if running_var is None else f32(running_var).copy()
        self.lib.oracle_batchnorm2d_fwd(i64(n), i64(c), i64(h * w), _p(f32(x)), _p(f32(gamma)), _p(f32(beta)),
                                        f64(eps), f64(momentum), _p(rm), _p(rv), _p(y), _p(mean), _p(rstd))
        return y, mean, rstd, rm, rv

    def batchnorm2d_bwd(self, x, dy, mean, rstd, gamma):
        n, c, h, w = x.shape
        dx = np.empty_like(f32(x))
        dg = np.empty((c,), np.float32)
        db = np.empty((c,), np.float32)
        self.lib.oracle_batchnorm2d_bwd(i64(n), i64(c), i64(h * w), _p(f32(x)), _p(f32(dy)), _p(f32(mean)),
                                        _p(f32(rstd)), _p(f32(gamma)), _p(dx), _p(dg), _p(db))
        return dx, dg, db

    def layernorm_fwd(self, x, gamma, beta, eps=1e-5):
        rows, d = x.shape
        y = np.empty_like(f32(x))
        mean = np.empty((rows,), np.float32)
        rstd = np.empty((rows,), np.float32)
        self.lib.oracle_layernorm_fwd(i64(rows), i64(d), _p(f32(x)), _p(f32(gamma)), _p(f32(beta)), f64(eps), _p(y),
                                      _p(mean), _p(rstd))
        return y, mean, rstd

    def layernorm_bwd(self, x, dy, mean, rstd, gamma):
        rows, d = x.shape
        dx = np.empty_like(f32(x))
        dg = np.empty((d,), np.float32)
        db = np.empty((d,), np.float32)
        self.lib.oracle_layernorm_bwd(i64(rows), i64(d), _p(f32(x)), _p(f32(dy)), _p(f32(mean)), _p(f32(rstd)),
                                      _p(f32(gamma)), _p(dx), _p(dg), _p(db))
        return dx, dg, db

    # loss -------------------------------------------------------------------
    def softmax_xent(self, logits, labels, label_smoothing=0.0, grad_scale=1.0):
        n, c = logits.shape
        dl = np.empty((n, c), np.float32)
        loss = np.empty((1,), np.float32)
        self.lib.oracle_softmax_xent(i64(n), i64(c), _p(f32(logits)), _p(np.ascontiguousarray(labels, np.int64)),
                                     f64(label_smoothing), f64(grad_scale), _p(dl), _p(loss))
        return dl, float(loss[0])

    # attention --------------------------------------------------------------
    def attention_fwd(self, d: AttnDesc, q, k, v):
        o = np.empty((d.b, d.h, d.t, d.dh), np.float32)
        lse = np.empty((d.b, d.h, d.t), np.float32)
        self.lib.oracle_attention_fwd(C.byref(d), _p(f32(q)), _p(f32(k)), _p(f32(v)), _p(o), _p(lse))
        return o, lse

    def attention_bwd(self, d: AttnDesc, q, k, v, o, dO):
        dq = np.empty((d.b, d.h, d.t, d.dh), np.float32)
        dk = np.empty((d.b, d.h, d.s, d.dh), np.float32)
        dv = np.empty((d.b, d.h, d.s, d.dh), np.float32)
        self.lib.oracle_attention_bwd(C.byref(d), _p(f32(q)), _p(f32(k)), _p(f32(v)), _p(f32(o)), _p(f32(dO)), _p(dq),
                                      _p(dk), _p(dv))
        return dq, dk, dv

    # adam -------------------------------------------------------------------
    def round_bf16(self, x):
        """oracle_round_bf16: fp32 -> nearest bf16 (RNE) -> fp32, elementwise."""
        x = f32(x).copy()
        self.lib.oracle_round_bf16(i64(x.size), _p(x))
        return x

    def adam_step(self, decoupled, p, g, m, v, lr, beta1, beta2, eps, weight_decay, step):
        p, m, v = f32(p).copy(), f32(m).copy(), f32(v).copy()
        self.lib.oracle_adam_step(C.c_int(int(decoupled)), i64(p.size), _p(p), _p(f32(g)), _p(m), _p(v), f64(lr),
                                  f64(beta1), f64(beta2), f64(eps), f64(weight_decay), i64(step))
        return p, m, v


class Ref:
    """The reference's own modules (oracle/_ref).  Raises if not built."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError("reference call failed")

    def set_threads(self, n: int):
        self.lib.ref_set_threads(C.c_int(n))

    def get_threads(self) -> int:
        return self.lib.ref_get_threads()

    def conv2d(self, d: Conv2dDesc, x, w, b, dy):
        p_, q_ = conv_out(d.h, d.r, d.stride_h, d.pad_h, d.dil_h), conv_out(d.w, d.s, d.stride_w, d.pad_w, d.dil_w)
        y = np.empty((d.n, d.k, p_, q_), np.float32)
        dx = np.empty((d.n, d.c, d.h, d.w), np.float32)
        dw = np.empty((d.k, d.c, d.r, d.s), np.float32)
        db = np.empty((d.k,), np.float32)
        self._ok(self.lib.ref_conv2d(C.byref(d), C.c_int(b is not None), _p(f32(x)), _p(f32(w)),
                                     _p(None if b is None else f32(b)), _p(f32(dy)), _p(y), _p(dx), _p(dw), _p(db)))
        return y, dx, dw, (db if b is not None else None)

    def conv2d_bwd_time(self, d: Conv2dDesc, x, w, dy, iters: int) -> float:
        sec = C.c_double()
        self._ok(self.lib.ref_conv2d_bwd_time(C.byref(d), _p(f32(x)), _p(f32(w)), _p(f32(dy)), C.c_int(iters),
                                              C.byref(sec)))
        return sec.value

    def linear(self, x, w, b, dy):
        m, kin = x.shape
        nout = w.shape[0]
        y = np.empty((m, nout), np.float32)
        dx = np.empty((m, kin), np.float32)
        dw = np.empty((nout, kin), np.float32)
        db = np.empty((nout,), np.float32)
        self._ok(self.lib.ref_linear(i64(m), i64(kin), i64(nout), C.c_int(b is not None), _p(f32(x)), _p(f32(w)),
                                     _p(None if b is None else f32(b)), _p(f32(dy)), _p(y), _p(dx), _p(dw), _p(db)))
        return y, dx, dw, (db if b is not None else None)

    def relu(self, x, dy):
        x, dy = f32(x), f32(dy)
        y, dx = np.empty_like(x), np.empty_like(x)
        self._ok(self.lib.ref_relu(i64(x.size), _p(x), _p(dy), _p(y), _p(dx)))
        return y, dx

    def maxpool2d(self, d: Pool2dDesc, x, dy):
        oh = pool_out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, d.ceil_mode)
        ow = pool_out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, d.ceil_mode)
        y = np.empty((d.n, d.c, oh, ow), np.float32)
        idx = np.empty((d.n, d.c, oh, ow), np.int64)
        dx = np.empty((d.n, d.c, d.h, d.w), np.float32)
        self._ok(self.lib.ref_maxpool2d(C.byref(d), _p(f32(x)), _p(f32(dy)), _p(y), _p(idx), _p(dx)))
        return y, idx, dx

    def avgpool_global(self, x, dy):
        n, c, h, w = x.shape
        y = np.empty((n, c, 1, 1), np.float32)
        dx = np.empty((n, c, h, w), np.float32)
        self._ok(self.lib.ref_avgpool_global(i64(n), i64(c), i64(h), i64(w), _p(f32(x)), _p(f32(dy)), _p(y), _p(dx)))
        return y, dx

    def batchnorm2d(self, x, gamma, beta, dy, eps=1e-5, momentum=0.1, running_mean=None, running_var=None):
        n, c, h, w = x.shape
        y, dx = np.empty_like(f32(x)), np.empty_like(f32(x))
        dg, db = np.empty((c,), np.float32), np.empty((c,), np.float32)
        rm = None if running_mean is None else f32(running_mean).copy()
        rv = None if running_var is None else f32(running_var).copy()
        self._ok(self.lib.ref_batchnorm2d(i64(n), i64(c), i64(h), i64(w), f64(eps), f64(momentum), _p(f32(x)),
                                          _p(f32(gamma)), _p(f32(beta)), _p(f32(dy)), _p(rm), _p(rv), _p(y), _p(dx),
                                          _p(dg), _p(db)))
        return y, dx, dg, db, rm, rv

    def layernorm(self, x, gamma, beta, dy, eps=1e-5):
        rows, d = x.shape
        y, dx = np.empty_like(f32(x)), np.empty_like(f32(x))
        dg, db = np.empty((d,), np.float32), np.empty((d,), np.float32)
        self._ok(self.lib.ref_layernorm(i64(rows), i64(d), f64(eps), _p(f32(x)), _p(f32(gamma)), _p(f32(beta)),
                                        _p(f32(dy)), _p(y), _p(dx), _p(dg), _p(db)))
        return y, dx, dg, db

    def cross_entropy(self, logits, labels, label_smoothing=0.0):
        n, c = logits.shape
        loss = C.c_float()
        dl = np.empty((n, c), np.float32)
        self._ok(self.lib.ref_cross_entropy(i64(n), i64(c), f64(label_smoothing), _p(f32(logits)),
                                            _p(np.ascontiguousarray(labels, np.int64)), C.byref(loss), _p(dl)))
        return dl, loss.value

    def adam_step(self, decoupled, p, g, m, v, lr, beta1, beta2, eps, weight_decay, step):
        p, m, v = f32(p).copy(), f32(m).copy(), f32(v).copy()
        self._ok(self.lib.ref_adam_step(C.c_int(int(decoupled)), i64(p.size), _p(p), _p(f32(g)), _p(m), _p(v),
                                        f64(lr), f64(beta1), f64(beta2), f64(eps), f64(weight_decay), i64(step)))
        return p, m, v

    def adamw_time(self, n: int, iters: int) -> float:
        sec = C.c_double()
        self._ok(self.lib.ref_adamw_time(i64(n), C.c_int(iters), C.byref(sec)))
        return sec.value

    def layernorm_bwd_time(self, rows: int, d: int, iters: int) -> float:
        sec = C.c_double()
        self._ok(self.lib.ref_layernorm_bwd_time(i64(rows), i64(d), C.c_int(iters), C.byref(sec)))
        return sec.value

    def cross_entropy_time(self, n: int, c: int, iters: int) -> float:
        sec = C.c_double()
        self._ok(self.lib.ref_cross_entropy_time(i64(n), i64(c), C.c_int(iters), C.byref(sec)))
        return sec.value

    def mha_bwd_time(self, b: int, t: int, e: int, heads: int, causal: bool, iters: int) -> float:
        sec = C.c_double()
        self._ok(self.lib.ref_mha_bwd_time(i64(b), i64(t), i64(e), i64(heads), C.c_int(int(causal)), C.c_int(iters),
                                           C.byref(sec)))
        return sec.value

    def small_cnn_forward_archive(self, path: str, x):
        """configs[0] logits of the reference-built model after loading the
        parameters.binary archive at `path`."""
        x = f32(x)
        logits = np.empty((x.shape[0], 10), np.float32)
        self._ok(self.lib.ref_small_cnn_forward_archive(C.c_char_p(path.encode()), i64(x.shape[0]), _p(x), _p(logits)))
        return logits

    def resnet18_step(self, x, labels, values: dict, lr: float, weight_decay: float, want_blocks: bool = False,
                      precision: str = "f32"):
        """One configs[4] step of the reference's ResNet-18 on the CPU
        (forward, CE mean, backward, AdamW).  `values` maps registration keys
        (parameters and float buffers) to their initial arrays.  Returns
        (loss, logits, grads, after, blocks): grads of the parameters, every
        tensor after the step, and the 9 stem/block outputs when asked.
        precision "f64": the same step in double precision (results as fp32);
        "bf16_storage": fp32 arithmetic with every activation and activation
        gradient rounded to bf16 where the mixed-precision path stores them."""
        x = f32(x)
        batch = x.shape[0]
        names = sorted(values)
        init = [f32(values[k]) for k in names]
        is_param = [not (k.endswith("running_mean") or k.endswith("running_var")) for k in names]
        grads = [np.empty_like(a) if ip else None for a, ip in zip(init, is_param)]
        after = [np.empty_like(a) for a in init]
        arr = lambda items: (C.c_void_p * len(items))(*[None if a is None else a.ctypes.data for a in items])
        cname = (C.c_char_p * len(names))(*[k.encode() for k in names])
        sizes = [(64, 56), (64, 56), (64, 56), (128, 28), (128, 28), (256, 14), (256, 14), (512, 7), (512, 7)]
        blocks = [np.empty((batch, c, h, h), np.float32) for c, h in sizes] if want_blocks else None
        loss = C.c_float()
        logits = np.empty((batch, 1000), np.float32)
        self._ok(self.lib.ref_resnet18_step(i64(batch), _p(x), _p(np.ascontiguousarray(labels, np.int64)), f64(lr),
                                            f64(weight_decay), i64(len(names)), cname, arr(init), arr(grads),
                                            arr(after), C.byref(loss), _p(logits),
                                            arr(blocks) if want_blocks else None,
                                            C.c_int({"f32": 0, "f64": 1, "bf16_storage": 2}[precision])))
        return (loss.value, logits, {k: g for k, g in zip(names, grads) if g is not None},
                dict(zip(names, after)), blocks)

    def resnet18_forward_archive(self, path: str, x):
        """configs[4] training-mode logits of the reference's ResNet-18 after
        loading the parameters.binary archive at `path`."""
        x = f32(x)
        logits = np.empty((x.shape[0], 1000), np.float32)
        self._ok(self.lib.ref_resnet18_forward_archive(C.c_char_p(path.encode()), i64(x.shape[0]), _p(x),
                                                       _p(logits)))
        return logits

    def save_archive(self, model: str, seed: int, batch: int, path: str):
        """parameters.binary of the reference's "small_cnn" or
        "resnet18" model, seeded weights and BatchNorm statistics
        after one training-mode forward at `batch`."""
        which = {"small_cnn": 0, "resnet18": 1}[model]
        self._ok(self.lib.ref_save_archive(C.c_int(which), C.c_uint64(seed), i64(batch), C.c_char_p(path.encode())))

    def init_params(self, model: str, seed: int, shapes: dict) -> dict:
        """Initial parameters of the reference's "small_cnn" or "resnet18"
        model built right after torch's CPU generator was seeded with `seed`;
        `shapes` maps the registration keys wanted to their shapes."""
        names = sorted(shapes)
        outs = [np.empty(shapes[k], np.float32) for k in names]
        cname = (C.c_char_p * len(names))(*[k.encode() for k in names])
        ptrs = (C.c_void_p * len(outs))(*[a.ctypes.data for a in outs])
        which = {"small_cnn": 0, "resnet18": 1}[model]
        self._ok(self.lib.ref_init_params(C.c_int(which), C.c_uint64(seed), i64(len(names)), cname, ptrs))
        return dict(zip(names, outs))

    def train_step_time(self, model: str, batch: int, iters: int) -> float:
        """Seconds per fp32 CPU training step of "small_cnn" or
        "resnet18" built from the reference's layer descriptors."""
        sec = C.c_double()
        which = {"small_cnn": 0, "resnet18": 1}[model]
        self._ok(self.lib.ref_train_step_time(C.c_int(which), i64(batch), C.c_int(iters), C.byref(sec)))
        return sec.value

    def attention(self, d: AttnDesc, q, k, v, dO):
        o = np.empty((d.b, d.h, d.t, d.dh), np.float32)
        dq = np.empty((d.b, d.h, d.t, d.dh), np.float32)
        dk = np.empty((d.b, d.h, d.s, d.dh), np.float32)
        dv = np.empty((d.b, d.h, d.s, d.dh), np.float32)
        self._ok(self.lib.ref_attention(C.byref(d), _p(f32(q)), _p(f32(k)), _p(f32(v)), _p(f32(dO)), _p(o), _p(dq),
                                        _p(dk), _p(dv)))
        return o, dq, dk, dv

    def mha(self, x, wq, wk, wv, wo, bq, bk, bv, bo, dy, heads, causal):
        b, t, e = x.shape
        with_bias = bq is not None
        outs = {k: np.empty(s, np.float32) for k, s in (("y", (b, t, e)), ("dx", (b, t, e)), ("dwq", (e, e)),
                                                        ("dwk", (e, e)), ("dwv", (e, e)), ("dwo", (e, e)),
                                                        ("dbq", (e,)), ("dbk", (e,)), ("dbv", (e,)), ("dbo", (e,)))}
        bz = [None if a is None else f32(a) for a in (bq, bk, bv, bo)]
        self._ok(self.lib.ref_mha(i64(b), i64(t), i64(e), i64(heads), C.c_int(int(causal)), C.c_int(int(with_bias)),
                                  _p(f32(x)), _p(f32(wq)), _p(f32(wk)), _p(f32(wv)), _p(f32(wo)), *[_p(a) for a in bz],
                                  _p(f32(dy)), *[_p(outs[k]) for k in ("y", "dx", "dwq", "dwk", "dwv", "dwo", "dbq",
                                                                       "dbk", "dbv", "dbo")]))
        return outs
