"""Helpers for the GPU parity tests (HIP path vs the CPU oracle)."""
from __future__ import annotations

import numpy as np
import torch

from oracle_lib import round_bf16

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def dev(a: np.ndarray, dt: str = "f32") -> torch.Tensor:
    """Host fp32 array -> device tensor of the test dtype (bf16: RNE rounding)."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda")
    return t.to(TORCH_DT[dt]).contiguous()


def host_input(a: np.ndarray, dt: str) -> np.ndarray:
    """What the oracle must see for an input fed to the GPU in dtype `dt`."""
    return round_bf16(a) if dt == "bf16" else np.ascontiguousarray(a, np.float32)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def check(got, want, dt: str = "f32", what: str = "", rtol=None, atol=None):
    """Elementwise |got − want| <= atol + rtol·|want|.

    fp32: rtol 1e-4, atol 1e-5·max(1, rms(want)) — the absolute floor scales
    with the output's magnitude so long fp32 reductions are judged relative
    to what they sum.  bf16: rtol 2e-2, atol 2e-2·rms(want) — "rel 2e-2"
    measured against the tensor's scale, since an element near zero that is
    a sum of bf16-rounded products cannot meet 2e-2 of its own size.
    NaN positions must agree."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN positions differ"
    g, w = got[~nan_w], want[~nan_w]
    if g.size == 0:
        return
    rms = float(np.sqrt(np.mean(w[np.isfinite(w)] ** 2))) if np.isfinite(w).any() else 1.0
    if dt == "bf16":
        rtol = 2e-2 if rtol is None else rtol
        atol = 2e-2 * rms if atol is None else atol
    else:
        rtol = 1e-4 if rtol is None else rtol
        atol = 1e-5 * max(1.0, rms) if atol is None else atol
    inf = ~np.isfinite(w)
    assert np.array_equal(g[inf], w[inf]), f"{what}: infinities differ"
    err = np.abs(g[~inf] - w[~inf]) - (atol + rtol * np.abs(w[~inf]))
    if err.size and err.max() > 0:
        i = int(np.argmax(err))
        raise AssertionError(f"{what}: {int((err > 0).sum())}/{err.size} out of tolerance; worst got "
                             f"{g[~inf][i]:.6g} want {w[~inf][i]:.6g} (rtol {rtol}, atol {atol:.3g})")
