"""Tolerance helpers shared by the parity tests (tolerances are stated where they are used)."""
from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy()


def bf16_ulp(ref: np.ndarray) -> np.ndarray:
    """Spacing of bfloat16 numbers at |ref| (8 significant bits)."""
    a = np.abs(np.asarray(ref, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def f16_ulp(ref: np.ndarray) -> np.ndarray:
    a = np.abs(np.asarray(ref, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 10)


def assert_within_ulp(got, ref, ulps: float = 1.0, atol: float = 0.0, kind: str = "bf16",
                      what: str = ""):
    """|got - ref| <= ulps * ulp_kind(ref) + atol, elementwise."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    ulp = bf16_ulp(r) if kind == "bf16" else f16_ulp(r)
    err = np.abs(g - r)
    bound = ulps * ulp + atol
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements exceed {ulps} {kind} ulp + {atol:g}; "
            f"worst at {i}: got {g[i]!r} ref {r[i]!r} err {err[i]:.3g} bound {bound[i]:.3g}")


def assert_close_rel(got, ref, rtol: float, what: str = ""):
    """Max-norm relative check: max|got - ref| <= rtol * max|ref| (for column sums)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    err = np.abs(g - r).max() if g.size else 0.0
    scale = np.abs(r).max() if r.size else 0.0
    assert err <= rtol * max(scale, 1e-30), f"{what}: max err {err:.3g} > {rtol:g} * {scale:.3g}"
