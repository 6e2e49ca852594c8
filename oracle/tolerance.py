"""Error model of fp32 evaluations of the normalizations, forward and backward (tests only).

The parity bar for dx is "within one ulp of the output type of the float64 reference" plus, per
element, what an fp32 evaluation of the same formula cannot avoid.  dx cancels:

    LayerNorm:  dx = rstd (g - c1 - xhat c2),   RMSNorm: dx = rstd (g - xhat c2),
    g = dy gamma (GELU epilogue: dy GELU'(a) gamma, a = xhat gamma + beta),
    c1 = mean(g), c2 = mean(g xhat)

(the contract of the reference's declared backward, csrc/layernorm.h:24-32 and
csrc/layernorm_cuda.cpp:97-141), so an element near zero carries the rounding of terms much larger
than itself.  `dx_allowance` bounds that rounding element by element, from the float64 terms:

    rstd * [ (2^-20 + 2^-23 log2 N) (|g| + |c1| + |xhat c2|)          the terms' own roundings
                                                                          (16 fp32 ulps) and the
                                                                          statistics' relative error
             + 2^-21 log2 N (mean|g| + |xhat| mean|g xhat|)            the row sums c1, c2
             + (|c2| + |xhat| mean|g|) e_x                              xhat's centring, e_x =
                                                                          2^-23 log2 N rstd mean|x|
             + (2^-21 + 0.8 max|gamma| e_x)                                     GELU' (tables
                 (|dy gamma| + mean|dy gamma| + |xhat| mean|dy gamma xhat|)     within 2.1e-7;
                                                                          |GELU''| <= 0.8 times
                                                                          a's centring error) ]
    + 2^-23 |dres|                                                     the residual gradient add

Every coefficient is an fp32 rounding count, not a fraction of max|dx|: an evaluation that rounds
g = dy gamma, xhat or dx to bf16 before the last step (relative error 2^-9) exceeds it by two
orders of magnitude.  tests/test_oracle.py checks the model on the CPU against an fp32 evaluation
of the formula (it must cover that) and against planted bf16 roundings of g and xhat (it must
reject them).

The forward output y = xhat gamma + beta cancels too, where xhat gamma and beta nearly cancel,
and there it also carries the rounding of the fp32 row mean, which shifts every xhat of the row:
`y_allowance` is

    2^-21 (|xhat gamma| + |beta|)          the affine step's own roundings (8 fp32 ulps)
    + |gamma| e_x                          LayerNorm: xhat's centring, e_x as above

times 1.13 (the largest |GELU'|) for LN + GELU.  torch's own fp32 layer_norm on the CPU needs
this term as much as the kernels do (bf16 h = x + r, 416 columns: an element at -4.6e-9 comes
out 9.6e-9 off from torch, 6.1e-9 from the kernel); tests/test_oracle.py checks that fp32
evaluations stay within it and that a mean rounded to bf16 does not.
"""
from __future__ import annotations

import json
import os

import numpy as np

_ULP_BITS = {"bf16": (7, -126), "f16": (10, -14), "f32": (23, -126)}


def ulp(ref, kind: str = "bf16") -> np.ndarray:
    """Spacing of `kind` numbers at |ref| (bf16 8, f16 11, f32 24 significant bits)."""
    mant, emin = _ULP_BITS[kind]
    a = np.abs(np.asarray(ref, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** emin)))
    return np.exp2(e - mant)


def _f64(a):
    return None if a is None else np.asarray(a, np.float64)


def dx_allowance(x, dy, gamma=None, eps=1e-5, rms=False, beta=None, approximate=None,
                 dres=None, chunk=2048) -> np.ndarray:
    """Elementwise fp32 evaluation allowance of dx (module docstring), float64, x's shape.
    `approximate` ("none" / "tanh") selects the GELU epilogue; rows are processed in chunks."""
    from . import norms
    x = np.asarray(x)
    dy = np.asarray(dy)
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    dy2 = dy.reshape(-1, n)
    out = np.empty(x2.shape, np.float64)
    g64 = np.ones(n) if gamma is None else _f64(gamma).reshape(n)
    b64 = None if beta is None else _f64(beta).reshape(n)
    lg = np.log2(max(n, 2))
    for r0 in range(0, x2.shape[0], chunk):
        xs = x2[r0:r0 + chunk].astype(np.float64)
        ds = dy2[r0:r0 + chunk].astype(np.float64)
        if rms:
            mu = np.zeros((xs.shape[0], 1))
            rstd = 1.0 / np.sqrt((xs * xs).mean(axis=1, keepdims=True) + eps)
        else:
            mu = xs.mean(axis=1, keepdims=True)
            rstd = 1.0 / np.sqrt(((xs - mu) ** 2).mean(axis=1, keepdims=True) + eps)
        xh = (xs - mu) * rstd
        dg = ds * g64
        if approximate is not None:
            a = xh * g64 + (0.0 if b64 is None else b64)
            g = dg * norms.gelu_grad(a, approximate)
        else:
            g = dg
        c1 = np.zeros_like(mu) if rms else g.mean(axis=1, keepdims=True)
        c2 = (g * xh).mean(axis=1, keepdims=True)
        terms = np.abs(g) + np.abs(c1) + np.abs(xh * c2)
        sums = np.abs(g).mean(axis=1, keepdims=True) + \
            np.abs(xh) * np.abs(g * xh).mean(axis=1, keepdims=True)
        e_x = 0.0 if rms else 2.0 ** -23 * lg * rstd * np.abs(xs).mean(axis=1, keepdims=True)
        a_ = (2.0 ** -20 + 2.0 ** -23 * lg) * terms + 2.0 ** -21 * lg * sums + \
            (np.abs(c2) + np.abs(xh) * np.abs(g).mean(axis=1, keepdims=True)) * e_x
        if approximate is not None:
            # GELU'(a) off by the tables' error and by GELU'' (at most 0.8) times the centring
            # error of a = xhat gamma + beta.
            dgp = 2.0 ** -21 + 0.8 * np.abs(g64).max() * e_x
            a_ = a_ + dgp * (np.abs(dg) + np.abs(dg).mean(axis=1, keepdims=True) +
                             np.abs(xh) * np.abs(dg * xh).mean(axis=1, keepdims=True))
        out[r0:r0 + chunk] = rstd * a_
    out = out.reshape(x.shape)
    if dres is not None:
        out = out + 2.0 ** -23 * np.abs(_f64(dres))
    return out


def y_allowance(x, gamma=None, beta=None, eps=1e-5, rms=False, approximate=None,
                chunk=2048) -> np.ndarray:
    """Elementwise fp32 evaluation allowance of the forward output y (module docstring), float64,
    x's shape: 2^-21 (|xhat gamma| + |beta|) + |gamma| e_x (LayerNorm), times 1.13 with a GELU
    epilogue (`approximate` "none" / "tanh")."""
    x = np.asarray(x)
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    out = np.empty(x2.shape, np.float64)
    g64 = np.ones(n) if gamma is None else _f64(gamma).reshape(n)
    b64 = np.zeros(n) if beta is None else _f64(beta).reshape(n)
    lg = np.log2(max(n, 2))
    for r0 in range(0, x2.shape[0], chunk):
        xs = x2[r0:r0 + chunk].astype(np.float64)
        if rms:
            rstd = 1.0 / np.sqrt((xs * xs).mean(axis=1, keepdims=True) + eps)
            xh = xs * rstd
            e_x = 0.0
        else:
            mu = xs.mean(axis=1, keepdims=True)
            rstd = 1.0 / np.sqrt(((xs - mu) ** 2).mean(axis=1, keepdims=True) + eps)
            xh = (xs - mu) * rstd
            e_x = 2.0 ** -23 * lg * rstd * np.abs(xs).mean(axis=1, keepdims=True)
        al = 2.0 ** -21 * (np.abs(xh * g64) + np.abs(b64)) + np.abs(g64) * e_x
        out[r0:r0 + chunk] = al * (1.13 if approximate is not None else 1.0)
    return out.reshape(x.shape)


def within_stats(got, ref, allowance, kind: str) -> dict:
    """How much of the bar |got - ref| <= ulp_kind(ref) + allowance is used: the worst error in
    ulps over the elements whose allowance is below a quarter ulp (no cancellation), the worst
    fraction of the whole bound, and the share of elements where the allowance is a quarter ulp
    or more."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    u = ulp(r, kind)
    err = np.abs(g - r)
    al = np.broadcast_to(np.asarray(allowance, np.float64), err.shape)
    clean = al < 0.25 * u
    return {"kind": kind, "n": int(err.size),
            "worst_ulps_clean": float((err[clean] / u[clean]).max()) if clean.any() else 0.0,
            "worst_bound_frac": float((err / (u + al)).max()) if err.size else 0.0,
            "cancelling_share": float(1.0 - clean.mean()) if err.size else 0.0}


def report(what: str, stats: dict) -> None:
    """Append one JSON line to the file named by FLN_PARITY_REPORT (if set)."""
    path = os.environ.get("FLN_PARITY_REPORT")
    if path:
        with open(path, "a") as fh:
            fh.write(json.dumps({"what": what, **stats}) + "\n")
