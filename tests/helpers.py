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
    """|got - ref| <= ulps * ulp_kind(ref) + atol, elementwise.  For the 1-ulp bar the share of
    the bound used is appended to $FLN_PARITY_REPORT when that is set."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    ulp = bf16_ulp(r) if kind == "bf16" else f16_ulp(r)
    err = np.abs(g - r)
    bound = ulps * ulp + atol
    bad = err > bound
    if ulps == 1.0:
        from oracle import tolerance
        tolerance.report(what, tolerance.within_stats(g, r, atol, kind))
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        extra = f"{atol:g}" if np.ndim(atol) == 0 else "elementwise atol"
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements exceed {ulps} {kind} ulp + {extra}; "
            f"worst at {i}: got {g[i]!r} ref {r[i]!r} err {err[i]:.3g} bound {bound[i]:.3g}")


def assert_dx(got, ref, allowance, kind: str = "bf16", what: str = "dx"):
    """dx bar: |got - ref| <= 1 ulp_kind(ref) + allowance elementwise, where allowance is the
    fp32 evaluation allowance of oracle.tolerance.dx_allowance (a few fp32 roundings of the
    terms that cancel in dx, not a fraction of max|dx|).  kind: "bf16", "f16" or "f32".  The
    share of the bound used is appended to $FLN_PARITY_REPORT when that is set."""
    from oracle import tolerance
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    u = tolerance.ulp(r, kind)
    err = np.abs(g - r)
    bound = u + allowance
    bad = err > bound
    tolerance.report(what, tolerance.within_stats(g, r, allowance, kind))
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        al = np.broadcast_to(allowance, err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements exceed 1 {kind} ulp + the fp32 "
            f"allowance; worst at {i}: got {g[i]!r} ref {r[i]!r} err {err[i]:.3g} ulp "
            f"{u[i]:.3g} allowance {al[i]:.3g}")


def assert_close_rel(got, ref, rtol: float, what: str = ""):
    """Max-norm relative check: max|got - ref| <= rtol * max|ref| (for column sums)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    err = np.abs(g - r).max() if g.size else 0.0
    scale = np.abs(r).max() if r.size else 0.0
    assert err <= rtol * max(scale, 1e-30), f"{what}: max err {err:.3g} > {rtol:g} * {scale:.3g}"


def fp8_ordinal(codes):
    """Signed position of an e4m3fn code on the number line (+0 and -0 both map to 0), so that
    adjacent representable values differ by exactly 1."""
    c = np.asarray(codes).astype(np.int32)
    mag = c & 0x7F
    return np.where(c & 0x80, -mag, mag)


def fp8_ambiguous(t, rel=2.0 ** -20):
    """Elements whose exact (float64) scaled value t lies within `rel` (relative) of an e4m3fn
    rounding midpoint: an fp32 computation of t (a few ulps of noise) may round them either
    way.  Exact ties are common when the row scale cancels a normalization factor (RMSNorm of
    low-precision inputs: t = 448 (h w) / max|h w|)."""
    from oracle import norms
    t = np.asarray(t, np.float64)
    return norms.fp8_e4m3fn_encode(t * (1 - rel)) != norms.fp8_e4m3fn_encode(t * (1 + rel))


def assert_fp8_close(q_got, s_got, q_ref, s_ref, what="", t_ref=None, s_atol=None):
    """fp8 output bar: per-row scales within 1e-6 relative (plus s_atol per row where given: the
    fp32 evaluation allowance of the row maximum over 448, for rows whose statistics are
    ill-conditioned); codes identical except +-1 code on at most 0.1% of the elements.  With
    t_ref (the reference's unquantized scaled values), a +-1 code at an element within fp32 noise
    of a rounding midpoint (fp8_ambiguous) does not count against the 0.1%."""
    s_got = np.asarray(s_got, np.float64)
    s_ref = np.asarray(s_ref, np.float64)
    err = np.abs(s_got - s_ref) - (0.0 if s_atol is None else np.asarray(s_atol, np.float64))
    rel = np.maximum(err, 0.0) / np.where(s_ref > 0, s_ref, 1.0)
    assert rel.max() <= 1e-6, f"{what}: scale rel err {rel.max():.3g}"
    diff = np.abs(fp8_ordinal(q_got) - fp8_ordinal(q_ref))
    assert int(diff.max()) <= 1, f"{what}: a code differs by {int(diff.max())} steps"
    counted = diff != 0
    if t_ref is not None:
        counted &= ~fp8_ambiguous(t_ref)
    n_diff = int(counted.sum())
    assert n_diff <= 1e-3 * diff.size, f"{what}: {n_diff} of {diff.size} codes differ"


def assert_mx_close(q_got, sc_got, q_ref, sc_ref, y_ref, what="", block=32):
    """MXFP8 bar.  E8M0 block scales identical, except that a block whose float64 maximum lies
    within 2^-20 (relative) of a power of two may take the neighbouring exponent (an fp32
    evaluation of the maximum can land on either side); codes compared in the blocks whose
    scales agree, to the fp8 bar of assert_fp8_close with ties excused."""
    from oracle import norms
    sc_got = np.asarray(sc_got).astype(np.int64)
    sc_ref = np.asarray(sc_ref).astype(np.int64)
    y = np.asarray(y_ref, np.float64).reshape(*sc_ref.shape, block)
    amax = np.abs(y).max(axis=-1)
    frac, _ = np.frexp(amax)
    near_pow2 = (np.abs(frac - 0.5) <= 2.0 ** -21) | (np.abs(frac - 1.0) <= 2.0 ** -21)
    bad = (sc_got != sc_ref) & ~((np.abs(sc_got - sc_ref) == 1) & near_pow2)
    assert not bad.any(), f"{what}: {int(bad.sum())} block scales differ"
    same = sc_got == sc_ref
    t = y * np.exp2(-(sc_ref - 127).astype(np.float64))[..., None]
    qg = np.asarray(q_got).reshape(y.shape)[same]
    qr = np.asarray(q_ref).reshape(y.shape)[same]
    diff = np.abs(fp8_ordinal(qg) - fp8_ordinal(qr))
    if diff.size:
        assert int(diff.max()) <= 1, f"{what}: a code differs by {int(diff.max())} steps"
        counted = (diff != 0) & ~fp8_ambiguous(t[same])
        assert int(counted.sum()) <= 1e-3 * diff.size, \
            f"{what}: {int(counted.sum())} of {diff.size} codes differ"
    del norms
