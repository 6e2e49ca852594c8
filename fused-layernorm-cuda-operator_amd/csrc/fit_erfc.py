"""Fits the polynomial behind erfc_terms() in fln_device.h (the exact-erf GELU and its derivative).

For x >= 0 and t = 1 / (1 + p x), the scaled complementary error function erfcx(x) =
exp(x^2) erfc(x) divided by t is smooth on t in (0, 1] (it tends to p / sqrt(pi) as t -> 0 and
is 1 at t = 1), so a low-degree polynomial F(t) in t gives

    0.5 erfc(x) = t F(t) exp(-x^2)     (the factor 0.5 folded into F's coefficients)

with a small relative error everywhere, including the far tail where 1 + erf(-x) cancels.  The
coefficients are a least-squares fit of the relative error on Chebyshev nodes of t, reweighted
towards the largest residuals (a few dozen rounds approach the minimax fit).

Run with scipy available: prints the coefficients (0.5 folded in, rounded to fp32) and the fit's
maximum relative error, plus the maximum errors of GELU and its derivative under an fp32
emulation of the device evaluation (gelu_erf() and gelu_erf_grad(): the same operations in the
same order, each rounded to fp32; FMAs rounded once).
"""
import numpy as np
from scipy.special import erfc, erfcx

P = 0.35
DEGREE = 7


def fit(p=P, deg=DEGREE, nodes=4000, rounds=60):
    k = np.arange(nodes)
    t = 0.5 - 0.5 * np.cos(np.pi * (k + 0.5) / nodes)
    x = (1 - t) / (p * t)
    f = erfcx(x) / t
    vand = np.vander(t, deg + 1, increasing=True)
    w = np.ones_like(t)
    c, *_ = np.linalg.lstsq(vand / f[:, None], np.ones_like(t), rcond=None)
    for _ in range(rounds):
        r = (vand @ c - f) / f
        w = w * (np.abs(r) / np.abs(r).max() + 1e-4) ** 0.5
        w /= w.max()
        c, *_ = np.linalg.lstsq(vand * (w / f)[:, None], w, rcond=None)
    rel = np.abs((vand @ c - f) / f).max()
    return [np.float32(0.5 * ci) for ci in c], rel


def _fma32(a, b, c):
    """fp32 FMA: the float64 product of two fp32 values is exact; one rounding to fp32."""
    return (a.astype(np.float64) * b.astype(np.float64) + c).astype(np.float32)


def terms(coef, v, p=P):
    """fp32 emulation of erfc_terms(): (t, exp(-v^2 / 2), F(t))."""
    f32 = np.float32
    v = v.astype(f32)
    e = np.exp2((f32(-0.5 * np.log2(np.e)) * v) * v).astype(f32)
    t = (f32(1) / _fma32(np.full_like(v, f32(p / np.sqrt(2))), np.abs(v), f32(1))).astype(f32)
    acc = np.full_like(t, coef[-1])
    for ci in coef[-2::-1]:
        acc = _fma32(acc, t, ci)
    return t, e, acc


def gelu(coef, v, p=P):
    """fp32 emulation of gelu_erf(): max(v, 0) - (|v| (t e)) F(t), |v| (t e) = 0 where t e = 0."""
    f32 = np.float32
    v = v.astype(f32)
    t, e, f = terms(coef, v, p)
    te = (t * e).astype(f32)
    with np.errstate(invalid="ignore"):
        q = np.where(te == 0, f32(0), (np.abs(v) * te).astype(f32))
    return _fma32(-q, f, np.maximum(v, f32(0)))


def gelu_grad(coef, v, p=P):
    """fp32 emulation of gelu_erf_grad(): 1/2 + copysign(1/2 - e (t F - |v| / sqrt(2 pi)), v)."""
    f32 = np.float32
    v = v.astype(f32)
    t, e, f = terms(coef, v, p)
    w = _fma32(np.full_like(v, f32(-1 / np.sqrt(2 * np.pi))), np.abs(v), (t * f).astype(f32))
    y = _fma32(-e, w, f32(0.5))
    return (f32(0.5) + np.copysign(y, v)).astype(f32)


K_U = np.sqrt(np.log2(np.e) / 2)  # kGeluU: u = v sqrt(log2(e) / 2), exp(-v^2 / 2) = 2^(-u^2)


def gelu_grad_scaled(coef, v, p=P):
    """fp32 emulation of gelu_erf_grad2_sign() on u = fp32(K_U v): the derivative it implies,
    (1 + s) / 2 with s = copysign(1 - e (t 2F - (2 / (sqrt(2 pi) K_U)) |u|), u)."""
    f32 = np.float32
    u = (f32(K_U) * v.astype(f32)).astype(f32)
    e = np.exp2(-(u * u).astype(f32)).astype(f32)
    a = f32(p / np.sqrt(2) / K_U)
    t = (f32(1) / _fma32(np.full_like(u, a), np.abs(u), f32(1))).astype(f32)
    acc = np.full_like(t, f32(2) * coef[-1])
    for ci in coef[-2::-1]:
        acc = _fma32(acc, t, f32(2) * ci)
    k2 = f32(2 / np.sqrt(2 * np.pi) / K_U)
    w2 = _fma32(np.full_like(u, -k2), np.abs(u), (t * acc).astype(f32))
    sgn = np.copysign(_fma32(-e, w2, f32(1)), u)
    return ((f32(1) + sgn) * f32(0.5)).astype(f32)


if __name__ == "__main__":
    coef, rel = fit()
    print("p =", P, "degree =", DEGREE, "fit max relative error %.3g" % rel)
    print("coefficients:", ", ".join("%.9ef" % c for c in coef))
    v = np.linspace(-13, 13, 2600001).astype(np.float32)
    g = gelu(coef, v)
    d = gelu_grad(coef, v)
    vd = v.astype(np.float64)
    phi = np.where(vd < 0, 0.5 * erfc(-vd / np.sqrt(2)), 1 - 0.5 * erfc(vd / np.sqrt(2)))
    gref = vd * phi
    dref = phi + vd * np.exp(-vd * vd / 2) / np.sqrt(2 * np.pi)
    big = np.abs(gref) > 1e-30
    print("GELU max abs error %.3g, max relative error %.3g (|GELU| > 1e-30)"
          % (np.abs(g - gref).max(), (np.abs(g - gref)[big] / np.abs(gref[big])).max()))
    print("derivative max abs error %.3g" % np.abs(d - dref).max())
    d2 = gelu_grad_scaled(coef, v)
    print("derivative (scaled input) max abs error %.3g" % np.abs(d2 - dref).max())
