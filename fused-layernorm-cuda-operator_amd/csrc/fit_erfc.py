"""Fits the polynomial behind normal_cdf() in fln_device.h (the exact-erf GELU and its derivative).

For x >= 0 and t = 1 / (1 + p x), the scaled complementary error function erfcx(x) =
exp(x^2) erfc(x) divided by t is smooth on t in (0, 1] (it tends to p / sqrt(pi) as t -> 0 and
is 1 at t = 1), so a low-degree polynomial F(t) in t gives

    0.5 erfc(x) = t F(t) exp(-x^2)     (the factor 0.5 folded into F's coefficients)

with a small relative error everywhere, including the far tail where 1 + erf(-x) cancels.  The
coefficients are a least-squares fit of the relative error on Chebyshev nodes of t, reweighted
towards the largest residuals (a few dozen rounds approach the minimax fit).

Run with scipy available: prints the coefficients (0.5 folded in, rounded to fp32) and the fit's
maximum relative error, plus the maximum errors of GELU and its derivative under an fp32
emulation of the device evaluation.
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


def emulate(coef, v, p=P):
    """fp32 emulation of normal_cdf(): (Phi(v), exp(-v^2 / 2))."""
    f32 = np.float32
    v = v.astype(f32)
    e = np.exp2((f32(-0.5 * np.log2(np.e)) * v) * v).astype(f32)
    t = (f32(1) / (f32(p / np.sqrt(2)) * np.abs(v) + f32(1))).astype(f32)
    acc = np.full_like(t, coef[-1])
    for ci in coef[-2::-1]:
        acc = (acc * t + ci).astype(f32)
    h = ((acc * t) * e).astype(f32)
    return np.where(v < 0, h, f32(1) - h).astype(f32), e


if __name__ == "__main__":
    coef, rel = fit()
    print("p =", P, "degree =", DEGREE, "fit max relative error %.3g" % rel)
    print("coefficients:", ", ".join("%.9ef" % c for c in coef))
    v = np.linspace(-13, 13, 2600001).astype(np.float32)
    cdf, e = emulate(coef, v)
    gelu = (v * cdf).astype(np.float32)
    grad = (v * (np.float32(1 / np.sqrt(2 * np.pi)) * e) + cdf).astype(np.float32)
    vd = v.astype(np.float64)
    phi = np.where(vd < 0, 0.5 * erfc(-vd / np.sqrt(2)), 1 - 0.5 * erfc(vd / np.sqrt(2)))
    gref = vd * phi
    dref = phi + vd * np.exp(-vd * vd / 2) / np.sqrt(2 * np.pi)
    big = np.abs(gref) > 1e-30
    print("GELU max abs error %.3g, max relative error %.3g (|GELU| > 1e-30)"
          % (np.abs(gelu - gref).max(), (np.abs(gelu - gref)[big] / np.abs(gref[big])).max()))
    print("derivative max abs error %.3g" % np.abs(grad - dref).max())
