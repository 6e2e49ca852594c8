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


TAB_N = 256      # kGeluTabN
TAB_MAX = 6.0    # kGeluTabMax


def gelu_table(kind="erf", n=TAB_N, vmax=TAB_MAX):
    """A GELU'-table of fln_gelu_table.h: for interval k of |v| in [k h, (k + 1) h), h = vmax /
    (n - 1), the quadratic c0 + c1 f + c2 f^2 (f in [0, 1)) through T(v) = 2 GELU'(v) - 1 at the
    interval's ends and middle, computed in float64 and rounded to fp32; the last interval is the
    constant 1.  kind "erf": T = erf(v / sqrt 2) + v sqrt(2 / pi) exp(-v^2 / 2); kind "tanh" (the
    tanh form, u = sqrt(2 / pi) (v + 0.044715 v^3)): T = tanh(u) + v u'(v) sech^2(u).
    Returns [n, 3] fp32."""
    from scipy.special import erf
    h = vmax / (n - 1)
    k = np.arange(n, dtype=np.float64)

    def t(v):
        if kind == "erf":
            return erf(v / np.sqrt(2)) + v * np.sqrt(2 / np.pi) * np.exp(-v * v / 2)
        k0, k1 = np.sqrt(2 / np.pi), 0.044715
        u = k0 * (v + k1 * v ** 3)
        return np.tanh(u) + v * k0 * (1 + 3 * k1 * v * v) / np.cosh(u) ** 2
    a, m, b = t(k * h), t((k + 0.5) * h), t((k + 1) * h)
    c = np.stack([a, 4 * m - 3 * a - b, 2 * (a + b) - 4 * m], axis=1)
    c[-1] = (1.0, 0.0, 0.0)
    return c.astype(np.float32)


def gelu_grad_table(tab, v, vmax=TAB_MAX):
    """fp32 emulation of gelu_erf_grad2_sign_tab() on u = fp32(v (n - 1) / vmax): the derivative
    it implies, (1 + s) / 2."""
    f32 = np.float32
    n = tab.shape[0]
    u = (v.astype(f32) * f32((n - 1) / vmax)).astype(f32)
    au = np.abs(u)
    with np.errstate(invalid="ignore"):
        f = (au - np.floor(au)).astype(f32)
        k = np.minimum(au, f32(n - 1))
        k = np.where(np.isnan(k), f32(n - 1), k).astype(np.int64)
    c = tab[k]
    r = _fma32(_fma32(c[:, 2], f, c[:, 1]), f, c[:, 0])
    return ((f32(1) + np.copysign(r, u)) * f32(0.5)).astype(f32)


LOG_TAB_N = 256     # kGeluLogTabN
LOG_TAB_INV_H = 16  # kGeluLogTabInvH: interval width 1 / 16, a power of two


def gelu_log_table(n=LOG_TAB_N, inv_h=LOG_TAB_INV_H):
    """The forward's GELU table (kGeluLogTabData): for interval k of x = |v| in [k h, (k + 1) h),
    h = 1 / inv_h, the quadratic c0 + c1 f + c2 f^2 through L(x) = log2(Phi(-x)) - log2(inv_h) at
    the interval's ends and middle (float64, rounded to fp32), so that 2^L = Phi(-|v|) h and
    GELU(v) = max(v, 0) - (|v| inv_h) 2^L; the last interval (|v| >= (n - 1) h, where Phi(-|v|)
    is far below the fp32 range) is the constant -inf.  Returns [n, 3] fp32."""
    from scipy.special import log_ndtr
    h = 1.0 / inv_h
    k = np.arange(n, dtype=np.float64)

    def lg(x):
        return log_ndtr(-x) / np.log(2) - np.log2(inv_h)
    a, m, b = lg(k * h), lg((k + 0.5) * h), lg((k + 1) * h)
    c = np.stack([a, 4 * m - 3 * a - b, 2 * (a + b) - 4 * m], axis=1)
    c[-1] = (-np.inf, 0.0, 0.0)
    return c.astype(np.float32)


def gelu_log_tab(tab, v, inv_h=LOG_TAB_INV_H):
    """fp32 emulation of gelu_erf_tab(): uc = min(|v| inv_h, n - 1), f = fract(uc), L from
    interval floor(uc), GELU = fma(-uc, 2^L, maximum(v, 0)) (maximum propagates NaN)."""
    f32 = np.float32
    n = tab.shape[0]
    v = v.astype(f32)
    with np.errstate(invalid="ignore", over="ignore"):
        au = (np.abs(v) * f32(inv_h)).astype(f32)
        uc = np.where(np.isnan(au), f32(n - 1), np.minimum(au, f32(n - 1))).astype(f32)
        f = (uc - np.floor(uc)).astype(f32)
        c = tab[uc.astype(np.int64)]
        lg = _fma32(_fma32(c[:, 2], f, c[:, 1]), f, c[:, 0])
        r = np.exp2(lg).astype(f32)
        m = np.where(np.isnan(v), v, np.maximum(v, f32(0))).astype(f32)
        return _fma32(-uc, r, m)


def table_header(tabs, vmax=TAB_MAX):
    """C++ source of fln_gelu_table.h from {"erf": table, "tanh": table}."""
    n = tabs["erf"].shape[0]

    def lit(x):
        return "-__builtin_huge_valf()" if x == -np.inf else "%.9ef" % x

    def body(tab):
        return ",\n".join("    %s, %s, %s, 0.0f" % tuple(lit(float(x)) for x in r) for r in tab)
    return ("// fln_gelu_table.h -- generated by `python3 fit_erfc.py table` (beside this file); do not\n"
            "// edit.  Interval k of |v| in [k h, (k + 1) h), h = %g / %d: the coefficients c0, c1, c2 (and\n"
            "// a zero pad) of the quadratic through T(v) = 2 GELU'(v) - 1 at the interval's ends and\n"
            "// middle, in float64 rounded to fp32; the last interval is the constant 1.  kGeluTabData:\n"
            "// the erf form, T = erf(v / sqrt 2) + v sqrt(2 / pi) exp(-v^2 / 2); kGeluTanhTabData: the\n"
            "// tanh form, T = tanh(u) + v u'(v) sech^2(u), u = sqrt(2 / pi) (v + 0.044715 v^3).\n"
            "#pragma once\n\nnamespace fln {\n\n"
            "constexpr int kGeluTabN = %d;\n"
            "constexpr float kGeluTabMax = %.1ff;\n\n"
            "__device__ __attribute__((aligned(16))) const float kGeluTabData[kGeluTabN * 4] = {\n%s};\n\n"
            "__device__ __attribute__((aligned(16))) const float kGeluTanhTabData[kGeluTabN * 4] = {\n%s};\n\n"
            "// The forward's table (fit_erfc.gelu_log_table): interval k of |v| in [k / %d, (k + 1) / %d),\n"
            "// the quadratic through L = log2(Phi(-|v|)) - log2(%d) (2^L = Phi(-|v|) / %d); the last\n"
            "// interval is -inf.\n"
            "constexpr int kGeluLogTabN = %d;\n"
            "constexpr float kGeluLogTabInvH = %d.0f;\n\n"
            "__device__ __attribute__((aligned(16))) const float kGeluLogTabData[kGeluLogTabN * 4] = {\n%s};\n\n"
            "}  // namespace fln\n" % (vmax, n - 1, n, vmax, body(tabs["erf"]), body(tabs["tanh"]),
                                        LOG_TAB_INV_H, LOG_TAB_INV_H, LOG_TAB_INV_H, LOG_TAB_INV_H,
                                        tabs["log"].shape[0], LOG_TAB_INV_H, body(tabs["log"])))


if __name__ == "__main__":
    import sys
    if sys.argv[1:] == ["table"]:
        sys.stdout.write(table_header({"erf": gelu_table("erf"), "tanh": gelu_table("tanh"),
                                       "log": gelu_log_table()}))
        sys.exit(0)
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
    d3 = gelu_grad_table(gelu_table(), v)
    print("derivative (table) max abs error %.3g" % np.abs(d3 - dref).max())
    g3 = gelu_log_tab(gelu_log_table(), v)
    print("GELU (log table) max abs error %.3g, max relative error %.3g (|GELU| > 1e-30)"
          % (np.abs(g3 - gref).max(), (np.abs(g3 - gref)[big] / np.abs(gref[big])).max()))
