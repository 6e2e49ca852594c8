"""numpy fp64 restatement of the fused normalization path (test infrastructure only).

Every function cites the reference code whose behaviour it restates (paths relative to the
JonSnow1807/Fused-LayerNorm-CUDA-Operator tree).  Where the reference has no code (RMSNorm,
residual add, fp8 output, every backward, erf-GELU) the function restates the mathematics and the
PyTorch semantics the reference defers to; ``tests/test_oracle.py`` pins each one against
PyTorch-CPU, closed forms, invariants, finite differences or a known-answer table.

All arithmetic is float64; inputs may be any float dtype (bf16 values arrive as exact float32).
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "layer_norm_fwd", "layer_norm_gelu_fwd", "gelu", "rms_norm_fwd", "round_to_bf16",
    "round_to_f16", "add_layer_norm_fwd", "add_rms_norm_fwd", "layer_norm_bwd", "rms_norm_bwd",
    "fp8_e4m3fn_encode", "fp8_e4m3fn_decode", "layer_norm_fp8_fwd", "rms_norm_fp8_fwd",
    "add_layer_norm_fp8_fwd", "add_rms_norm_fp8_fwd", "gelu_grad", "layer_norm_gelu_bwd",
    "mx_e4m3_quantize", "layer_norm_mxfp8_fwd", "rms_norm_mxfp8_fwd", "add_rms_norm_mxfp8_fwd",
    "FP8_E4M3FN_MAX", "MX_BLOCK",
]

FP8_E4M3FN_MAX = 448.0
MX_BLOCK = 32


def _f64(a):
    return None if a is None else np.asarray(a, dtype=np.float64)


def layer_norm_fwd(x, gamma=None, beta=None, eps=1e-5):
    """LayerNorm over the last axis -> (y, mean, rstd).

    Follows ``layernorm_kernel`` (csrc/layernorm_cuda_kernel.cu:39-92): mean = sum(x)/N
    (:57-66), two-pass biased variance sum((x-mean)^2)/N (:69-80), rstd = 1/sqrt(var + eps)
    (:79), y = (x - mean) * rstd (:86).  The affine step follows torch.nn.functional.layer_norm
    (gamma and beta applied independently), which is what the reference's module wraps
    (fused_layernorm/layernorm.py:189-193); the reference kernel's "both or neither" gating
    (:87) is enforced by the binding's argument check instead.
    """
    x = _f64(x)
    mean = x.mean(axis=-1, keepdims=True)
    var = np.square(x - mean).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (x - mean) * rstd
    if gamma is not None:
        y = y * _f64(gamma)
    if beta is not None:
        y = y + _f64(beta)
    return y, mean[..., 0], rstd[..., 0]


def gelu(v, approximate="none"):
    """GELU.  'tanh' is the reference's fused form (csrc/layernorm_cuda_kernel.cu:31-36):
    0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))).  'none' is the exact
    0.5 v (1 + erf(v / sqrt 2)) (torch approximate='none'), the form the C2 config uses.
    """
    v = _f64(v)
    if approximate == "tanh":
        return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))
    if approximate == "none":
        from scipy.special import erf
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    raise ValueError(approximate)


def gelu_grad(v, approximate="none"):
    """d GELU / dv.  'none': Phi(v) + v phi(v); 'tanh': with u = sqrt(2/pi)(v + 0.044715 v^3),
    t = tanh(u): 0.5 (1 + t) + 0.5 v (1 - t^2) sqrt(2/pi) (1 + 3 * 0.044715 v^2) -- the
    derivative of the reference's gelu() (csrc/layernorm_cuda_kernel.cu:31-36)."""
    v = _f64(v)
    if approximate == "tanh":
        k0, k1 = np.sqrt(2.0 / np.pi), 0.044715
        t = np.tanh(k0 * (v + k1 * v ** 3))
        return 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t * t) * k0 * (1.0 + 3.0 * k1 * v * v)
    if approximate == "none":
        from scipy.special import erf
        return 0.5 * (1.0 + erf(v / np.sqrt(2.0))) + v * np.exp(-0.5 * v * v) / np.sqrt(2 * np.pi)
    raise ValueError(approximate)


def layer_norm_gelu_fwd(x, gamma=None, beta=None, eps=1e-5, approximate="tanh"):
    """GELU(LayerNorm(x)) -- ``layernorm_gelu_kernel`` (csrc/layernorm_cuda_kernel.cu:96-148):
    the LayerNorm of :113-144 followed by gelu() on the affine output (:146)."""
    y, _, _ = layer_norm_fwd(x, gamma, beta, eps)
    return gelu(y, approximate)


def rms_norm_fwd(x, weight=None, eps=1e-6):
    """RMSNorm over the last axis -> (y, rstd): rstd = 1/sqrt(mean(x^2) + eps), y = x rstd w.
    No reference code (new on this path); semantics of torch.nn.functional.rms_norm."""
    x = _f64(x)
    rstd = 1.0 / np.sqrt(np.square(x).mean(axis=-1, keepdims=True) + eps)
    y = x * rstd
    if weight is not None:
        y = y * _f64(weight)
    return y, rstd[..., 0]


def round_to_bf16(a):
    """Round to the nearest bfloat16 (ties to even) via float32, as torch's bf16 add does:
    the float32 sum is rounded once more to bf16.  Returns float32 values."""
    a32 = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    bits = a32.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    r = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a32), a32, r)


def round_to_f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def _round_io(a, dtype):
    if dtype == "bf16":
        return round_to_bf16(a)
    if dtype == "f16":
        return round_to_f16(a)
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "f64":
        return np.asarray(a, dtype=np.float64)
    raise ValueError(dtype)


def add_layer_norm_fwd(x, residual, gamma=None, beta=None, eps=1e-5, io_dtype="bf16"):
    """Residual add + LayerNorm -> (y, h, mean, rstd).  h = x + residual computed in float32 and
    rounded to the I/O type (what the kernel stores); the statistics are taken over that rounded
    h, so y == LayerNorm(h_stored).  No reference code (new on this path)."""
    s = np.asarray(x, np.float32) + np.asarray(residual, np.float32)
    h = _round_io(s, io_dtype) if io_dtype != "f64" else _f64(x) + _f64(residual)
    y, mean, rstd = layer_norm_fwd(h, gamma, beta, eps)
    return y, h, mean, rstd


def add_rms_norm_fwd(x, residual, weight=None, eps=1e-6, io_dtype="bf16"):
    """Residual add + RMSNorm -> (y, h, rstd); same rounding rule for h as add_layer_norm_fwd."""
    s = np.asarray(x, np.float32) + np.asarray(residual, np.float32)
    h = _round_io(s, io_dtype)
    y, rstd = rms_norm_fwd(h, weight, eps)
    return y, h, rstd


def layer_norm_bwd(dy, x, gamma=None, eps=1e-5):
    """LayerNorm backward closed form -> (dx, dgamma, dbeta), statistics recomputed in fp64.

    The reference declares this contract (``layernorm_backward_cuda``, csrc/layernorm.h:24-32;
    inputs grad_output, input, mean, rstd, gamma; outputs grad_input, grad_gamma, grad_beta,
    csrc/layernorm_cuda.cpp:97-141) without defining it.  With xhat = (x - mean) rstd and
    g = dy gamma:  dx = rstd (g - mean(g) - xhat mean(g xhat)),  dgamma = sum_rows dy xhat,
    dbeta = sum_rows dy.
    """
    dy, x = _f64(dy), _f64(x)
    _, mean, rstd = layer_norm_fwd(x, None, None, eps)
    mean, rstd = mean[..., None], rstd[..., None]
    xh = (x - mean) * rstd
    g = dy * _f64(gamma) if gamma is not None else dy
    dx = rstd * (g - g.mean(axis=-1, keepdims=True) - xh * (g * xh).mean(axis=-1, keepdims=True))
    red = tuple(range(dy.ndim - 1))
    return dx, (dy * xh).sum(axis=red), dy.sum(axis=red)


def layer_norm_gelu_bwd(dy, x, gamma=None, beta=None, eps=1e-5, approximate="tanh"):
    """Backward of GELU(LayerNorm(x) gamma + beta) -> (dx, dgamma, dbeta): with a the GELU
    input, the LayerNorm backward (layer_norm_bwd) of the upstream gradient dy GELU'(a).  No
    reference code (the reference has no backward for its fused LayerNorm + GELU)."""
    y, _, _ = layer_norm_fwd(x, gamma, beta, eps)
    return layer_norm_bwd(_f64(dy) * gelu_grad(y, approximate), x, gamma, eps)


def rms_norm_bwd(dy, x, weight=None, eps=1e-6):
    """RMSNorm backward closed form -> (dx, dweight): xhat = x rstd, g = dy w,
    dx = rstd (g - xhat mean(g xhat)), dweight = sum_rows dy xhat.  No reference code."""
    dy, x = _f64(dy), _f64(x)
    _, rstd = rms_norm_fwd(x, None, eps)
    rstd = rstd[..., None]
    xh = x * rstd
    g = dy * _f64(weight) if weight is not None else dy
    dx = rstd * (g - xh * (g * xh).mean(axis=-1, keepdims=True))
    red = tuple(range(dy.ndim - 1))
    return dx, (dy * xh).sum(axis=red)


def fp8_e4m3fn_encode(v):
    """OCP fp8 e4m3fn encoder with saturation and round-to-nearest-even -> uint8 codes.

    Format: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; no infinities; 0x7F/0xFF are
    NaN; the largest finite magnitude is 448 (0x7E); subnormals are m * 2^-9 (m = 1..7).
    Magnitudes above 448 saturate to 448; NaN maps to 0x7F.  Written from the format definition
    (no reference code: fp8 output is new on this path).
    """
    v = np.asarray(v, dtype=np.float64)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.minimum(np.abs(np.nan_to_num(v, nan=0.0)), FP8_E4M3FN_MAX)
    code = np.zeros(v.shape, dtype=np.int64)
    sub = a < 2.0 ** -6
    # Subnormal range (a rounding up to 8 * 2^-9 lands exactly on the smallest normal, code 8).
    code[sub] = np.rint(a[sub] / 2.0 ** -9).astype(np.int64)
    nrm = ~sub
    f, k = np.frexp(a[nrm])             # a = f 2^k, f in [0.5, 1)
    e = k - 1                            # a = (2f) 2^e, 2f in [1, 2)
    mq = np.rint(16.0 * f - 8.0).astype(np.int64)  # (2f - 1) * 8, ties to even
    carry = mq == 8
    e = np.where(carry, e + 1, e)
    mq = np.where(carry, 0, mq)
    code[nrm] = ((e + 7) << 3) | mq
    code = np.minimum(code, 0x7E)        # saturation (448 = 0x7E)
    out = (code.astype(np.uint8) | sign)
    return np.where(np.isnan(v), np.uint8(0x7F), out).astype(np.uint8)


def fp8_e4m3fn_decode(codes):
    """Decode e4m3fn codes to float64 (NaN for 0x7F / 0xFF)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = s * val
    return np.where((c & 0x7F) == 0x7F, np.nan, val)


def layer_norm_fp8_fwd(x, gamma=None, beta=None, eps=1e-5):
    """LayerNorm with fp8 output -> (codes uint8, scale float32 per row).
    v = LayerNorm(x) (affine), scale = max|v| / 448 per row, codes = sat_rne_e4m3fn(v / scale);
    a row with max|v| == 0 gets scale 0 and all-zero codes.  A row whose statistics are not usable
    (see unusable_rows: a NaN or an infinity in the row) gets a NaN scale, and the codes under a
    NaN scale carry no value; for such rows this is torch's amax of v as well.  gamma and beta are
    taken to be finite.  No reference code."""
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        y, mean, rstd = layer_norm_fwd(x, gamma, beta, eps)
    return _row_fp8(y, unusable_rows(mean, rstd))


def unusable_rows(mean, rstd):
    """Rows whose statistics leave every output meaningless: a mean that is not finite, or an rstd
    outside (0, inf) -- a NaN or an infinity in the row (in float64; fp32 statistics also flag a
    sum of squares past 3.4e38), or a constant row with eps = 0.  Their fp8 row scale is NaN and
    every MX block scale 0xFF (E8M0's NaN), so a reader sees NaN throughout."""
    mean, rstd = np.asarray(mean), np.asarray(rstd)
    return ~np.isfinite(mean) | ~((rstd > 0) & (rstd < np.inf))


def _row_fp8(y, bad):
    with np.errstate(invalid="ignore"):
        amax = np.abs(y).max(axis=-1, keepdims=True)
    scale = np.where(bad[..., None], np.nan, amax / FP8_E4M3FN_MAX)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(amax > 0, y / np.where(amax > 0, scale, 1.0), 0.0)
    return fp8_e4m3fn_encode(q), scale[..., 0].astype(np.float32)


def rms_norm_fp8_fwd(x, weight=None, eps=1e-6):
    """RMSNorm with fp8 output -> (codes, scale): the row rule of layer_norm_fp8_fwd applied to
    rms_norm_fwd's output.  No reference code."""
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        y, rstd = rms_norm_fwd(x, weight, eps)
    return _row_fp8(y, unusable_rows(np.zeros_like(rstd), rstd))


def add_layer_norm_fp8_fwd(x, residual, gamma=None, beta=None, eps=1e-5, io_dtype="bf16"):
    """Residual add + LayerNorm -> fp8: (codes, scale, h); h rounded as in add_layer_norm_fwd.
    No reference code."""
    y, h, mean, rstd = add_layer_norm_fwd(x, residual, gamma, beta, eps, io_dtype)
    q, scale = _row_fp8(y, unusable_rows(mean, rstd))
    return q, scale, h


def add_rms_norm_fp8_fwd(x, residual, weight=None, eps=1e-6, io_dtype="bf16"):
    """Residual add + RMSNorm -> fp8: (codes, scale, h).  No reference code."""
    y, h, rstd = add_rms_norm_fwd(x, residual, weight, eps, io_dtype)
    q, scale = _row_fp8(y, unusable_rows(np.zeros_like(rstd), rstd))
    return q, scale, h


def mx_e4m3_quantize(y, block=MX_BLOCK):
    """OCP Microscaling (MX v1.0) MXFP8 E4M3 of the last axis -> (codes uint8, E8M0 scales uint8
    [..., n / block]).  Per block of `block` consecutive elements: shared exponent
    e = floor(log2(max|y|)) - 8 (8 = emax of E4M3), clamped to [-127, 127] (a zero maximum gives
    -127); scale byte e + 127; codes = sat_rne_e4m3fn(y 2^-e).  A block whose maximum is not
    finite (an infinity, or a NaN, which the maximum propagates) gets the scale byte 0xFF, E8M0's
    NaN (torch's float8_e8m0fnu cast of 2^(floor(log2 max) - 8) gives the same byte), under which
    every element of the block reads as NaN: its codes carry no value (here those of e = 120).
    Written from the format definition (no reference code)."""
    y = _f64(y)
    n = y.shape[-1]
    if n % block:
        raise ValueError("the row length must be a multiple of the block")
    yb = y.reshape(*y.shape[:-1], n // block, block)
    amax = np.abs(yb).max(axis=-1)
    finite = np.isfinite(amax)
    _, k = np.frexp(np.where(finite, amax, 1.0))  # amax = f 2^k, f in [0.5, 1): floor(log2) = k - 1
    e = np.where(finite, np.where(amax > 0, k - 1 - 8, -127), 120)
    e = np.clip(e, -127, 127).astype(np.int64)
    with np.errstate(invalid="ignore"):
        codes = fp8_e4m3fn_encode(yb * np.exp2(-e.astype(np.float64))[..., None])
    return codes.reshape(y.shape), np.where(finite, e + 127, 0xFF).astype(np.uint8)


def _mx_rows(y, bad):
    q, sc = mx_e4m3_quantize(y)
    sc[np.asarray(bad)] = 0xFF  # every block of a row with unusable statistics reads as NaN
    return q, sc


def layer_norm_mxfp8_fwd(x, gamma=None, beta=None, eps=1e-5):
    """LayerNorm -> MXFP8 E4M3 (codes, E8M0 block scales); rows with unusable statistics
    (unusable_rows) get 0xFF in every block.  No reference code."""
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        y, mean, rstd = layer_norm_fwd(x, gamma, beta, eps)
    return _mx_rows(y, unusable_rows(mean, rstd))


def rms_norm_mxfp8_fwd(x, weight=None, eps=1e-6):
    """RMSNorm -> MXFP8 E4M3; rows with unusable statistics get 0xFF in every block (an infinity
    makes rstd 0: torch's composition would give only the block holding it 0xFF, the others the
    scale and codes of zeros).  No reference code."""
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        y, rstd = rms_norm_fwd(x, weight, eps)
    return _mx_rows(y, unusable_rows(np.zeros_like(rstd), rstd))


def add_rms_norm_mxfp8_fwd(x, residual, weight=None, eps=1e-6, io_dtype="bf16"):
    """Residual add + RMSNorm -> MXFP8 E4M3: (codes, block scales, h).  No reference code."""
    y, h, rstd = add_rms_norm_fwd(x, residual, weight, eps, io_dtype)
    q, sc = _mx_rows(y, unusable_rows(np.zeros_like(rstd), rstd))
    return q, sc, h
