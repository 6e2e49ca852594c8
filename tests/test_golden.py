"""Golden fixtures (tests/golden/norm_cases.npz, written by tests/golden/make_golden.py from
PyTorch-CPU float64) against the oracle (CPU) and against the HIP kernels through the C ABI (GPU).

The fixtures come from an implementation independent of both: a wrong term, sign, index or
rounding rule in the oracle or in a kernel shows up here even where the two would agree.
Expected float outputs are stored as float32; tolerances are those of the parity bar (stated in
each test).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import capi
from helpers import assert_close_rel, assert_fp8_close, assert_within_ulp, to_np
from oracle import c_oracle, norms

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "norm_cases.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def bf16_from_bits(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


LN_CASES = [0, 1, 2, 3]
BWD_CASES = [0, 1, 2]


def close_f32(got, ref, rtol=2e-7, what=""):
    """Float64 oracle vs a float32-stored PyTorch float64 result: the storage rounding is the
    only difference (<= 2^-24 relative, plus an absolute floor for values near zero)."""
    scale = np.abs(ref).max()
    err = np.abs(np.asarray(got, np.float64) - ref)
    bound = rtol * np.abs(ref) + 1e-7 * scale
    assert (err <= bound).all(), f"{what}: max err {err.max():.3g}"


# ------------------------------------------------------------------------------------------------
# CPU: the oracle reproduces PyTorch's float64 results.
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("i", LN_CASES)
def test_oracle_layer_norm_forward(gold, i):
    k = f"ln{i}"
    x, g, b = gold[f"{k}_x"], gold[f"{k}_g"], gold[f"{k}_b"]
    y, mean, rstd = norms.layer_norm_fwd(x, g, b, 1e-5)
    close_f32(y, gold[f"{k}_y"], what="y")
    close_f32(mean, gold[f"{k}_mean"], what="mean")
    close_f32(rstd, gold[f"{k}_rstd"], what="rstd")
    y0, _, _ = norms.layer_norm_fwd(x, None, None, 1e-5)
    close_f32(y0, gold[f"{k}_y_noaffine"], what="y (no affine)")
    yc, mc, rc = c_oracle.layernorm_fwd(x, g, b, 1e-5)
    close_f32(yc, gold[f"{k}_y"], 3e-7, what="C oracle y")


def test_oracle_layer_norm_gelu(gold):
    for mode, key in (("none", "gelu_y_erf"), ("tanh", "gelu_y_tanh")):
        y = norms.layer_norm_gelu_fwd(gold["gelu_x"], gold["gelu_g"], gold["gelu_b"], 1e-5, mode)
        close_f32(y, gold[key], what=mode)


@pytest.mark.parametrize("mode", ["none", "tanh"])
def test_oracle_layer_norm_gelu_backward(gold, mode):
    dx, dg, db = norms.layer_norm_gelu_bwd(gold["gb_dy"], gold["gb_x"], gold["gb_g"],
                                           gold["gb_b"], 1e-5, mode)
    close_f32(dx, gold[f"gb_{mode}_dx"], 1e-6, what="dx")
    close_f32(dg, gold[f"gb_{mode}_dg"], 1e-6, what="dgamma")
    close_f32(db, gold[f"gb_{mode}_db"], 1e-6, what="dbeta")


@pytest.mark.parametrize("i", [0, 1])
def test_oracle_rms_norm_forward(gold, i):
    k = f"rms{i}"
    y, rstd = norms.rms_norm_fwd(gold[f"{k}_x"], gold[f"{k}_w"], 1e-6)
    close_f32(y, gold[f"{k}_y"], what="y")
    close_f32(rstd, gold[f"{k}_rstd"], what="rstd")


@pytest.mark.parametrize("i", BWD_CASES)
def test_oracle_backward(gold, i):
    k = f"lnb{i}"
    x, g, dy = gold[f"{k}_x"], gold[f"{k}_g"], gold[f"{k}_dy"]
    dx, dg, db = norms.layer_norm_bwd(dy, x, g, 1e-5)
    close_f32(dx, gold[f"{k}_dx"], 1e-6, what="dx")
    close_f32(dg, gold[f"{k}_dg"], 1e-6, what="dgamma")
    close_f32(db, gold[f"{k}_db"], 1e-6, what="dbeta")
    dxr, dw = norms.rms_norm_bwd(dy, x, g, 1e-6)
    close_f32(dxr, gold[f"rmsb{i}_dx"], 1e-6, what="rms dx")
    close_f32(dw, gold[f"rmsb{i}_dw"], 1e-6, what="rms dw")
    dxc, dgc, dbc = c_oracle.layernorm_bwd(dy, x, g, 1e-5)
    close_f32(dxc, gold[f"{k}_dx"], 1e-6, what="C oracle dx")


def test_oracle_residual_add(gold):
    x, r = bf16_from_bits(gold["res_x_bf16"]), bf16_from_bits(gold["res_r_bf16"])
    g, b = bf16_from_bits(gold["res_g_bf16"]), bf16_from_bits(gold["res_b_bf16"])
    y, h, _, _ = norms.add_layer_norm_fwd(x, r, g, b, 1e-5, "bf16")
    assert np.array_equal(h, bf16_from_bits(gold["res_h_bf16"])), "h must be bit-exact"
    close_f32(y, gold["res_y"], what="y")


def test_oracle_fp8(gold):
    x = bf16_from_bits(gold["fp8_x_bf16"])
    g, b = bf16_from_bits(gold["fp8_g_bf16"]), bf16_from_bits(gold["fp8_b_bf16"])
    q, s = norms.layer_norm_fp8_fwd(x, g, b, 1e-5)
    assert_fp8_close(q, s, gold["fp8_q"], gold["fp8_scale"], "oracle fp8")
    assert np.array_equal(norms.fp8_e4m3fn_encode(gold["enc_v"].astype(np.float64)),
                          gold["enc_q"])


def test_oracle_residual_rms_fp8(gold):
    x, r = bf16_from_bits(gold["arf_x_bf16"]), bf16_from_bits(gold["arf_r_bf16"])
    w = bf16_from_bits(gold["arf_w_bf16"])
    q, s, h = norms.add_rms_norm_fp8_fwd(x, r, w, 1e-6, "bf16")
    assert np.array_equal(h, bf16_from_bits(gold["arf_h_bf16"]))
    assert_fp8_close(q, s, gold["arf_q"], gold["arf_scale"], "oracle residual rms fp8")


# ------------------------------------------------------------------------------------------------
# GPU: the kernels reproduce the same fixtures.
# ------------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lib(gpu_available):
    return capi.load()


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to("cuda")


@pytest.mark.gpu
@pytest.mark.parametrize("i", LN_CASES)
def test_gpu_layer_norm_forward_fp32(lib, gold, i):
    from gpu_calls import ln_forward
    k = f"ln{i}"
    x, g, b = dev(gold[f"{k}_x"]), dev(gold[f"{k}_g"]), dev(gold[f"{k}_b"])
    y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    ref = gold[f"{k}_y"].astype(np.float64)
    assert np.abs(to_np(y) - ref).max() <= 1e-5  # fp32 bar: max-abs 1e-5
    assert np.abs(to_np(mean) - gold[f"{k}_mean"]).max() <= 1e-5 * max(1, np.abs(ref).max())
    assert np.abs(to_np(rstd) / gold[f"{k}_rstd"] - 1).max() <= 1e-5
    y0, _, _ = ln_forward(lib, x, None, None, 1e-5, stats=False)
    assert np.abs(to_np(y0) - gold[f"{k}_y_noaffine"]).max() <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["erf", "tanh"])
def test_gpu_layer_norm_gelu_fp32(lib, gold, mode):
    x, g, b = dev(gold["gelu_x"]), dev(gold["gelu_g"]), dev(gold["gelu_b"])
    y = torch.empty_like(x)
    capi.check(lib.fln_layernorm_gelu(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y),
                                      x.shape[0], x.shape[1], capi.F32, 1e-5,
                                      capi.GELU_ERF if mode == "erf" else capi.GELU_TANH,
                                      capi.stream()))
    assert np.abs(to_np(y) - gold[f"gelu_y_{mode}"]).max() <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("i", [0, 1])
def test_gpu_rms_norm_forward_fp32(lib, gold, i):
    from gpu_calls import rms_forward
    k = f"rms{i}"
    y, rstd = rms_forward(lib, dev(gold[f"{k}_x"]), dev(gold[f"{k}_w"]), 1e-6)
    assert np.abs(to_np(y) - gold[f"{k}_y"]).max() <= 1e-5
    assert np.abs(to_np(rstd) / gold[f"{k}_rstd"] - 1).max() <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("i", BWD_CASES)
def test_gpu_backward_fp32(lib, gold, i):
    from gpu_calls import ln_backward, ln_forward, rms_backward, rms_forward
    k = f"lnb{i}"
    x, g, b, dy = (dev(gold[f"{k}_{n}"]) for n in ("x", "g", "b", "dy"))
    _, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
    # fp32 gradients: dx elementwise 1e-4 relative + 1e-5 * max|dx|; column sums 1e-4 max-norm.
    ref = gold[f"{k}_dx"].astype(np.float64)
    assert (np.abs(to_np(dx) - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max()).all()
    assert_close_rel(to_np(dg), gold[f"{k}_dg"], 1e-4, "dgamma")
    assert_close_rel(to_np(db), gold[f"{k}_db"], 1e-4, "dbeta")
    _, rs = rms_forward(lib, x, g, 1e-6)
    dxr, dw = rms_backward(lib, dy, x, rs, g)
    ref = gold[f"rmsb{i}_dx"].astype(np.float64)
    assert (np.abs(to_np(dxr) - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max()).all()
    assert_close_rel(to_np(dw), gold[f"rmsb{i}_dw"], 1e-4, "dweight")


@pytest.mark.gpu
def test_gpu_residual_add_layer_norm_bf16(lib, gold):
    x = dev(bf16_from_bits(gold["res_x_bf16"]), torch.bfloat16)
    r = dev(bf16_from_bits(gold["res_r_bf16"]), torch.bfloat16)
    g = dev(bf16_from_bits(gold["res_g_bf16"]), torch.bfloat16)
    b = dev(bf16_from_bits(gold["res_b_bf16"]), torch.bfloat16)
    y, h = torch.empty_like(x), torch.empty_like(x)
    capi.check(lib.fln_add_layernorm_forward(
        capi.ptr(x), capi.ptr(r), capi.ptr(g), capi.ptr(b), capi.ptr(h), capi.ptr(y), None, None,
        x.shape[0], x.shape[1], capi.BF16, 1e-5, capi.stream()))
    assert np.array_equal(to_np(h), bf16_from_bits(gold["res_h_bf16"])), "h bit-exact"
    # bf16 bar: 1 ulp of the reference, plus the fp32 rounding allowance of the affine step.
    hb = bf16_from_bits(gold["res_h_bf16"]).astype(np.float64)
    xh, _, _ = norms.layer_norm_fwd(hb, None, None, 1e-5)
    gb, bb = to_np(g).astype(np.float64), to_np(b).astype(np.float64)
    atol = 2.0 ** -21 * (np.abs(xh * gb) + np.abs(bb))
    assert_within_ulp(to_np(y), gold["res_y"], 1.0, atol=atol, what="residual y")


@pytest.mark.gpu
def test_gpu_layer_norm_fp8(lib, gold):
    x = dev(bf16_from_bits(gold["fp8_x_bf16"]), torch.bfloat16)
    g = dev(bf16_from_bits(gold["fp8_g_bf16"]), torch.bfloat16)
    b = dev(bf16_from_bits(gold["fp8_b_bf16"]), torch.bfloat16)
    rows, cols = x.shape
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    s = torch.empty(rows, device="cuda")
    capi.check(lib.fln_layernorm_fp8_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(q),
                                             capi.ptr(s), None, None, rows, cols, capi.BF16,
                                             1e-5, capi.stream()))
    assert_fp8_close(q.cpu().numpy(), to_np(s), gold["fp8_q"], gold["fp8_scale"], "gpu fp8")


@pytest.mark.gpu
def test_gpu_fp8_encoder_matches_torch_cast(lib, gold):
    v = dev(gold["enc_v"])
    q = torch.empty(v.numel(), device="cuda", dtype=torch.uint8)
    capi.check(lib.fln_fp8_e4m3fn_encode(capi.ptr(v), capi.ptr(q), v.numel(), capi.stream()))
    assert np.array_equal(q.cpu().numpy(), gold["enc_q"])  # bit-exact


@pytest.mark.gpu
def test_gpu_residual_rms_fp8(lib, gold):
    x = dev(bf16_from_bits(gold["arf_x_bf16"]), torch.bfloat16)
    r = dev(bf16_from_bits(gold["arf_r_bf16"]), torch.bfloat16)
    w = dev(bf16_from_bits(gold["arf_w_bf16"]), torch.bfloat16)
    rows, cols = x.shape
    h = torch.empty_like(x)
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    s = torch.empty(rows, device="cuda")
    capi.check(lib.fln_add_rmsnorm_fp8_forward(capi.ptr(x), capi.ptr(r), capi.ptr(w),
                                               capi.ptr(h), capi.ptr(q), capi.ptr(s), None,
                                               rows, cols, capi.BF16, 1e-6, capi.stream()))
    assert np.array_equal(to_np(h), bf16_from_bits(gold["arf_h_bf16"])), "h bit-exact"
    assert_fp8_close(q.cpu().numpy(), to_np(s), gold["arf_q"], gold["arf_scale"],
                     "gpu residual rms fp8")


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["none", "tanh"])
def test_gpu_layer_norm_gelu_backward_fp32(lib, gold, mode):
    from gpu_calls import workspace
    x, g, b, dy = (dev(gold[f"gb_{n}"]) for n in ("x", "g", "b", "dy"))
    rows, cols = x.shape
    gm = capi.GELU_ERF if mode == "none" else capi.GELU_TANH
    y = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    capi.check(lib.fln_layernorm_gelu_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y),
                                              capi.ptr(mean), capi.ptr(rstd), rows, cols,
                                              capi.F32, 1e-5, gm, capi.stream()))
    dx, dg, db = torch.empty_like(x), torch.empty_like(g), torch.empty_like(b)
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_gelu_backward(
        capi.ptr(dy), capi.ptr(x), capi.ptr(mean), capi.ptr(rstd), capi.ptr(g), capi.ptr(b),
        capi.ptr(dx), capi.ptr(dg), capi.ptr(db), rows, cols, capi.F32, capi.F32, gm,
        capi.ptr(ws), n, capi.stream()))
    ref = gold[f"gb_{mode}_dx"].astype(np.float64)
    # fp32 gradients: dx elementwise 1e-4 relative + 1e-5 * max|dx|; column sums 1e-4 max-norm.
    assert (np.abs(to_np(dx) - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max()).all()
    assert_close_rel(to_np(dg), gold[f"gb_{mode}_dg"], 1e-4, "dgamma")
    assert_close_rel(to_np(db), gold[f"gb_{mode}_db"], 1e-4, "dbeta")
