"""GPU parity of the HIP kernels, called through the C ABI (libfln.so via ctypes).

Every check compares against the CPU oracle (oracle/norms.py in numpy fp64, oracle/fln_oracle.c
for the full benchmark sizes) on the same seeded inputs (fused_layernorm.testing).  Tolerances
(those of the benchmark contract):
  * fp32 outputs: max-abs <= 1e-5;
  * bf16 outputs (y, h): within 1 bf16 ulp of the fp64 reference; h = x + r is bit-exact.
    For LayerNorm with a bias, y = xhat*gamma + beta can cancel to ~1e-7 while its terms are
    ~1e-2; there the fp32 rounding of the affine step (a few fp32 ulps of |xhat gamma| + |beta|)
    and the fp32 row mean's shift of xhat are allowed on top: bound = 1 ulp_bf16(ref) +
    oracle.tolerance.y_allowance (which torch's own fp32 layer_norm needs as well);
  * dx (every dtype): within 1 ulp of the output type + an elementwise fp32 evaluation
    allowance (oracle.tolerance.dx_allowance: dx = rstd (g - c1 - xhat c2) cancels, so an element
    near zero carries a few fp32 roundings of the terms g, c1, xhat c2 and of the row sums,
    2^-20 .. 2^-21 log2 N of their magnitudes -- not a fraction of max|dx|);
  * dgamma / dbeta / dweight (fp32 column sums): max|err| <= 1e-4 * max|ref|;
  * fp8 codes: identical except +-1 code on <= 0.1% of elements; per-row scales within 1e-6
    relative.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import capi
from gpu_calls import cuda, f32, ln_backward, ln_forward, rms_backward, rms_forward, workspace
from helpers import (assert_close_rel, assert_dx, assert_fp8_close, assert_mx_close,
                     assert_within_ulp, to_np)
from oracle import c_oracle, norms, tolerance
from fused_layernorm.testing import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def lib(gpu_available):
    return capi.load()


# ------------------------------------------------------------------------------------------------
# Benchmark configurations C1..C5 and the 8192 x 4096 headline.
# ------------------------------------------------------------------------------------------------
def test_library_exports_every_declared_symbol(lib):
    for name in capi.declared_functions():
        assert hasattr(lib, name), name


def test_c1_layernorm_fp32_32x768(lib):
    w = WORKLOADS["c1_ln_fwd_fp32_32x768"]
    inp = make_inputs(w)
    x, g, b = (cuda(inp[k]) for k in ("x", "gamma", "beta"))
    y = torch.empty_like(x)
    capi.check(lib.fln_layernorm(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y), 32, 768,
                                 capi.F32, w.eps, capi.stream()))
    ref, _, _ = norms.layer_norm_fwd(to_np(inp["x"]), to_np(inp["gamma"]), to_np(inp["beta"]),
                                     w.eps)
    assert np.abs(to_np(y) - ref).max() <= 1e-5
    ref_t = torch.nn.functional.layer_norm(inp["x"], (768,), inp["gamma"], inp["beta"], w.eps)
    assert (y.cpu() - ref_t).abs().max().item() <= 1e-5


@pytest.mark.parametrize("name", ["c2_ln_gelu_fp32_17x1023", "c2_ln_gelu_fp32_64x4096"])
@pytest.mark.parametrize("mode", ["none", "tanh"])
def test_c2_layernorm_gelu_fp32(lib, name, mode):
    w = WORKLOADS[name]
    inp = make_inputs(w)
    x, g, b = (cuda(inp[k]) for k in ("x", "gamma", "beta"))
    y = torch.empty_like(x)
    capi.check(lib.fln_layernorm_gelu(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y),
                                      w.rows, w.cols, capi.F32, w.eps,
                                      capi.GELU_ERF if mode == "none" else capi.GELU_TANH,
                                      capi.stream()))
    ref = norms.layer_norm_gelu_fwd(to_np(inp["x"]), to_np(inp["gamma"]), to_np(inp["beta"]),
                                    w.eps, mode)
    assert np.abs(to_np(y) - ref).max() <= 1e-5


@pytest.mark.parametrize("mode", ["none", "tanh"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("cols", [4096, 7168, 18432, 40960, 131072],
                         ids=["4096", "7168", "18432", "40960", "131072"])
def test_gelu_full_range_fwd_bwd(lib, monkeypatch, capfd, mode, dtype, cols):
    """LN + GELU forward and backward with the GELU input swept over [-13, 13] (beta a ramp) and a
    random dy: the GELU and GELU' tables (|a| < 6 interpolated, past 6 the constant last
    interval; the forward's log table out to 16) against the oracle at both signs and across
    every interval boundary, for both forms; 18432 columns take the 768-thread register backward
    with 3 vectors per lane (16-bit) and the two-pass one (fp32); 40960 and 131072 columns the
    LDS-staged forward (the 16-bit exact GELU from its LDS table; fp32 with half of each row
    in registers, from the polynomial, both forms), the 16-bit exact GELU at 131072 the
    streamed wide-row forward (table), and the two-pass backward.  48 rows would take the split
    forward: FLN_FWD_NO_SPLIT keeps them on the kernels named, and the dispatcher's trace must
    show the route fln_forward_plan reports."""
    rows = 48
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    expect = fl_functional().get_optimal_config(rows, cols, dtype, approximate=mode)["route"]
    assert expect != "split"
    assert expect == ("registers" if cols <= 16384 or (cols == 18432 and dtype != torch.float32)
                      else "lds+registers" if cols == 40960 and dtype == torch.float32
                      else "lds" if cols <= 65536 else "lds+registers"
                      if mode == "tanh" and dtype != torch.float32 else "wide"), expect
    gen = torch.Generator().manual_seed(977 + (mode == "tanh") + cols)
    xc = (torch.rand(rows, cols, generator=gen) * 2 - 1).to(dtype)
    gc = torch.ones(cols).to(dtype)
    bc = torch.linspace(-12.0, 12.0, cols).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy = cuda(xc), cuda(gc), cuda(bc), cuda(dyc)
    gm = capi.GELU_ERF if mode == "none" else capi.GELU_TANH
    code = capi.dtype_code(x)
    p = capi.ptr
    y = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    routes, _ = _traced_routes(capfd, monkeypatch, lambda: capi.check(
        lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows, cols,
                                       code, 1e-5, gm, capi.stream())))
    assert routes == [expect], routes
    dx = torch.empty_like(x)
    dg = torch.empty(cols, device="cuda")
    db = torch.empty(cols, device="cuda")
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b), p(dx),
                                               p(dg), p(db), rows, cols, code, capi.F32, gm,
                                               p(ws), n, capi.stream()))
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    y_ref = norms.layer_norm_gelu_fwd(xs, gs, bs, 1e-5, mode)
    dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, mode)
    al = tolerance.dx_allowance(xs, dys, gs, 1e-5, beta=bs, approximate=mode)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5
        assert_dx(to_np(dx), dx_ref, al, "f32", f"gelu {mode} f32 {cols} dx")
    else:
        kind = "bf16" if dtype == torch.bfloat16 else "f16"
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, 1e-5), kind=kind,
                          what="y")
        assert_dx(to_np(dx), dx_ref, al, kind, f"gelu {mode} {kind} {cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")


@pytest.mark.parametrize("cols", [4096, 12288], ids=["registers", "lds"])
def test_gelu_erf_tails_fp32(lib, cols):
    """The exact-erf GELU over a = LayerNorm(x) + beta spanning [-13.6, 13.6] (beta a ramp):
    within 1e-5 of the oracle everywhere, and within 1e-4 relative in the lower tail (GELU down
    to 1e-30), which a 0.5 a (1 + erf(a / sqrt 2)) evaluation loses to cancellation -- in fp32,
    and in float64 too past a = -6, so the tail reference is a Phi(a) with scipy's ndtr on the
    oracle's float64 a.  The derivative is checked through the backward with dy = 1 against
    the oracle."""
    from scipy.special import ndtr
    rows = 64
    gen = torch.Generator().manual_seed(cols)
    xc = torch.rand(rows, cols, generator=gen) * 2 - 1
    gc = torch.ones(cols)
    bc = torch.linspace(-12.0, 12.0, cols)
    x, g, b = cuda(xc), cuda(gc), cuda(bc)
    p = capi.ptr
    y = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                              cols, capi.F32, 1e-5, capi.GELU_ERF,
                                              capi.stream()))
    ref = norms.layer_norm_gelu_fwd(xc.numpy(), gc.numpy(), bc.numpy(), 1e-5, "none")
    got = to_np(y)
    assert np.abs(got - ref).max() <= 1e-5
    a64, _, _ = norms.layer_norm_fwd(xc.numpy(), gc.numpy(), bc.numpy(), 1e-5)
    exact = a64 * ndtr(a64)
    # The lower tail only: near a = 0 the relative error is that of a's own fp32 rounding.
    tail = (a64 < -3.0) & (np.abs(exact) > 1e-30)
    rel = np.abs(got[tail] - exact[tail]) / np.abs(exact[tail])
    assert rel.max() <= 1e-4, f"tail relative error {rel.max():.3g}"
    assert np.abs(exact[tail]).min() < 1e-29  # the tail is exercised
    dy = torch.ones_like(x)
    dx = torch.empty_like(x)
    dg = torch.empty(cols, device="cuda")
    db = torch.empty(cols, device="cuda")
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b), p(dx),
                                               p(dg), p(db), rows, cols, capi.F32, capi.F32,
                                               capi.GELU_ERF, p(ws), n, capi.stream()))
    dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(np.ones((rows, cols)), xc.numpy(),
                                                       gc.numpy(), bc.numpy(), 1e-5, "none")
    assert_dx(to_np(dx), dx_ref,
              tolerance.dx_allowance(xc.numpy(), np.ones((rows, cols)), gc.numpy(), 1e-5,
                                     beta=bc.numpy(), approximate="none"),
              "f32", f"erf tails {cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")


def test_c3_add_layernorm_bf16_8192x4096(lib):
    w = WORKLOADS["c3_add_ln_fwd_bf16_8192x4096"]
    inp = make_inputs(w)
    x, r, g, b = (cuda(inp[k]) for k in ("x", "residual", "gamma", "beta"))
    y, h = torch.empty_like(x), torch.empty_like(x)
    mean = torch.empty(w.rows, device="cuda")
    rstd = torch.empty(w.rows, device="cuda")
    capi.check(lib.fln_add_layernorm_forward(
        capi.ptr(x), capi.ptr(r), capi.ptr(g), capi.ptr(b), capi.ptr(h), capi.ptr(y),
        capi.ptr(mean), capi.ptr(rstd), w.rows, w.cols, capi.BF16, w.eps, capi.stream()))
    h_ref = (inp["x"] + inp["residual"])  # torch CPU bf16 add: fp32 sum rounded to bf16
    assert torch.equal(h.cpu(), h_ref), "h must be bit-exact"
    h_np = norms.round_to_bf16(to_np(inp["x"]) + to_np(inp["residual"]))
    assert np.array_equal(h_np, to_np(h_ref))
    y_ref, m_ref, r_ref = c_oracle.layernorm_fwd(h_np, f32(inp["gamma"]), f32(inp["beta"]), w.eps)
    assert_within_ulp(to_np(y), y_ref, 1.0,
                      atol=affine_atol(h_np, f32(inp["gamma"]), f32(inp["beta"]), w.eps),
                      what="c3 y")
    assert np.abs(to_np(mean) - m_ref).max() <= 1e-5 * max(1.0, np.abs(m_ref).max())
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5


def affine_atol(x, gamma, beta, eps, approximate=None):
    """Elementwise fp32 evaluation allowance of a LayerNorm output (see module doc): the affine
    step's roundings plus the fp32 row mean's shift of xhat (oracle.tolerance.y_allowance)."""
    return tolerance.y_allowance(x, gamma, beta, eps, approximate=approximate)


def _ln_fwd_bwd_check(lib, name, rows=None):
    w = WORKLOADS[name]
    inp = make_inputs(w, rows)
    x, g, b, dy = (cuda(inp[k]) for k in ("x", "gamma", "beta", "dy"))
    y, mean, rstd = ln_forward(lib, x, g, b, w.eps)
    dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
    xs, gs, bs, dys = f32(inp["x"]), f32(inp["gamma"]), f32(inp["beta"]), f32(inp["dy"])
    y_ref, m_ref, r_ref = c_oracle.layernorm_fwd(xs, gs, bs, w.eps)
    assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, w.eps),
                      what=f"{name} y")
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5
    dx_ref, dg_ref, db_ref = c_oracle.layernorm_bwd(dys, xs, gs, w.eps)
    assert_dx(to_np(dx), dx_ref, tolerance.dx_allowance(xs, dys, gs, w.eps), "bf16",
              f"{name} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, f"{name} dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, f"{name} dbeta")


def _rms_fwd_bwd_check(lib, name, rows=None):
    w = WORKLOADS[name]
    inp = make_inputs(w, rows)
    x, g, dy = (cuda(inp[k]) for k in ("x", "gamma", "dy"))
    y, rstd = rms_forward(lib, x, g, w.eps)
    dx, dw = rms_backward(lib, dy, x, rstd, g)
    xs, gs, dys = f32(inp["x"]), f32(inp["gamma"]), f32(inp["dy"])
    y_ref, r_ref = c_oracle.rmsnorm_fwd(xs, gs, w.eps)
    assert_within_ulp(to_np(y), y_ref, 1.0, what=f"{name} y")
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5
    dx_ref, dw_ref = c_oracle.rmsnorm_bwd(dys, xs, gs, w.eps)
    assert_dx(to_np(dx), dx_ref, tolerance.dx_allowance(xs, dys, gs, w.eps, rms=True), "bf16",
              f"{name} dx")
    assert_close_rel(to_np(dw), dw_ref, 1e-4, f"{name} dweight")


def test_headline_layernorm_fwd_bwd_bf16_8192x4096(lib):
    _ln_fwd_bwd_check(lib, "ln_fwd_bwd_bf16_8192x4096")


def test_headline_rmsnorm_fwd_bwd_bf16_8192x4096(lib):
    _rms_fwd_bwd_check(lib, "rms_fwd_bwd_bf16_8192x4096")


def test_c4_rmsnorm_fwd_bwd_bf16_16384x8192(lib):
    _rms_fwd_bwd_check(lib, "c4_rms_fwd_bwd_bf16_16384x8192")


def test_c5_layernorm_fp8_bf16_32768x7168(lib):
    w = WORKLOADS["c5_ln_fp8_bf16_32768x7168"]
    inp = make_inputs(w)
    x, g, b = (cuda(inp[k]) for k in ("x", "gamma", "beta"))
    q = torch.empty(x.shape, device="cuda", dtype=torch.uint8)
    scale = torch.empty(w.rows, device="cuda", dtype=torch.float32)
    capi.check(lib.fln_layernorm_fp8_forward(
        capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(q), capi.ptr(scale), None, None,
        w.rows, w.cols, capi.BF16, w.eps, capi.stream()))
    del x
    q_ref, s_ref = c_oracle.layernorm_fp8(f32(inp["x"]), f32(inp["gamma"]), f32(inp["beta"]),
                                          w.eps)
    assert_fp8_close(q.cpu().numpy(), to_np(scale), q_ref, s_ref, "c5")
    # The outlier channels must reach the top of the fp8 range in every row.
    assert (np.abs(norms.fp8_e4m3fn_decode(q_ref)).max(axis=1) == 448).all()


def test_tensors_past_2_to_the_31_elements(lib):
    """A bf16 batch of 266240 x 8192 (2.18e9 elements, 4.4 GB per tensor): row offsets past 2^31
    elements and 4 GiB.  LayerNorm forward + backward, RMSNorm forward and LayerNorm -> fp8 on
    the same x; rows on both sides of the 2^31-element boundary (and the first and last rows)
    against the oracle, every row's statistics and the column sums dgamma / dbeta (over all
    rows) against a float64 torch reduction of the same inputs."""
    rows, cols, eps = 266240, 8192, 1e-5
    if torch.cuda.mem_get_info()[0] < 40 * 2 ** 30:
        pytest.skip("needs 40 GiB of free device memory")
    gen = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn(rows, cols, device="cuda", generator=gen).to(torch.bfloat16)
    dy = torch.randn(rows, cols, device="cuda", generator=gen).to(torch.bfloat16)
    g = (1 + 0.1 * torch.randn(cols, device="cuda", generator=gen)).to(torch.bfloat16)
    b = (0.1 * torch.randn(cols, device="cuda", generator=gen)).to(torch.bfloat16)
    y, mean, rstd = ln_forward(lib, x, g, b, eps)
    dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
    torch.cuda.synchronize()
    boundary = (1 << 31) // cols
    sample = [0, 1, boundary - 2, boundary - 1, boundary, boundary + 1, rows - 2, rows - 1]
    xs, dys = f32(x[sample]), f32(dy[sample])
    gs, bs = f32(g), f32(b)
    y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, gs, bs, eps)
    assert_within_ulp(to_np(y[sample]), y_ref, 1.0, atol=affine_atol(xs, gs, bs, eps), what="y")
    dx_ref, _, _ = norms.layer_norm_bwd(dys, xs, gs, eps)
    assert_dx(to_np(dx[sample]), dx_ref, tolerance.dx_allowance(xs, dys, gs, eps), "bf16",
              "2^31 rows dx")
    del y, dx
    # Statistics of every row and the column sums, float64 in chunks of rows.
    dg_ref = torch.zeros(cols, device="cuda", dtype=torch.float64)
    db_ref = torch.zeros_like(dg_ref)
    m_err = r_err = 0.0
    for r0 in range(0, rows, 16384):
        xf = x[r0:r0 + 16384].double()
        mu = xf.mean(dim=1, keepdim=True)
        xf -= mu
        rs = torch.rsqrt(xf.square().mean(dim=1, keepdim=True) + eps)
        xf *= rs
        dyf = dy[r0:r0 + 16384].double()
        dg_ref += (dyf * xf).sum(dim=0)
        db_ref += dyf.sum(dim=0)
        m_err = max(m_err, (mean[r0:r0 + 16384].double() - mu[:, 0]).abs().max().item())
        r_err = max(r_err, (rstd[r0:r0 + 16384].double() / rs[:, 0] - 1).abs().max().item())
        del xf, dyf
    assert m_err <= 1e-6 and r_err <= 1e-5, (m_err, r_err)
    assert_close_rel(to_np(dg), to_np(dg_ref), 1e-4, "dgamma")
    assert_close_rel(to_np(db), to_np(db_ref), 1e-4, "dbeta")
    del dy
    y2, rstd2 = rms_forward(lib, x, g, 1e-6)
    y2_ref, _ = norms.rms_norm_fwd(xs, gs, 1e-6)
    assert_within_ulp(to_np(y2[sample]), y2_ref, 1.0, what="rms y")
    del y2
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    scale = torch.empty(rows, device="cuda", dtype=torch.float32)
    capi.check(lib.fln_layernorm_fp8_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(q),
                                             capi.ptr(scale), None, None, rows, cols,
                                             capi.BF16, eps, capi.stream()))
    q_ref, s_ref = norms.layer_norm_fp8_fwd(xs, gs, bs, eps)
    assert_fp8_close(q[sample].cpu().numpy(), to_np(scale[sample]), q_ref, s_ref, "fp8")


def test_fp8_rows_feed_a_rowwise_scaled_gemm(lib):
    """The step after the norm: LayerNorm -> fp8 codes [M, K] with one fp32 scale per row are
    exactly the A operand and row-wise A scale of an fp8 GEMM (torch._scaled_mm on hipBLASLt,
    weight quantized per output channel).  The GEMM output must match a float64 product of the
    decoded operands (the layout and scale convention y ~ decode(q) * scale), and stay within the
    fp8 quantization error of LayerNorm(x) @ W^T."""
    m, k, n, eps = 512, 4096, 1024, 1e-5
    gen = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
    g = (1 + 0.1 * torch.randn(k, device="cuda", generator=gen)).to(torch.bfloat16)
    b = (0.1 * torch.randn(k, device="cuda", generator=gen)).to(torch.bfloat16)
    w = (torch.randn(n, k, device="cuda", generator=gen) / 64).to(torch.bfloat16)
    q = torch.empty(m, k, device="cuda", dtype=torch.uint8)
    scale = torch.empty(m, device="cuda", dtype=torch.float32)
    capi.check(lib.fln_layernorm_fp8_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(q),
                                             capi.ptr(scale), None, None, m, k, capi.BF16, eps,
                                             capi.stream()))
    w_scale = (w.float().abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    wq = (w.float() / w_scale[:, None]).to(torch.float8_e4m3fn)
    try:
        out = torch._scaled_mm(q.view(torch.float8_e4m3fn), wq.t(), scale_a=scale.view(m, 1),
                               scale_b=w_scale.view(1, n), out_dtype=torch.bfloat16)
    except (RuntimeError, NotImplementedError) as e:  # row-wise scaling absent from this build
        pytest.skip(f"torch._scaled_mm with row-wise scales unavailable: {e}")
    torch.cuda.synchronize()
    a64 = norms.fp8_e4m3fn_decode(q.cpu().numpy()) * to_np(scale)[:, None]
    b64 = wq.float().cpu().numpy().astype(np.float64) * to_np(w_scale)[:, None]
    ref = a64 @ b64.T
    got = to_np(out)
    # One bf16 ulp of output rounding (its rounding mode is the library's) + fp32 accumulation.
    bound = 2.0 ** -7 * np.abs(ref) + 1e-5 * (np.abs(a64) @ np.abs(b64).T)
    assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()
    y64, _, _ = norms.layer_norm_fwd(f32(x), f32(g), f32(b), eps)
    exact = y64 @ f32(w).astype(np.float64).T
    # Both operands carry e4m3 rounding (3 mantissa bits): 3.5% of max|exact| in a CPU
    # emulation of these shapes.
    assert np.abs(got - exact).max() <= 0.08 * np.abs(exact).max()


def test_mxfp8_blocks_feed_a_block_scaled_gemm(lib):
    """LayerNorm -> MXFP8 (E4M3 codes [M, K], one E8M0 scale per 32 elements of a row in
    [M, K / 32]) is the A operand of an MX-scaled fp8 GEMM as produced: torch._scaled_mm on
    hipBLASLt with float8_e8m0fnu block scales, the weight quantized by the same block rule.
    The output must match a float64 product of the decoded blocks to one bf16 ulp (the GEMM's
    output rounding) plus fp32 accumulation, and LayerNorm(x) @ W^T to the fp8 quantization
    error."""
    m, k, n, eps = 256, 4096, 512, 1e-5
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
    g = (1 + 0.1 * torch.randn(k, device="cuda", generator=gen)).to(torch.bfloat16)
    b = (0.1 * torch.randn(k, device="cuda", generator=gen)).to(torch.bfloat16)
    w = (torch.randn(n, k, device="cuda", generator=gen) / 64).to(torch.bfloat16)
    q = torch.empty(m, k, device="cuda", dtype=torch.uint8)
    sa = torch.empty(m, k // 32, device="cuda", dtype=torch.uint8)
    capi.check(lib.fln_layernorm_mxfp8_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(q),
                                               capi.ptr(sa), None, None, m, k, capi.BF16, eps,
                                               capi.stream()))
    # The weight by the same block rule: 2^e, e = floor(log2 max|block|) - 8, codes saturated.
    wf = w.float().view(n, k // 32, 32)
    e = (torch.floor(torch.log2(wf.abs().amax(dim=2).clamp_min(2.0 ** -126))) - 8).clamp(-127, 127)
    wq = (wf * torch.exp2(-e)[:, :, None]).clamp(-448, 448).view(n, k).to(torch.float8_e4m3fn)
    sb = (e + 127).to(torch.uint8)
    try:
        out = torch._scaled_mm(q.view(torch.float8_e4m3fn), wq.t(),
                               scale_a=sa.view(torch.float8_e8m0fnu),
                               scale_b=sb.view(torch.float8_e8m0fnu), out_dtype=torch.bfloat16)
    except (RuntimeError, NotImplementedError) as ex:  # MX scaling absent from this build
        pytest.skip(f"torch._scaled_mm with E8M0 block scales unavailable: {ex}")
    torch.cuda.synchronize()
    a64 = (norms.fp8_e4m3fn_decode(q.cpu().numpy()).reshape(m, k // 32, 32)
           * np.exp2(sa.cpu().numpy().astype(np.float64) - 127)[:, :, None]).reshape(m, k)
    b64 = (wq.float().cpu().numpy().astype(np.float64).reshape(n, k // 32, 32)
           * np.exp2(sb.cpu().numpy().astype(np.float64) - 127)[:, :, None]).reshape(n, k)
    ref = a64 @ b64.T
    got = to_np(out)
    bound = 2.0 ** -7 * np.abs(ref) + 1e-5 * (np.abs(a64) @ np.abs(b64).T)
    assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()
    y64, _, _ = norms.layer_norm_fwd(f32(x), f32(g), f32(b), eps)
    exact = y64 @ f32(w).astype(np.float64).T
    assert np.abs(got - exact).max() <= 0.08 * np.abs(exact).max()


def test_fp8_encoder_bit_exact(lib):
    """The device conversion (v_cvt_pk_fp8_f32 after a +-448 clamp) against the oracle's
    format-level encoder, over every exponent of the e4m3fn range and beyond, all 8 mantissa
    codes, the midpoints between codes (ties to even) and +-1 float32 ulp around them."""
    vals = [0.0, -0.0, 448.0, -448.0, 449.0, 464.0, 480.0, 1e30, -1e30, 2.0 ** -9, 2.0 ** -10,
            3 * 2.0 ** -11, 2.0 ** -6, 2.0 ** -7 * 1.0625]
    for e in range(-12, 10):
        for m in range(16):  # codes and midpoints (m odd)
            v = (1.0 + m / 16.0) * 2.0 ** e
            for d in (-1, 0, 1):
                f = np.nextafter(np.float32(v), np.float32(np.inf if d > 0 else -np.inf)) \
                    if d else np.float32(v)
                vals += [float(f), -float(f)]
    rng = np.random.RandomState(0)
    vals += list(rng.randn(20000) * 50)
    a = np.asarray(vals, np.float32)
    xg = torch.from_numpy(a).cuda()
    qg = torch.empty(a.shape, dtype=torch.uint8, device="cuda")
    capi.check(lib.fln_fp8_e4m3fn_encode(capi.ptr(xg), capi.ptr(qg), a.size, capi.stream()))
    ref = norms.fp8_e4m3fn_encode(a.astype(np.float64))
    got = qg.cpu().numpy()
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(float(a[i]), hex(got[i]), hex(ref[i])) for i in bad[:10]]


# ------------------------------------------------------------------------------------------------
# Shapes, dtypes and paths beyond the benchmark configurations.
# ------------------------------------------------------------------------------------------------
EDGE_SHAPES = [(1, 1), (1, 17), (1000, 1), (1, 100000), (512, 512), (1, 32767), (1, 65536),
               (13, 13), (1, 4095), (1, 4097), (2, 16384), (32, 1)]


@pytest.mark.parametrize("rows,cols", EDGE_SHAPES)
def test_edge_shapes_fp32(lib, rows, cols):
    """The reference's edge list (tests/edge_cases.py:12-23, test_layernorm.py:340-358) with its
    tolerance allclose(rtol=1e-4, atol=1e-5) (edge_cases.py:37), against the oracle."""
    gen = torch.Generator().manual_seed(rows * 100003 + cols)
    xc = torch.randn(rows, cols, generator=gen)
    gc = 1 + 0.1 * torch.randn(cols, generator=gen)
    bc = 0.1 * torch.randn(cols, generator=gen)
    y, mean, rstd = ln_forward(lib, cuda(xc), cuda(gc), cuda(bc), 1e-5)
    ref, m_ref, r_ref = norms.layer_norm_fwd(xc.numpy(), gc.numpy(), bc.numpy(), 1e-5)
    np.testing.assert_allclose(to_np(y), ref, rtol=1e-4, atol=1e-5)
    if cols == 1:
        np.testing.assert_array_equal(to_np(y), np.broadcast_to(bc.numpy(), (rows, 1)))


DTYPES = [torch.float32, torch.bfloat16, torch.float16]
SHAPES = [(1, 768), (8, 768), (32, 1024), (64, 2048), (128, 4096), (3, 1023), (5, 5120),
          (4, 16384), (2, 32768), (33, 7168), (7, 96), (5, 12288), (300, 20480), (3, 40960),
          (2, 65536), (260, 36864)]


def _tol_fwd(dtype):
    return dict(kind="bf16" if dtype == torch.bfloat16 else "f16")


def _kind(dtype):
    return {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]


def fl_functional():
    import fused_layernorm
    return fused_layernorm.functional


def _traced_routes(capfd, monkeypatch, fn):
    """Runs fn() with the forward dispatcher's trace on (FLN_DEBUG_GEOMETRY) and returns the
    kernel route of each forward launch it made ("registers", "lds", "lds+registers", "wide",
    "split", "loop")."""
    import re
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    out = fn()
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    return re.findall(r"fln forward: .* -> (\S+) wpr=", capfd.readouterr().err), out


def _flavour_allowance(kind, xs, dys, gs, bs=None, drs=None):
    """dx allowance of a backward flavour: "ln", "rms", "ln_dres", "gelu_none", "gelu_tanh"."""
    if kind == "rms":
        return tolerance.dx_allowance(xs, dys, gs, 1e-6, rms=True)
    if kind.startswith("gelu"):
        return tolerance.dx_allowance(xs, dys, gs, 1e-5, beta=bs, approximate=kind[5:])
    return tolerance.dx_allowance(xs, dys, gs, 1e-5, dres=drs if kind == "ln_dres" else None)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_layernorm_fwd_bwd_matrix(lib, dtype, rows, cols):
    gen = torch.Generator().manual_seed(rows * 7919 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy = cuda(xc), cuda(gc), cuda(bc), cuda(dyc)
    y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    y_ref, _, _ = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
    dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
    al = tolerance.dx_allowance(xs, dys, gs, 1e-5)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, 1e-5),
                          **_tol_fwd(dtype), what="y")
    assert_dx(to_np(dx), dx_ref, al, _kind(dtype), f"ln matrix {_kind(dtype)} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_rmsnorm_fwd_bwd_matrix(lib, dtype, rows, cols):
    gen = torch.Generator().manual_seed(rows * 104729 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    wc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, wt, dy = cuda(xc), cuda(wc), cuda(dyc)
    y, rstd = rms_forward(lib, x, wt, 1e-6)
    dx, dw = rms_backward(lib, dy, x, rstd, wt)
    xs, ws, dys = f32(xc), f32(wc), f32(dyc)
    y_ref, _ = norms.rms_norm_fwd(xs, ws, 1e-6)
    dx_ref, dw_ref = norms.rms_norm_bwd(dys, xs, ws, 1e-6)
    al = tolerance.dx_allowance(xs, dys, ws, 1e-6, rms=True)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        assert_within_ulp(to_np(y), y_ref, 1.0, **_tol_fwd(dtype), what="y")
    assert_dx(to_np(dx), dx_ref, al, _kind(dtype), f"rms matrix {_kind(dtype)} {rows}x{cols} dx")
    assert_close_rel(to_np(dw), dw_ref, 1e-4, "dweight")


def test_unaligned_rows_take_scalar_path(lib):
    """Input offset by one element (not 16-byte aligned): the scalar path must agree."""
    gen = torch.Generator().manual_seed(11)
    base = torch.randn(64 * 1024 + 1, generator=gen).to(torch.bfloat16).cuda()
    x = base[1:].view(64, 1024)
    gc = (1 + 0.1 * torch.randn(1024, generator=gen)).to(torch.bfloat16)
    bc = (0.1 * torch.randn(1024, generator=gen)).to(torch.bfloat16)
    y, mean, rstd = ln_forward(lib, x, cuda(gc), cuda(bc), 1e-5)
    xs = f32(x.cpu())
    ref, _, _ = norms.layer_norm_fwd(xs, f32(gc), f32(bc), 1e-5)
    assert_within_ulp(to_np(y), ref, 1.0, atol=affine_atol(xs, f32(gc), f32(bc), 1e-5),
                      what="unaligned y")


def test_output_canaries_untouched(lib):
    """Outputs carved out of larger buffers: the guard bytes after them must survive."""
    rows, cols, pad = 37, 1000, 4096
    gen = torch.Generator().manual_seed(5)
    xc = torch.randn(rows, cols, generator=gen).to(torch.bfloat16)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16)
    x, g, b = cuda(xc), cuda(gc), cuda(gc * 0.1)
    ybuf = torch.full((rows * cols + pad,), 7.0, device="cuda", dtype=torch.bfloat16)
    y = ybuf[: rows * cols].view(rows, cols)
    mbuf = torch.full((rows + pad,), 7.0, device="cuda")
    capi.check(lib.fln_layernorm_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y),
                                         capi.ptr(mbuf), None, rows, cols, capi.BF16, 1e-5,
                                         capi.stream()))
    dxbuf = torch.full((rows * cols + pad,), 7.0, device="cuda", dtype=torch.bfloat16)
    dgbuf = torch.full((cols + pad,), 7.0, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    ln_forward(lib, x, g, b, 1e-5)
    _, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_backward(
        capi.ptr(x), capi.ptr(x), capi.ptr(mean), capi.ptr(rstd), capi.ptr(g), None,
        capi.ptr(dxbuf), capi.ptr(dgbuf), None, rows, cols, capi.BF16, capi.F32, capi.ptr(ws), n,
        capi.stream()))
    torch.cuda.synchronize()
    assert (ybuf[rows * cols:] == 7).all()
    assert (mbuf[rows:] == 7).all()
    assert (dxbuf[rows * cols:] == 7).all()
    assert (dgbuf[cols:] == 7).all()


def test_backward_is_deterministic(lib):
    w = WORKLOADS["ln_fwd_bwd_bf16_8192x4096"]
    inp = make_inputs(w, 2048)
    x, g, b, dy = (cuda(inp[k]) for k in ("x", "gamma", "beta", "dy"))
    _, mean, rstd = ln_forward(lib, x, g, b, w.eps)
    first = ln_backward(lib, dy, x, mean, rstd, g)
    for _ in range(3):
        again = ln_backward(lib, dy, x, mean, rstd, g)
        for a, c in zip(first, again):
            assert torch.equal(a, c)


@pytest.mark.parametrize("dtype,rows,cols", [
    (torch.bfloat16, 1000, 4096), (torch.float16, 333, 1023), (torch.bfloat16, 3, 7168),
    (torch.float16, 4096, 768)])
def test_parameter_gradients_in_parameter_dtype(lib, dtype, rows, cols):
    """dgamma / dbeta written as bf16 / f16 (the fp32 column sums rounded once on store): each
    element within half an ulp of the parameter type, plus the fp32 reduction tolerance."""
    gen = torch.Generator().manual_seed(rows * 31 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, dy = cuda(xc), cuda(gc), cuda(dyc)
    _, mean, rstd = ln_forward(lib, x, g, g, 1e-5)
    _, dg, db = ln_backward(lib, dy, x, mean, rstd, g, dparam_f32=False)
    assert dg.dtype == dtype and db.dtype == dtype
    _, dg_ref, db_ref = norms.layer_norm_bwd(f32(dyc), f32(xc), f32(gc), 1e-5)
    kind = "bf16" if dtype == torch.bfloat16 else "f16"
    for got, ref, what in ((dg, dg_ref, "dgamma"), (db, db_ref, "dbeta")):
        assert_within_ulp(to_np(got), ref, 0.5, atol=1e-4 * np.abs(ref).max(), kind=kind,
                          what=what)


def test_c6_add_rmsnorm_fp8_bf16_32768x7168(lib):
    """Residual add + RMSNorm -> fp8 at C5's shape: h bit-exact, codes and scales to the fp8
    bar against the C oracle (RMSNorm -> fp8 of the bf16-rounded h)."""
    w = WORKLOADS["c6_add_rms_fp8_bf16_32768x7168"]
    inp = make_inputs(w)
    x, r, g = (cuda(inp[k]) for k in ("x", "residual", "gamma"))
    h = torch.empty_like(x)
    q = torch.empty(x.shape, device="cuda", dtype=torch.uint8)
    scale = torch.empty(w.rows, device="cuda", dtype=torch.float32)
    capi.check(lib.fln_add_rmsnorm_fp8_forward(
        capi.ptr(x), capi.ptr(r), capi.ptr(g), capi.ptr(h), capi.ptr(q), capi.ptr(scale), None,
        w.rows, w.cols, capi.BF16, w.eps, capi.stream()))
    del x, r
    h_ref = inp["x"] + inp["residual"]  # torch CPU bf16 add
    assert torch.equal(h.cpu(), h_ref), "h must be bit-exact"
    q_ref, s_ref = c_oracle.rmsnorm_fp8(f32(h_ref), f32(inp["gamma"]), w.eps)
    assert_fp8_close(q.cpu().numpy(), to_np(scale), q_ref, s_ref, "c6")


def _scaled(y):
    """Unquantized fp8 values of the row rule: y / (max|y| / 448) per row."""
    amax = np.abs(y).max(axis=-1, keepdims=True)
    return np.where(amax > 0, y * 448.0 / np.where(amax > 0, amax, 1.0), 0.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(64, 4096), (7, 1023), (33, 7168), (2, 16384),
                                       (3, 12288), (2, 32768), (300, 24576), (2, 40960),
                                       (300, 65536)])
def test_fp8_variants_dtype_shape_matrix(lib, dtype, rows, cols):
    """LayerNorm -> fp8, RMSNorm -> fp8, residual + LayerNorm -> fp8, residual + RMSNorm -> fp8
    over dtypes and widths (1023: the scalar path; 12288..32768: 12-16 waves and the RAW tiles,
    300 x 24576: several rows per block through their prefetch ring; 40960 / 65536: the
    LDS-staged kernel), against the oracle."""
    gen = torch.Generator().manual_seed(rows * 31 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    kind = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    code = capi.dtype_code(x)
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    s = torch.empty(rows, device="cuda")
    h = torch.empty_like(x)
    p = capi.ptr
    capi.check(lib.fln_rmsnorm_fp8_forward(p(x), p(g), p(q), p(s), None, rows, cols, code, 1e-6,
                                           capi.stream()))
    q_ref, s_ref = norms.rms_norm_fp8_fwd(f32(xc), f32(gc), 1e-6)
    assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "rms fp8",
                     t_ref=_scaled(norms.rms_norm_fwd(f32(xc), f32(gc), 1e-6)[0]))
    capi.check(lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(s), None, None, rows,
                                             cols, code, 1e-5, capi.stream()))
    q_ref, s_ref = norms.layer_norm_fp8_fwd(f32(xc), f32(gc), f32(bc), 1e-5)
    assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "ln fp8",
                     t_ref=_scaled(norms.layer_norm_fwd(f32(xc), f32(gc), f32(bc), 1e-5)[0]))
    h_ref = to_np(xc + rc)  # torch CPU add in the I/O type
    capi.check(lib.fln_add_layernorm_fp8_forward(p(x), p(r), p(g), p(b), p(h), p(q), p(s), None,
                                                 None, rows, cols, code, 1e-5, capi.stream()))
    assert np.array_equal(to_np(h), h_ref), "h bit-exact"
    q_ref, s_ref, _ = norms.add_layer_norm_fp8_fwd(f32(xc), f32(rc), f32(gc), f32(bc), 1e-5,
                                                   kind)
    assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "add ln fp8")
    h.zero_()
    capi.check(lib.fln_add_rmsnorm_fp8_forward(p(x), p(r), p(g), p(h), p(q), p(s), None, rows,
                                               cols, code, 1e-6, capi.stream()))
    assert np.array_equal(to_np(h), h_ref), "h bit-exact"
    q_ref, s_ref, h_o = norms.add_rms_norm_fp8_fwd(f32(xc), f32(rc), f32(gc), 1e-6, kind)
    assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "add rms fp8",
                     t_ref=_scaled(norms.rms_norm_fwd(h_o, f32(gc), 1e-6)[0]))


ODD_TILES = [  # op, dtype, rows, cols, (waves per row, vectors per lane, threads)
    ("ln", torch.bfloat16, 1024, 1536, (1, 3, 256)), ("rms", torch.float16, 1024, 2560, (1, 5, 256)),
    ("ln", torch.bfloat16, 512, 3072, (2, 3, 256)), ("ln", torch.bfloat16, 1024, 3584, (1, 7, 256)),
    ("rms", torch.float16, 1100, 3584, (1, 7, 256)), ("rms", torch.bfloat16, 342, 4608, (3, 3, 192)),
    ("ln", torch.float16, 512, 5120, (2, 5, 256)), ("ln", torch.bfloat16, 256, 6144, (4, 3, 256)),
    ("ln_fp8", torch.bfloat16, 1024, 2560, (1, 5, 256)),
    ("ln_fp8", torch.bfloat16, 1024, 3072, (1, 6, 256)),
    ("rms_fp8", torch.bfloat16, 342, 4608, (3, 3, 192)),
    ("rms_fp8", torch.float16, 512, 6144, (2, 6, 256)),
    ("ln_fp8", torch.bfloat16, 600, 7168, (2, 7, 256)),
    ("rms_fp8", torch.float16, 512, 7168, (2, 7, 256)),
    ("ln_fp8", torch.bfloat16, 256, 10240, (4, 5, 256)),
    ("gelu_tanh", torch.bfloat16, 1024, 2560, (1, 5, 256)),
    ("gelu_none", torch.float16, 1024, 3072, (1, 6, 256)),
    ("gelu_tanh", torch.bfloat16, 342, 4608, (3, 3, 192)),
    ("gelu_none", torch.bfloat16, 512, 7168, (2, 7, 256)),
    ("gelu_tanh", torch.float16, 256, 6144, (4, 3, 256)),
    ("add_ln", torch.bfloat16, 1024, 1536, (1, 3, 256)),
    ("add_ln", torch.float16, 342, 4608, (3, 3, 192)),
    ("add_rms_fp8", torch.bfloat16, 1024, 2560, (1, 5, 256)),
    ("add_rms_fp8", torch.float16, 512, 5120, (2, 5, 256)),
    ("add_rms_mx", torch.bfloat16, 512, 3072, (2, 3, 256)),
    ("add_rms_mx", torch.bfloat16, 256, 6144, (4, 3, 256)),
    # rows that leave the last block part-empty (4 / 2 row groups per 256-thread block)
    ("ln", torch.bfloat16, 1027, 2560, (1, 5, 256)),
    ("rms_fp8", torch.float16, 1026, 3072, (1, 6, 256)),
    ("gelu_none", torch.bfloat16, 513, 5120, (2, 5, 256))]


@pytest.mark.parametrize("op,dtype,rows,cols,tile", ODD_TILES,
                         ids=[f"{o}-{str(d)[6:]}-{r}x{c}" for o, d, r, c, _ in ODD_TILES])
def test_odd_vector_tiles(lib, capfd, monkeypatch, op, dtype, rows, cols, tile):
    """The exact register tilings of 3, 5, 6 or 7 vectors per lane (16-bit LayerNorm / RMSNorm
    and the fp8 row scale, blocks of at most 256 threads), with rows enough to fill the device:
    the dispatcher's trace must show the tiling fln_forward_plan reports, and the outputs must
    meet the oracle's bar."""
    import re
    w_exp, v_exp, t_exp = tile
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if rows * w_exp < 4 * cus:
        pytest.skip(f"{cus} CUs: the tiling needs more rows to be planned")
    form = op[5:] if op.startswith("gelu") else None
    fp8 = 1 if op.endswith("fp8") else 2 if op.endswith("mx") else 0
    plan = fl_functional().get_optimal_config(rows, cols, dtype, fp8=fp8, approximate=form,
                                              residual=op.startswith("add"))
    assert (plan["waves_per_row"], plan["vectors_per_lane"], plan["exact_tiling"],
            plan["threads_per_block"]) == (w_exp, v_exp, True, t_exp), plan
    gen = torch.Generator().manual_seed(rows + cols)
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, g, b = cuda(xc), cuda(gc), cuda(bc)
    xs, gs, bs = f32(xc), f32(gc), f32(bc)
    kind = "bf16" if dtype == torch.bfloat16 else "f16"
    code = capi.dtype_code(x)
    p = capi.ptr
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if op == "ln":
        y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    elif op == "rms":
        y, rstd = rms_forward(lib, x, g, 1e-6)
    elif op.startswith("add"):
        rc = torch.randn(rows, cols, generator=gen).to(dtype)
        r = cuda(rc)
        h = torch.empty_like(x)
        if op == "add_ln":
            y = torch.empty_like(x)
            mean = torch.empty(rows, device="cuda")
            rstd = torch.empty(rows, device="cuda")
            capi.check(lib.fln_add_layernorm_forward(p(x), p(r), p(g), p(b), p(h), p(y), p(mean),
                                                     p(rstd), rows, cols, code, 1e-5,
                                                     capi.stream()))
        elif op == "add_rms_fp8":
            q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
            s = torch.empty(rows, device="cuda")
            capi.check(lib.fln_add_rmsnorm_fp8_forward(p(x), p(r), p(g), p(h), p(q), p(s), None,
                                                       rows, cols, code, 1e-6, capi.stream()))
        else:
            q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
            sc = torch.empty(rows, cols // 32, device="cuda", dtype=torch.uint8)
            capi.check(lib.fln_add_rmsnorm_mxfp8_forward(p(x), p(r), p(g), p(h), p(q), p(sc),
                                                         None, rows, cols, code, 1e-6,
                                                         capi.stream()))
    elif form is not None:
        y = torch.empty_like(x)
        capi.check(lib.fln_layernorm_gelu(p(x), p(g), p(b), p(y), rows, cols, code, 1e-5,
                                          capi.GELU_TANH if form == "tanh" else capi.GELU_ERF,
                                          capi.stream()))
    else:
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        s = torch.empty(rows, device="cuda")
        if op == "ln_fp8":
            capi.check(lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(s), None, None,
                                                     rows, cols, code, 1e-5, capi.stream()))
        else:
            capi.check(lib.fln_rmsnorm_fp8_forward(p(x), p(g), p(q), p(s), None, rows, cols,
                                                   code, 1e-6, capi.stream()))
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"-> (\S+) wpr=(\d+) vpl=(\d+) exact=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    assert trace == [("registers", str(w_exp), str(v_exp), "1", str(t_exp))], trace
    if op == "ln":
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, 1e-5), kind=kind,
                          what="y")
        assert np.abs(to_np(mean) - m_ref).max() <= 1e-5 * np.abs(xs).max()
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5
    elif op == "rms":
        y_ref, r_ref = norms.rms_norm_fwd(xs, gs, 1e-6)
        assert_within_ulp(to_np(y), y_ref, 1.0, kind=kind, what="y")
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5
    elif op.startswith("add"):
        rs = f32(rc)
        assert np.array_equal(to_np(h), to_np(xc + rc)), "h bit-exact"
        if op == "add_ln":
            y_ref, h_ref, m_ref, r_ref = norms.add_layer_norm_fwd(xs, rs, gs, bs, 1e-5, kind)
            assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(h_ref, gs, bs, 1e-5),
                              kind=kind, what="add ln y")
            assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5
        elif op == "add_rms_fp8":
            q_ref, s_ref, h_o = norms.add_rms_norm_fp8_fwd(xs, rs, gs, 1e-6, kind)
            assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "add rms fp8",
                             t_ref=_scaled(norms.rms_norm_fwd(h_o, gs, 1e-6)[0]))
        else:
            q_ref, sc_ref, y_ref = _mx_ref("add_rms", xs, rs, gs, bs, kind)
            assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, sc_ref, y_ref, "mx add_rms")
    elif form is not None:
        y_ref = norms.layer_norm_gelu_fwd(xs, gs, bs, 1e-5, form)
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, 1e-5), kind=kind,
                          what="gelu y")
    elif op == "ln_fp8":
        q_ref, s_ref = c_oracle.layernorm_fp8(xs, gs, bs, 1e-5)
        assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "ln fp8",
                         t_ref=_scaled(norms.layer_norm_fwd(xs, gs, bs, 1e-5)[0]))
    else:
        q_ref, s_ref = c_oracle.rmsnorm_fp8(xs, gs, 1e-6)
        assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, "rms fp8",
                         t_ref=_scaled(norms.rms_norm_fwd(xs, gs, 1e-6)[0]))


@pytest.mark.parametrize("rms", [False, True], ids=["ln", "rms"])
@pytest.mark.parametrize("rows", [512, 1024, 1500])
def test_fp32_8192_wide_row_groups(lib, capfd, monkeypatch, rms, rows):
    """fp32 rows of 8192 columns with 2-8 rows per CU take 16 waves x 2 vectors per lane in a
    1024-thread block: the trace must show it and the outputs must match the oracle (1500 rows
    leave the grid's last round part-empty)."""
    import re
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if not 2 * cus <= rows <= 8 * cus:
        pytest.skip(f"{cus} CUs: {rows} rows are outside the planned range")
    cols = 8192
    gen = torch.Generator().manual_seed(rows * 3 + rms)
    xc = torch.randn(rows, cols, generator=gen) * 3 + 1
    gc = 1 + 0.1 * torch.randn(cols, generator=gen)
    bc = 0.1 * torch.randn(cols, generator=gen)
    x, g, b = cuda(xc), cuda(gc), cuda(bc)
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if rms:
        y, rstd = rms_forward(lib, x, g, 1e-6)
    else:
        y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"-> (\S+) wpr=(\d+) vpl=(\d+) exact=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    assert trace == [("registers", "16", "2", "1", "1024")], trace
    xs, gs, bs = f32(xc), f32(gc), f32(bc)
    if rms:
        y_ref, r_ref = norms.rms_norm_fwd(xs, gs, 1e-6)
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1.0, np.abs(y_ref).max())
    else:
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1.0, np.abs(y_ref).max())
        assert np.abs(to_np(mean) - m_ref).max() <= 1e-6 * np.abs(xs).max()
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5


FP32_HALVED = [(4096, 2048, (2, 4, 256)), (2048, 4096, (4, 4, 256)), (3001, 4096, (4, 4, 256)),
               (2048, 6144, (6, 4, 384)), (2500, 6144, (6, 4, 384)), (16384, 8192, (8, 4, 512))]


@pytest.mark.parametrize("rms", [False, True], ids=["ln", "rms"])
@pytest.mark.parametrize("rows,cols,tile", FP32_HALVED,
                         ids=[f"{r}x{c}" for r, c, _ in FP32_HALVED])
def test_fp32_halved_vector_tiles(lib, capfd, monkeypatch, rms, rows, cols, tile):
    """fp32 LayerNorm / RMSNorm rows that would take 8 vectors per lane over 1-4 waves, with
    rows enough for 32 waves per CU, take twice the waves at 4 vectors per lane (6 and 8 waves
    in the 1024-thread instantiation; 3001 and 2500 rows leave the last round part-empty): the
    trace must show the tiling fln_forward_plan reports, and the outputs must match the oracle
    (the C oracle: up to 134 M elements)."""
    import re
    w, v, t = tile
    plan = fl_functional().get_optimal_config(rows, cols, torch.float32)
    if (plan["waves_per_row"], plan["vectors_per_lane"]) != (w, v):
        assert torch.cuda.get_device_properties(0).multi_processor_count != 256, plan
        pytest.skip("the tiling is planned for another CU count")
    gen = torch.Generator().manual_seed(rows * 5 + cols + rms)
    xc = torch.randn(rows, cols, generator=gen) * 2 - 0.5
    gc = 1 + 0.1 * torch.randn(cols, generator=gen)
    bc = 0.1 * torch.randn(cols, generator=gen)
    x, g, b = cuda(xc), cuda(gc), cuda(bc)
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if rms:
        y, rstd = rms_forward(lib, x, g, 1e-6)
    else:
        y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"-> (\S+) wpr=(\d+) vpl=(\d+) exact=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    assert trace == [("registers", str(w), str(v), "1", str(t))], trace
    xs, gs, bs = f32(xc), f32(gc), f32(bc)
    if rms:
        y_ref, r_ref = c_oracle.rmsnorm_fwd(xs, gs, 1e-6)
    else:
        y_ref, m_ref, r_ref = c_oracle.layernorm_fwd(xs, gs, bs, 1e-5)
        assert np.abs(to_np(mean) - m_ref).max() <= 1e-6 * np.abs(xs).max()
    assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1.0, np.abs(y_ref).max())
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5


FP32_HALVED_FLAVOURS = [("add_ln", 8192, 4096, (4, 4, 256)), ("add_ln", 16384, 2048, (2, 4, 256)),
                        ("add_ln", 9001, 4096, (4, 4, 256)),
                        ("gelu_tanh", 2048, 4096, (4, 4, 256)),
                        ("gelu_none", 3001, 4096, (4, 4, 256)),
                        ("gelu_tanh", 2048, 6144, (6, 4, 384)),
                        ("gelu_none", 8192, 8192, (8, 4, 512))]


@pytest.mark.parametrize("kind,rows,cols,tile", FP32_HALVED_FLAVOURS,
                         ids=[f"{k}-{r}x{c}" for k, r, c, _ in FP32_HALVED_FLAVOURS])
def test_fp32_halved_vector_tiles_residual_and_gelu(lib, capfd, monkeypatch, kind, rows, cols,
                                                     tile):
    """The halved fp32 tiles (twice the waves at 4 vectors per lane) in the residual + LayerNorm
    and LN + GELU flavours: the trace must show the tiling fln_forward_plan reports; h must be
    bit-exact and y must match the oracle (max-abs 1e-5 of max(1, |y|))."""
    import re
    w, v, t = tile
    form = kind[5:] if kind.startswith("gelu") else None
    plan = fl_functional().get_optimal_config(rows, cols, torch.float32, approximate=form,
                                              residual=kind == "add_ln")
    if (plan["waves_per_row"], plan["vectors_per_lane"]) != (w, v):
        assert torch.cuda.get_device_properties(0).multi_processor_count != 256, plan
        pytest.skip("the tiling is planned for another CU count")
    gen = torch.Generator().manual_seed(rows * 7 + cols)
    xc = torch.randn(rows, cols, generator=gen) * 1.5 + 0.25
    rc = torch.randn(rows, cols, generator=gen)
    gc = 1 + 0.1 * torch.randn(cols, generator=gen)
    bc = 0.1 * torch.randn(cols, generator=gen)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    p = capi.ptr
    y = torch.empty_like(x)
    h = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if kind == "add_ln":
        capi.check(lib.fln_add_layernorm_forward(p(x), p(r), p(g), p(b), p(h), p(y), p(mean),
                                                 p(rstd), rows, cols, capi.F32, 1e-5,
                                                 capi.stream()))
    else:
        capi.check(lib.fln_layernorm_gelu_forward(
            p(x), p(g), p(b), p(y), p(mean), p(rstd), rows, cols, capi.F32, 1e-5,
            capi.GELU_TANH if form == "tanh" else capi.GELU_ERF, capi.stream()))
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"-> (\S+) wpr=(\d+) vpl=(\d+) exact=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    assert trace == [("registers", str(w), str(v), "1", str(t))], trace
    xs, rs, gs, bs = f32(xc), f32(rc), f32(gc), f32(bc)
    if kind == "add_ln":
        assert torch.equal(h.cpu(), xc + rc), "h bit-exact"
        y_ref, _, _, r_ref = norms.add_layer_norm_fwd(xs, rs, gs, bs, 1e-5, "f32")
    else:
        y_ref = norms.layer_norm_gelu_fwd(xs, gs, bs, 1e-5, form)
        _, _, r_ref = norms.layer_norm_fwd(xs, None, None, 1e-5)
    assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1.0, np.abs(y_ref).max())
    assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5


BWD_EXACT_GROUPS = [("ln", torch.bfloat16, 4608), ("rms", torch.bfloat16, 5120),
                    ("ln_dres", torch.float16, 5632), ("gelu_tanh", torch.bfloat16, 6144),
                    ("gelu_none", torch.float16, 4608), ("ln", torch.float16, 6144)]


@pytest.mark.parametrize("kind,dtype,cols", BWD_EXACT_GROUPS,
                         ids=[f"{k}-{str(d)[6:]}-{c}" for k, d, c in BWD_EXACT_GROUPS])
@pytest.mark.parametrize("rows", [300, 2048])
def test_backward_exact_row_groups(lib, capfd, monkeypatch, kind, dtype, rows, cols):
    """16-bit backward rows of 9-12 whole waves of vectors (4608-6144 columns) take a row group
    of exactly cols / 512 waves (one per block) instead of 16: the backward's trace must show it,
    and dx, dgamma, dbeta must meet the oracle's bar for every flavour."""
    import re
    gen = torch.Generator().manual_seed(rows + 3 * cols)
    xc = (torch.randn(rows, cols, generator=gen) + 0.3).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = torch.linspace(-3.0, 3.0, cols).to(dtype)
    x, dy, dr, g, b = cuda(xc), cuda(dyc), cuda(drc), cuda(gc), cuda(bc)
    xs, dys, drs, gs, bs = f32(xc), f32(dyc), f32(drc), f32(gc), f32(bc)
    p = capi.ptr
    code = capi.dtype_code(x)
    eps = 1e-6 if kind == "rms" else 1e-5
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, eps)
    elif kind.startswith("gelu"):
        gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
        y = torch.empty_like(x)
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                                  cols, code, eps, gm, capi.stream()))
    else:
        _, mean, rstd = ln_forward(lib, x, g, b, eps)
    torch.cuda.synchronize()
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if kind == "rms":
        dx, dg = rms_backward(lib, dy, x, rstd, g)
        db = None
    elif kind.startswith("gelu"):
        dx = torch.empty_like(x)
        dg = torch.empty(cols, device="cuda")
        db = torch.empty(cols, device="cuda")
        ws, n = workspace(lib, rows, cols, x)
        capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                   p(dx), p(dg), p(db), rows, cols, code,
                                                   capi.F32, gm, p(ws), n, capi.stream()))
    else:
        dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g,
                                 dres=dr if kind == "ln_dres" else None)
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"fln backward: .* -> (\S+) wpr=(\d+) vpl=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    w = cols // 512
    assert trace == [("registers", str(w), "1", str(64 * w))], trace
    if kind == "rms":
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, eps)
        db_ref = None
    elif kind.startswith("gelu"):
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, eps, kind[5:])
    else:
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, eps)
        if kind == "ln_dres":
            dx_ref = dx_ref + drs
    k = "bf16" if dtype == torch.bfloat16 else "f16"
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs, bs, drs), k,
              f"{kind} {cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db_ref is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")


BWD_TWO_VECTORS = [("ln", torch.bfloat16, 4096, 768, (1, 2)),
                   ("rms", torch.float16, 4096, 1536, (2, 2)),
                   ("ln", torch.bfloat16, 8193, 1280, (2, 2)),
                   ("rms", torch.bfloat16, 4100, 2560, (4, 2)),
                   ("ln", torch.float16, 4096, 7168, (8, 2)),
                   ("ln", torch.bfloat16, 4096, 1024, (2, 1)),
                   ("ln", torch.bfloat16, 1000, 768, (2, 1))]


@pytest.mark.parametrize("kind,dtype,rows,cols,tile", BWD_TWO_VECTORS,
                         ids=[f"{k}-{str(d)[6:]}-{r}x{c}" for k, d, r, c, _ in BWD_TWO_VECTORS])
def test_backward_two_vectors_on_masked_widths(lib, capfd, monkeypatch, kind, dtype, rows, cols,
                                               tile):
    """16-bit LayerNorm / RMSNorm backwards whose one-vector tile would leave lanes masked take 2
    vectors per lane over half the waves once there are 16 rows per CU; whole power-of-two
    tiles (1024 columns) and fewer rows (1000) keep one vector: the backward's trace must show
    the tiling, and dx, dgamma, dbeta must meet the oracle's bar."""
    import re
    w, v = tile
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"{cus} CUs: the row thresholds are for 256")
    gen = torch.Generator().manual_seed(rows + 11 * cols)
    xc = (torch.randn(rows, cols, generator=gen) + 0.2).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, dy, g, b = cuda(xc), cuda(dyc), cuda(gc), cuda(bc)
    xs, dys, gs = f32(xc), f32(dyc), f32(gc)
    eps = 1e-6 if kind == "rms" else 1e-5
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, eps)
    else:
        _, mean, rstd = ln_forward(lib, x, g, b, eps)
    torch.cuda.synchronize()
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    if kind == "rms":
        dx, dg = rms_backward(lib, dy, x, rstd, g)
    else:
        dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    trace = re.findall(r"fln backward: .* -> (\S+) wpr=(\d+) vpl=(\d+) threads=(\d+)",
                       capfd.readouterr().err)
    assert [t[:3] for t in trace] == [("registers", str(w), str(v))], trace
    io = "bf16" if dtype == torch.bfloat16 else "f16"
    if kind == "rms":
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, eps)
    else:
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, eps)
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs), io, f"{kind} {cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")


WIDE_KINDS = ["ln", "rms", "add_ln", "add_rms", "gelu_none", "gelu_tanh", "ln_fp8", "rms_fp8",
              "add_rms_fp8", "ln_mx", "rms_mx", "add_rms_mx"]


@pytest.mark.parametrize("kind", WIDE_KINDS)
@pytest.mark.parametrize("dtype,rows,cols,aligned", [
    (torch.bfloat16, 3, 131072, True), (torch.float16, 600, 65544, True),
    (torch.float32, 5, 40000, True), (torch.bfloat16, 1100, 20001, False),
    (torch.float32, 7, 33344, False)],
    ids=["bf16-131072", "f16-65544x600", "f32-40000", "bf16-20001-scalar",
         "f32-33344-scalar"])
def test_wide_rows_forward(lib, monkeypatch, capfd, kind, dtype, rows, cols, aligned):
    """Rows past the LDS tile (16-bit > 65536 columns, fp32 > 32768) and long rows off the
    vector path (odd widths; 16-byte misaligned pointers) take the streamed wide-row kernel,
    save LayerNorm / RMSNorm / LN + GELU rows (tanh; erf in fp32) on the vector path of up to
    twice the tile (16-bit 131072, fp32 65536), which take the LDS-staged kernel with the rest
    of each row in registers: every forward flavour against the oracle, statistics included,
    bitwise reproducible (600 / 1100 rows: several rows per block).  MXFP8 at widths that are
    not a multiple of 32 must be refused before any launch, outputs untouched.  3 / 5 / 7 rows
    would take the split forward: FLN_FWD_NO_SPLIT keeps every case on the kernel named, and
    the dispatcher's trace must show it."""
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    if kind.endswith("_mx") and cols % 32:
        x = torch.zeros(rows, cols, device="cuda", dtype=dtype)
        g = torch.ones(cols, device="cuda", dtype=dtype)
        q = torch.full((rows, cols), 0x5A, device="cuda", dtype=torch.uint8)
        sc = torch.full((rows, -(-cols // 32)), 0x5A, device="cuda", dtype=torch.uint8)
        h = torch.empty_like(x)
        rc = _mx_call(lib, kind[:-3], x, x, g, None, q, sc, h, rows, cols, capi.dtype_code(x))
        torch.cuda.synchronize()
        assert rc == 1 and (q == 0x5A).all() and (sc == 0x5A).all()
        return
    gen = torch.Generator().manual_seed(cols + 17 * WIDE_KINDS.index(kind))
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    if aligned:
        x, r = cuda(xc), cuda(rc)
    else:  # one element of offset: 16-byte misaligned device pointers
        xbuf, rbuf = (torch.zeros(rows * cols + 1, dtype=dtype) for _ in range(2))
        xbuf[1:] = xc.flatten()
        rbuf[1:] = rc.flatten()
        x, r = cuda(xbuf)[1:].view(rows, cols), cuda(rbuf)[1:].view(rows, cols)
    g, b = cuda(gc), cuda(bc)
    xs, rs, gs, bs = f32(xc), f32(rc), f32(gc), f32(bc)
    io = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    code = capi.dtype_code(x)
    p = capi.ptr
    # Zero-filled, so the buffers a flavour does not write compare equal between runs.
    out = torch.zeros(rows, cols, device="cuda", dtype=torch.uint8 if "fp8" in kind or "mx" in
                      kind else dtype)
    h = torch.zeros(rows, cols, device="cuda", dtype=dtype)
    mean = torch.zeros(rows, device="cuda")
    rstd = torch.zeros(rows, device="cuda")
    sc = torch.zeros(rows, cols // 32 if kind.endswith("_mx") else 1, device="cuda",
                     dtype=torch.uint8 if kind.endswith("_mx") else torch.float32)

    def run():
        st = capi.stream()
        if kind == "ln":
            rc_ = lib.fln_layernorm_forward(p(x), p(g), p(b), p(out), p(mean), p(rstd), rows,
                                            cols, code, 1e-5, st)
        elif kind == "rms":
            rc_ = lib.fln_rmsnorm_forward(p(x), p(g), p(out), p(rstd), rows, cols, code, 1e-6,
                                          st)
        elif kind == "add_ln":
            rc_ = lib.fln_add_layernorm_forward(p(x), p(r), p(g), p(b), p(h), p(out), p(mean),
                                                p(rstd), rows, cols, code, 1e-5, st)
        elif kind == "add_rms":
            rc_ = lib.fln_add_rmsnorm_forward(p(x), p(r), p(g), p(h), p(out), p(rstd), rows,
                                              cols, code, 1e-6, st)
        elif kind.startswith("gelu"):
            gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
            rc_ = lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(out), p(mean), p(rstd),
                                                 rows, cols, code, 1e-5, gm, st)
        elif kind == "ln_fp8":
            rc_ = lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(out), p(sc), p(mean),
                                                p(rstd), rows, cols, code, 1e-5, st)
        elif kind == "rms_fp8":
            rc_ = lib.fln_rmsnorm_fp8_forward(p(x), p(g), p(out), p(sc), p(rstd), rows, cols,
                                              code, 1e-6, st)
        elif kind == "add_rms_fp8":
            rc_ = lib.fln_add_rmsnorm_fp8_forward(p(x), p(r), p(g), p(h), p(out), p(sc),
                                                  p(rstd), rows, cols, code, 1e-6, st)
        else:
            rc_ = _mx_call(lib, kind[:-3], x, r, g, b if kind == "ln_mx" else None, out, sc, h,
                           rows, cols, code)
        capi.check(rc_)
        torch.cuda.synchronize()
        return out.clone(), sc.clone(), mean.clone(), rstd.clone(), h.clone()

    routes, (got, sc_got, m_got, r_got, h_got) = _traced_routes(capfd, monkeypatch, run)
    vs = 16 // x.element_size()
    half_in_registers = aligned and (kind in ("ln", "rms", "gelu_tanh") or
                                     (kind == "gelu_none" and dtype == torch.float32)) and \
        8 * 1024 < cols // vs <= 16 * 1024
    assert routes == ["lds+registers" if half_in_registers else "wide"], routes
    again = run()
    for name, a, c in zip(("out", "scale", "mean", "rstd", "h"),
                          (got, sc_got, m_got, r_got, h_got), again):
        assert torch.equal(a, c), f"{name} bitwise reproducible"
    if kind.startswith("add"):
        h_ref = xc + rc  # torch CPU add in the I/O type
        assert torch.equal(h_got.cpu(), h_ref), "h bit-exact"
        hs = f32(h_ref)
    else:
        hs = xs
    rms = "rms" in kind
    if rms:
        y_ref, r_ref = norms.rms_norm_fwd(hs, gs, 1e-6)
        m_ref = None
    else:
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(hs, gs, bs, 1e-5)
    if not kind.endswith("_mx"):  # the MX entry points are called without statistics
        assert np.abs(to_np(r_got) / np.asarray(r_ref).reshape(-1) - 1).max() <= 1e-5
        if m_ref is not None:
            m_ref = np.asarray(m_ref).reshape(-1)
            assert np.abs(to_np(m_got) - m_ref).max() <= 1e-5 * max(1.0, np.abs(m_ref).max())
    if kind.endswith("_fp8"):
        if kind == "ln_fp8":
            q_ref, s_ref = norms.layer_norm_fp8_fwd(hs, gs, bs, 1e-5)
        else:
            q_ref, s_ref = norms.rms_norm_fp8_fwd(hs, gs, 1e-6)
        assert_fp8_close(got.cpu().numpy(), to_np(sc_got).reshape(-1), q_ref, s_ref, kind,
                         t_ref=_scaled(y_ref))
        return
    if kind.endswith("_mx"):
        q_ref, s_ref = norms.mx_e4m3_quantize(y_ref)
        assert_mx_close(got.cpu().numpy(), sc_got.cpu().numpy(), q_ref, s_ref, y_ref, kind)
        return
    if kind.startswith("gelu"):
        y_ref = norms.gelu(y_ref, kind[5:])
    if dtype == torch.float32:
        assert np.abs(to_np(got) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        atol = affine_atol(hs, gs, None if rms else bs, 1e-5)
        if not rms:
            # These rows have mean ~0.5: the fp32 mean's own rounding (a few ulps of |mean|)
            # shifts every output by rstd |gamma| times it -- more than an f16 ulp where the
            # output is subnormal (fixed 2^-24 spacing below 6.1e-5).
            atol = atol + 2.0 ** -21 * (np.abs(m_ref)[:, None] * np.asarray(r_ref).reshape(-1, 1)
                                        * np.abs(gs))
        assert_within_ulp(to_np(got), y_ref, 1.0, atol=atol, **_tol_fwd(dtype), what=kind)


@pytest.mark.parametrize("kind,dtype,rows,cols", [
    ("ln", torch.bfloat16, 16, 262144), ("rms", torch.float16, 40, 70000),
    ("gelu_none", torch.bfloat16, 8, 140000), ("gelu_tanh", torch.float32, 60, 40000),
    ("add_ln", torch.bfloat16, 24, 100000), ("add_ln_noh", torch.float16, 12, 90000),
    ("add_rms", torch.float16, 4, 524288), ("gelu_none", torch.float32, 6, 65536),
    ("ln", torch.float32, 30, 32768), ("ln", torch.bfloat16, 300, 140000),
    ("gelu_tanh", torch.bfloat16, 20, 200000), ("rms", torch.float32, 50, 70000)],
    ids=["ln-bf16-16x262144", "rms-f16-40x70000", "gelu_none-bf16-8x140000",
         "gelu_tanh-f32-60x40000", "add_ln-bf16-24x100000", "add_ln_noh-f16-12x90000",
         "add_rms-f16-4x524288", "gelu_none-f32-6x65536", "ln-f32-30x32768",
         "ln-bf16-300x140000", "gelu_tanh-bf16-20x200000", "rms-f32-50x70000"])
def test_split_rows_forward(lib, monkeypatch, kind, dtype, rows, cols):
    """Few rows past the register tiles (fewer than 4 per CU where the streamed kernel would
    run, a quarter of the CUs where an LDS-staged one would): each row split into up to 64 column chunks
    (one block each; the chunk statistics handed to the output pass through the first bytes of
    the row's own y; 70000 fp16 columns: a last chunk of 46 vectors; a residual with and
    without h).  Outputs and statistics against the oracle, bitwise reproducible, within 1 ulp
    of one block per row (FLN_FWD_NO_SPLIT), and an in-place call (y = x, so no split) equal to
    that."""
    gen = torch.Generator().manual_seed(cols + rows)
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    code = capi.dtype_code(x)
    p = capi.ptr
    rms = "rms" in kind
    eps = 1e-6 if rms else 1e-5

    def run(src=None, inplace=False):
        src = x if src is None else src
        out = src if inplace else torch.empty_like(x)
        h = torch.zeros_like(x)
        mean = torch.zeros(rows, device="cuda")
        rstd = torch.zeros(rows, device="cuda")
        st = capi.stream()
        if kind == "ln":
            rc_ = lib.fln_layernorm_forward(p(src), p(g), p(b), p(out), p(mean), p(rstd), rows,
                                            cols, code, eps, st)
        elif kind == "rms":
            rc_ = lib.fln_rmsnorm_forward(p(src), p(g), p(out), p(rstd), rows, cols, code, eps,
                                          st)
        elif kind.startswith("gelu"):
            gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
            rc_ = lib.fln_layernorm_gelu_forward(p(src), p(g), p(b), p(out), p(mean), p(rstd),
                                                 rows, cols, code, eps, gm, st)
        elif kind.startswith("add_ln"):
            rc_ = lib.fln_add_layernorm_forward(p(src), p(r), p(g), p(b),
                                                None if kind == "add_ln_noh" else p(h), p(out),
                                                p(mean), p(rstd), rows, cols, code, eps, st)
        else:
            rc_ = lib.fln_add_rmsnorm_forward(p(src), p(r), p(g), p(h), p(out), p(rstd), rows,
                                              cols, code, eps, st)
        capi.check(rc_)
        torch.cuda.synchronize()
        return out.clone(), mean, rstd, h

    got, m_got, r_got, h_got = run()
    again = run()
    for name, a, c in zip(("out", "mean", "rstd", "h"), (got, m_got, r_got, h_got), again):
        assert torch.equal(a, c), f"{name} bitwise reproducible"
    xs, gs, bs = f32(xc), f32(gc), f32(bc)
    if kind.startswith("add"):
        h_ref = xc + rc  # torch CPU add in the I/O type
        if kind != "add_ln_noh":
            assert torch.equal(h_got.cpu(), h_ref), "h bit-exact"
        hs = f32(h_ref)
    else:
        hs = xs
    if rms:
        y_ref, r_ref = norms.rms_norm_fwd(hs, gs, eps)
        m_ref = None
    else:
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(hs, gs, bs, eps)
    assert np.abs(to_np(r_got) / np.asarray(r_ref).reshape(-1) - 1).max() <= 1e-5
    if m_ref is not None:
        m_ref = np.asarray(m_ref).reshape(-1)
        assert np.abs(to_np(m_got) - m_ref).max() <= 1e-5 * max(1.0, np.abs(m_ref).max())
    if kind.startswith("gelu"):
        y_ref = norms.gelu(y_ref, kind[5:])
    if dtype == torch.float32:
        assert np.abs(to_np(got) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        atol = affine_atol(hs, gs, None if rms else bs, eps)
        if not rms:
            atol = atol + 2.0 ** -21 * (np.abs(m_ref)[:, None] * np.asarray(r_ref).reshape(-1, 1)
                                        * np.abs(gs))
        assert_within_ulp(to_np(got), y_ref, 1.0, atol=atol, **_tol_fwd(dtype), what=kind)
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    one, m_one, r_one, _ = run()
    monkeypatch.delenv("FLN_FWD_NO_SPLIT")
    capi.reload_tuning()
    assert np.abs(to_np(r_got) / to_np(r_one) - 1).max() <= 1e-6
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10 if dtype == torch.float16 else 1e-5
    assert float((got.float() - one.float()).abs().max()) <= ulp * max(1.0, float(one.float().abs().max()))
    inplace, _, _, _ = run(src=x.clone(), inplace=True)
    assert torch.equal(inplace, one), "in place (no split) equals one block per row"


@pytest.mark.parametrize("kind,dtype,rows,cols", [
    ("ln_fp8", torch.bfloat16, 16, 262144), ("add_rms_fp8", torch.float16, 8, 131072),
    ("ln_fp8", torch.float32, 20, 40000), ("rms_mx", torch.bfloat16, 12, 200000),
    ("add_rms_mx", torch.float16, 4, 524288), ("rms_fp8", torch.bfloat16, 10, 131080),
    ("add_ln_fp8", torch.bfloat16, 8, 262144), ("ln_mx", torch.float16, 6, 200000)],
    ids=["ln_fp8-bf16-16x262144", "add_rms_fp8-f16-8x131072", "ln_fp8-f32-20x40000",
         "rms_mx-bf16-12x200000", "add_rms_mx-f16-4x524288", "rms_fp8-bf16-10x131080-nosplit",
         "add_ln_fp8-bf16-8x262144", "ln_mx-f16-6x200000"])
def test_split_rows_forward_fp8(lib, monkeypatch, kind, dtype, rows, cols):
    """The split forward with fp8 outputs: the per-row scale takes a fourth launch (chunk
    maxima after the chunk triples in the head, which then spans several waves' worth of code
    vectors), MX keeps the head a whole number of 32-element blocks; 131080 columns (rows not a
    multiple of 16 bytes of codes) keep one block per row.  Codes and scales against the
    oracle, bitwise reproducible, and scales within 1e-6 of one block per row
    (FLN_FWD_NO_SPLIT)."""
    gen = torch.Generator().manual_seed(cols + rows + 3)
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    code = capi.dtype_code(x)
    p = capi.ptr
    mx = kind.endswith("_mx")

    def run():
        q = torch.zeros(rows, cols, device="cuda", dtype=torch.uint8)
        sc = torch.zeros(rows, cols // 32 if mx else 1, device="cuda",
                         dtype=torch.uint8 if mx else torch.float32)
        h = torch.zeros_like(x)
        mean = torch.zeros(rows, device="cuda")
        rstd = torch.zeros(rows, device="cuda")
        st = capi.stream()
        if kind == "ln_fp8":
            rc_ = lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(sc), p(mean), p(rstd),
                                                rows, cols, code, 1e-5, st)
        elif kind == "rms_fp8":
            rc_ = lib.fln_rmsnorm_fp8_forward(p(x), p(g), p(q), p(sc), p(rstd), rows, cols, code,
                                              1e-6, st)
        elif kind == "add_rms_fp8":
            rc_ = lib.fln_add_rmsnorm_fp8_forward(p(x), p(r), p(g), p(h), p(q), p(sc), p(rstd),
                                                  rows, cols, code, 1e-6, st)
        elif kind == "add_ln_fp8":
            rc_ = lib.fln_add_layernorm_fp8_forward(p(x), p(r), p(g), p(b), p(h), p(q), p(sc),
                                                    p(mean), p(rstd), rows, cols, code, 1e-5, st)
        else:
            rc_ = _mx_call(lib, kind[:-3], x, r, g, b if kind == "ln_mx" else None, q, sc, h,
                           rows, cols, code)
        capi.check(rc_)
        torch.cuda.synchronize()
        return q, sc, mean, rstd, h

    got = run()
    again = run()
    for name, a, c in zip(("codes", "scale", "mean", "rstd", "h"), got, again):
        assert torch.equal(a, c), f"{name} bitwise reproducible"
    q, sc, mean, rstd, h = got
    xs, gs, bs = f32(xc), f32(gc), f32(bc)
    io = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    if kind.startswith("add"):
        h_ref = xc + rc  # torch CPU add in the I/O type
        assert torch.equal(h.cpu(), h_ref), "h bit-exact"
    if mx:
        q_ref, s_ref, y_ref = _mx_ref(kind[:-3], xs, f32(rc), gs, bs, io)
        assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, s_ref, y_ref, kind)
    else:
        hs = f32(xc + rc) if kind.startswith("add") else xs
        if kind in ("ln_fp8", "add_ln_fp8"):
            y_ref, m_ref, r_ref = norms.layer_norm_fwd(hs, gs, bs, 1e-5)
            q_ref, s_ref = norms.layer_norm_fp8_fwd(hs, gs, bs, 1e-5)
            m_ref = np.asarray(m_ref).reshape(-1)
            assert np.abs(to_np(mean) - m_ref).max() <= 1e-5 * max(1.0, np.abs(m_ref).max())
        else:
            y_ref, r_ref = norms.rms_norm_fwd(hs, gs, 1e-6)
            q_ref, s_ref = norms.rms_norm_fp8_fwd(hs, gs, 1e-6)
        assert np.abs(to_np(rstd) / np.asarray(r_ref).reshape(-1) - 1).max() <= 1e-5
        assert_fp8_close(q.cpu().numpy(), to_np(sc).reshape(-1), q_ref, s_ref, kind,
                         t_ref=_scaled(y_ref))
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    one = run()
    monkeypatch.delenv("FLN_FWD_NO_SPLIT")
    capi.reload_tuning()
    if mx:
        assert float((q.float() - one[0].float()).abs().gt(1).float().mean()) <= 1e-3
    else:
        assert np.abs(to_np(sc) / to_np(one[1]) - 1).max() <= 1e-6
        assert float((q != one[0]).float().mean()) <= 1e-3


@pytest.mark.parametrize("splits", [1, 3, 7, 64])
@pytest.mark.parametrize("kind", ["ln", "ln_fp8", "add_rms_mx"])
def test_split_rows_forced_counts(lib, monkeypatch, kind, splits):
    """The split forward at forced chunk counts (FLN_FWD_SPLITS: one chunk, so the head block
    and the output block share the row; odd counts with a short last chunk; the most, whose
    fp8 head spans several waves): outputs within 1 ulp of one block per row (fp8 / MX codes:
    at most 0.1% differ), scales and statistics to 1e-6."""
    rows, cols = 6, 139264  # 17408 bf16 vectors: 34 steps of 512
    gen = torch.Generator().manual_seed(splits + 97 * len(kind))
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(torch.bfloat16)
    rc = torch.randn(rows, cols, generator=gen).to(torch.bfloat16)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    code = capi.dtype_code(x)
    p = capi.ptr

    def run():
        out = torch.zeros(rows, cols, device="cuda",
                          dtype=torch.bfloat16 if kind == "ln" else torch.uint8)
        sc = torch.zeros(rows, cols // 32 if kind == "add_rms_mx" else 1, device="cuda",
                         dtype=torch.uint8 if kind == "add_rms_mx" else torch.float32)
        h = torch.zeros_like(x)
        mean = torch.zeros(rows, device="cuda")
        rstd = torch.zeros(rows, device="cuda")
        if kind == "ln":
            rc_ = lib.fln_layernorm_forward(p(x), p(g), p(b), p(out), p(mean), p(rstd), rows,
                                            cols, code, 1e-5, capi.stream())
        elif kind == "ln_fp8":
            rc_ = lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(out), p(sc), p(mean), p(rstd),
                                                rows, cols, code, 1e-5, capi.stream())
        else:
            rc_ = _mx_call(lib, "add_rms", x, r, g, None, out, sc, h, rows, cols, code)
        capi.check(rc_)
        torch.cuda.synchronize()
        return out, sc, mean, rstd, h

    monkeypatch.setenv("FLN_FWD_SPLITS", str(splits))
    capi.reload_tuning()
    got = run()
    monkeypatch.delenv("FLN_FWD_SPLITS")
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    one = run()
    monkeypatch.delenv("FLN_FWD_NO_SPLIT")
    capi.reload_tuning()
    if kind == "ln":
        d = (got[0].float() - one[0].float()).abs().max()
        assert float(d) <= 2.0 ** -7 * max(1.0, float(one[0].float().abs().max()))
        assert np.abs(to_np(got[2]) - to_np(one[2])).max() <= 1e-6 * max(1.0, float(one[2].abs().max()))
    else:
        assert float((got[0] != one[0]).float().mean()) <= 1e-3
        if kind == "ln_fp8":
            assert np.abs(to_np(got[1]) / to_np(one[1]) - 1).max() <= 1e-6
        else:
            assert torch.equal(got[4], one[4]), "h"
    if kind != "add_rms_mx":
        assert np.abs(to_np(got[3]) / to_np(one[3]) - 1).max() <= 1e-6


@pytest.mark.parametrize("kind", ["ln", "rms", "ln_fp8"])
def test_split_rows_forward_optional_pointers(lib, monkeypatch, kind):
    """The split forward without gamma / beta (identity affine) and without the mean / rstd
    outputs: the same outputs as one block per row to 1 ulp (fp8: codes differ on at most 0.1%,
    scales to 1e-6), against the oracle with gamma = 1, beta = 0."""
    rows, cols = 16, 262144
    gen = torch.Generator().manual_seed(5 + len(kind))
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(torch.bfloat16)
    x = cuda(xc)
    code = capi.dtype_code(x)
    p = capi.ptr

    def run():
        if kind == "ln_fp8":
            q = torch.zeros(rows, cols, device="cuda", dtype=torch.uint8)
            sc = torch.zeros(rows, device="cuda")
            capi.check(lib.fln_layernorm_fp8_forward(p(x), None, None, p(q), p(sc), None, None,
                                                     rows, cols, code, 1e-5, capi.stream()))
            torch.cuda.synchronize()
            return q, sc
        y = torch.zeros_like(x)
        if kind == "ln":
            capi.check(lib.fln_layernorm_forward(p(x), None, None, p(y), None, None, rows, cols,
                                                 code, 1e-5, capi.stream()))
        else:
            capi.check(lib.fln_rmsnorm_forward(p(x), None, p(y), None, rows, cols, code, 1e-6,
                                               capi.stream()))
        torch.cuda.synchronize()
        return y, None

    got = run()
    monkeypatch.setenv("FLN_FWD_NO_SPLIT", "1")
    capi.reload_tuning()
    one = run()
    monkeypatch.delenv("FLN_FWD_NO_SPLIT")
    capi.reload_tuning()
    xs = f32(xc)
    if kind == "ln_fp8":
        q_ref, s_ref = norms.layer_norm_fp8_fwd(xs, None, None, 1e-5)
        y_ref, _, _ = norms.layer_norm_fwd(xs, None, None, 1e-5)
        assert_fp8_close(got[0].cpu().numpy(), to_np(got[1]), q_ref, s_ref, kind,
                         t_ref=_scaled(y_ref))
        assert float((got[0] != one[0]).float().mean()) <= 1e-3
        assert np.abs(to_np(got[1]) / to_np(one[1]) - 1).max() <= 1e-6
        return
    atol = affine_atol(xs, None, None, 1e-5)
    if kind == "ln":
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, None, None, 1e-5)
        atol = atol + 2.0 ** -21 * (np.abs(np.asarray(m_ref)).reshape(-1, 1) *
                                    np.asarray(r_ref).reshape(-1, 1))
    else:
        y_ref, _ = norms.rms_norm_fwd(xs, None, 1e-6)
    assert_within_ulp(to_np(got[0]), y_ref, 1.0, atol=atol, kind="bf16", what=kind)
    d = (got[0].float() - one[0].float()).abs().max()
    assert float(d) <= 2.0 ** -7 * max(1.0, float(one[0].float().abs().max()))


def test_fp8_variants_reject_bad_arguments(lib):
    x = torch.randn(4, 64, device="cuda")
    q = torch.empty(4, 64, device="cuda", dtype=torch.uint8)
    s = torch.empty(4, device="cuda")
    p = capi.ptr
    # residual is required; a scale buffer is required; fp64 has no fp8 path
    assert lib.fln_add_rmsnorm_fp8_forward(p(x), None, None, None, p(q), p(s), None, 4, 64,
                                           capi.F32, 1e-6, capi.stream()) == 1
    assert lib.fln_add_layernorm_fp8_forward(p(x), p(x), None, None, None, p(q), None, None,
                                             None, 4, 64, capi.F32, 1e-5, capi.stream()) == 1
    assert lib.fln_rmsnorm_fp8_forward(p(x), None, p(q), p(s), None, 4, 64, capi.F64, 1e-6,
                                       capi.stream()) == 1


@pytest.mark.parametrize("mode", ["none", "tanh"])
@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(64, 4096), (17, 1023), (33, 7168), (2, 16384), (300, 768),
                                       (3, 12288), (600, 10248), (2, 32768), (300, 24576),
                                       (2, 40960)])
def test_layernorm_gelu_backward_matrix(lib, mode, dtype, rows, cols):
    """Backward of GELU(LayerNorm(x) gamma + beta): the forward with statistics, then the fused
    backward, against the numpy oracle (LayerNorm backward of dy GELU'(a)).  16-bit rows of
    8193..16384 columns keep gamma / beta in LDS in the register kernel (600 rows: several per
    block)."""
    gen = torch.Generator().manual_seed(rows * 7 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.2 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy = cuda(xc), cuda(gc), cuda(bc), cuda(dyc)
    gm = capi.GELU_ERF if mode == "none" else capi.GELU_TANH
    code = capi.dtype_code(x)
    y = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    p = capi.ptr
    capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                              cols, code, 1e-5, gm, capi.stream()))
    dx = torch.empty_like(x)
    dg = torch.empty(cols, device="cuda")
    db = torch.empty(cols, device="cuda")
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b), p(dx),
                                               p(dg), p(db), rows, cols, code, capi.F32, gm,
                                               p(ws), n, capi.stream()))
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    y_ref = norms.layer_norm_gelu_fwd(xs, gs, bs, 1e-5, mode)
    dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, mode)
    al = tolerance.dx_allowance(xs, dys, gs, 1e-5, beta=bs, approximate=mode)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        kind = "bf16" if dtype == torch.bfloat16 else "f16"
        # GELU(a) near a = 0 inherits the affine rounding allowance of a (slope 1/2 there)
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(xs, gs, bs, 1e-5), kind=kind,
                          what="y")
    assert_dx(to_np(dx), dx_ref, al, _kind(dtype),
              f"gelu {mode} matrix {_kind(dtype)} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")


def test_layernorm_gelu_entry_points_reject_bad_mode(lib):
    x = torch.randn(4, 64, device="cuda")
    p = capi.ptr
    y = torch.empty_like(x)
    assert lib.fln_layernorm_gelu_forward(p(x), None, None, p(y), None, None, 4, 64, capi.F32,
                                          1e-5, 0, capi.stream()) == 1
    assert lib.fln_layernorm_gelu_backward(p(x), p(x), p(x), p(x), None, None, p(y), None, None,
                                           4, 64, capi.F32, capi.F32, 3, None, 0,
                                           capi.stream()) == 1


def _mx_call(lib, kind, x, r, g, b, q, sc, h, rows, cols, code):
    p = capi.ptr
    if kind == "ln":
        return lib.fln_layernorm_mxfp8_forward(p(x), p(g), p(b), p(q), p(sc), None, None, rows,
                                               cols, code, 1e-5, capi.stream())
    if kind == "rms":
        return lib.fln_rmsnorm_mxfp8_forward(p(x), p(g), p(q), p(sc), None, rows, cols, code,
                                             1e-6, capi.stream())
    return lib.fln_add_rmsnorm_mxfp8_forward(p(x), p(r), p(g), p(h), p(q), p(sc), None, rows,
                                             cols, code, 1e-6, capi.stream())


def _mx_ref(kind, xs, rs, gs, bs, io):
    if kind == "ln":
        y, _, _ = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
    elif kind == "rms":
        y, _ = norms.rms_norm_fwd(xs, gs, 1e-6)
    else:
        y, _, _ = norms.add_rms_norm_fwd(xs, rs, gs, 1e-6, io)
    q, sc = norms.mx_e4m3_quantize(y)
    return q, sc, y


@pytest.mark.parametrize("kind", ["ln", "rms", "add_rms"])
@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols,path", [
    (64, 4096, "vec"), (33, 7168, "vec"), (9, 96, "vec"), (2, 16384, "vec"), (2, 32768, "vec"),
    (300, 24576, "vec"), (3, 12288, "vec"), (2, 40960, "vec"), (300, 65536, "vec"),
    (13, 1024, "scalar"), (3, 2048, "loop")])
def test_mxfp8_matrix(lib, monkeypatch, kind, dtype, rows, cols, path):
    """OCP MXFP8 outputs (codes + E8M0 block scales) of LayerNorm, RMSNorm and residual +
    RMSNorm over dtypes and widths, on the vector path (block = 32 / VEC adjacent lanes), the
    scalar path (misaligned pointers: block = 32 lanes) and the looped kernel."""
    gen = torch.Generator().manual_seed(rows * 131 + cols)
    xc = (torch.randn(rows, cols, generator=gen) * torch.exp(torch.randn(rows, 1, generator=gen))
          ).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    if path == "scalar":  # one element of offset: 16-byte misaligned device pointers
        xbuf, rbuf = (torch.zeros(rows * cols + 1, dtype=dtype) for _ in range(2))
        xbuf[1:] = xc.flatten()
        rbuf[1:] = rc.flatten()
        xd, rd = cuda(xbuf)[1:].view(rows, cols), cuda(rbuf)[1:].view(rows, cols)
    else:
        xd, rd = cuda(xc), cuda(rc)
    g, b = cuda(gc), cuda(bc)
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    sc = torch.empty(rows, cols // 32, device="cuda", dtype=torch.uint8)
    h = torch.empty(rows, cols, device="cuda", dtype=dtype)
    if path == "loop":
        monkeypatch.setenv("FLN_FORCE_LOOP", "1")
        capi.reload_tuning()
    capi.check(_mx_call(lib, kind, xd, rd, g, b if kind == "ln" else None, q, sc, h, rows, cols,
                        capi.dtype_code(xd)))
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_FORCE_LOOP", raising=False)
    capi.reload_tuning()
    io = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    q_ref, sc_ref, y_ref = _mx_ref(kind, f32(xc), f32(rc), f32(gc), f32(bc), io)
    if kind == "add_rms":
        assert np.array_equal(to_np(h), to_np(xc + rc)), "h bit-exact"
    assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, sc_ref, y_ref, f"mx {kind}")


def test_mxfp8_add_rmsnorm_bf16_4096x7168(lib):
    """Residual + RMSNorm -> MXFP8 at C5's width (bf16, 7 outlier channels x20)."""
    w = WORKLOADS["c5_ln_fp8_bf16_32768x7168"]
    inp = make_inputs(w, 4096)
    gen = torch.Generator().manual_seed(77)
    rc = torch.randn(4096, 7168, generator=gen).to(torch.bfloat16)
    x, r, g = cuda(inp["x"]), cuda(rc), cuda(inp["gamma"])
    q = torch.empty(4096, 7168, device="cuda", dtype=torch.uint8)
    sc = torch.empty(4096, 224, device="cuda", dtype=torch.uint8)
    h = torch.empty_like(x)
    capi.check(_mx_call(lib, "add_rms", x, r, g, None, q, sc, h, 4096, 7168, capi.BF16))
    q_ref, sc_ref, y_ref = _mx_ref("add_rms", f32(inp["x"]), f32(rc), f32(inp["gamma"]), None,
                                   "bf16")
    assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, sc_ref, y_ref, "mx 4096x7168")


def test_mxfp8_rejects_widths_not_multiple_of_32(lib):
    x = torch.randn(4, 48, device="cuda")
    q = torch.empty(4, 48, device="cuda", dtype=torch.uint8)
    sc = torch.empty(8, device="cuda", dtype=torch.uint8)
    assert lib.fln_rmsnorm_mxfp8_forward(capi.ptr(x), None, capi.ptr(q), capi.ptr(sc), None, 4,
                                         48, capi.F32, 1e-6, capi.stream()) == 1
    assert lib.fln_layernorm_mxfp8_forward(capi.ptr(x), None, None, capi.ptr(q), None, None,
                                           None, 4, 64, capi.F32, 1e-5, capi.stream()) == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(96, 2048), (3, 12288), (5, 16384), (2, 32768),
                                       (600, 12296)])
def test_residual_gradient_is_added(lib, dtype, rows, cols):
    """dx + dres for LayerNorm and RMSNorm; 16-bit rows of 8193..16384 columns take the
    register kernel with gamma parked in LDS (600 rows: several per block), 32768 the two
    passes."""
    gen = torch.Generator().manual_seed(9 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, dy, dr, g = cuda(xc), cuda(dyc), cuda(drc), cuda(gc)
    _, mean, rstd = ln_forward(lib, x, g, g, 1e-5)
    dx, _, _ = ln_backward(lib, dy, x, mean, rstd, g, want_params=False, dres=dr)
    dx_ref, _, _ = norms.layer_norm_bwd(f32(dyc), f32(xc), f32(gc), 1e-5)
    dx_ref = dx_ref + f32(drc)
    assert_dx(to_np(dx), dx_ref,
              tolerance.dx_allowance(f32(xc), f32(dyc), f32(gc), 1e-5, dres=f32(drc)),
              _kind(dtype), f"dx + dres {_kind(dtype)} {rows}x{cols}")
    _, rs = rms_forward(lib, x, g, 1e-6)
    dxr, _ = rms_backward(lib, dy, x, rs, g, dres=dr)
    dxr_ref, _ = norms.rms_norm_bwd(f32(dyc), f32(xc), f32(gc), 1e-6)
    dxr_ref = dxr_ref + f32(drc)
    assert_dx(to_np(dxr), dxr_ref,
              tolerance.dx_allowance(f32(xc), f32(dyc), f32(gc), 1e-6, rms=True, dres=f32(drc)),
              _kind(dtype), f"rms dx + dres {_kind(dtype)} {rows}x{cols}")


@pytest.mark.parametrize("kind", ["ln", "rms", "ln_dres", "gelu_none", "gelu_tanh"])
@pytest.mark.parametrize("cols", [8196, 12288, 12292, 16384])
def test_fp32_wide_row_backward(lib, monkeypatch, kind, cols):
    """fp32 rows of 8193..12288 columns take the register backward with 3 vectors per lane in
    1024-thread blocks, LayerNorm / RMSNorm rows up to 16384 with 4, the other flavours there
    the LDS-staged backward (one 1024-thread block per row, several rows per block here): parity
    with the oracle for every flavour, dgamma/dbeta bitwise reproducible, and agreement with
    the route those rows take without either (FLN_BWD_NO_LDS)."""
    rows = 600
    gen = torch.Generator().manual_seed(cols * 3 + len(kind))
    xc = torch.randn(rows, cols, generator=gen) * 2 + 0.5
    gc = 1 + 0.1 * torch.randn(cols, generator=gen)
    bc = 0.2 * torch.randn(cols, generator=gen)
    dyc = torch.randn(rows, cols, generator=gen)
    drc = torch.randn(rows, cols, generator=gen)
    x, g, b, dy, dr = cuda(xc), cuda(gc), cuda(bc), cuda(dyc), cuda(drc)
    xs, gs, bs, dys = xc.numpy(), gc.numpy(), bc.numpy(), dyc.numpy()
    p = capi.ptr

    def run():
        if kind == "rms":
            _, rs = rms_forward(lib, x, g, 1e-6)
            dx, dw = rms_backward(lib, dy, x, rs, g)
            return dx, dw, None
        if kind.startswith("gelu"):
            gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
            y = torch.empty_like(x)
            mean = torch.empty(rows, device="cuda")
            rstd = torch.empty(rows, device="cuda")
            capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd),
                                                      rows, cols, capi.F32, 1e-5, gm,
                                                      capi.stream()))
            dx = torch.empty_like(x)
            dg = torch.empty(cols, device="cuda")
            db = torch.empty(cols, device="cuda")
            ws, n = workspace(lib, rows, cols, x)
            capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                       p(dx), p(dg), p(db), rows, cols, capi.F32,
                                                       capi.F32, gm, p(ws), n, capi.stream()))
            return dx, dg, db
        _, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
        return ln_backward(lib, dy, x, mean, rstd, g, dres=dr if kind == "ln_dres" else None)

    dx, dg, db = run()
    if kind == "rms":
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, 1e-6)
    elif kind.startswith("gelu"):
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, kind[5:])
    else:
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
        if kind == "ln_dres":
            dx_ref = dx_ref + drc.numpy()
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs, bs, drc.numpy()), "f32",
              f"fp32 wide {kind} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    again = run()
    for a, c in zip((dx, dg, db), again):
        if a is not None:
            assert torch.equal(a, c)
    monkeypatch.setenv("FLN_BWD_NO_LDS", "1")
    capi.reload_tuning()
    looped = run()
    monkeypatch.delenv("FLN_BWD_NO_LDS")
    capi.reload_tuning()
    for a, c in zip((dx, dg, db), looped):
        if a is not None:
            scale = float(c.abs().max())
            assert float((a - c).abs().max()) <= 1e-5 * max(1.0, scale)


ROUTE_WIDTHS_16 = [8192, 8200, 16384, 16392, 18432, 18440, 24576, 24584, 32768, 32776, 65536,
                   65544]
ROUTE_WIDTHS_32 = [4096, 4100, 8192, 8196, 16384, 16388, 32768, 32772]


@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, c) for c in ROUTE_WIDTHS_16] +
                         [(torch.float16, c) for c in (18432, 24584, 65544)] +
                         [(torch.float32, c) for c in ROUTE_WIDTHS_32],
                         ids=lambda v: str(v).replace("torch.", ""))
@pytest.mark.parametrize("nrows", ["few", "many"])
def test_route_boundaries(lib, dtype, nrows, cols):
    """Widths on both sides of every kernel-route boundary (register tiles, RAW tiles, the
    768-thread register backward with 3 vectors, the backward raw tiles, the LDS-staged forward, the two passes, the
    streamed wide forward) at a few rows (small backward blocks) and at several rows per block:
    LayerNorm fwd + bwd with a residual gradient and RMSNorm fwd + bwd against the oracle."""
    rows = 37 if nrows == "few" else (700 if cols <= 32776 else 300)
    gen = torch.Generator().manual_seed(rows * 131 + cols)
    xc = (torch.randn(rows, cols, generator=gen) * 1.5 + 0.25).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy, dr = cuda(xc), cuda(gc), cuda(bc), cuda(dyc), cuda(drc)
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
    dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g, dres=dr)
    y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
    dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
    dx_ref = dx_ref + f32(drc)
    assert np.abs(to_np(rstd) / np.asarray(r_ref).reshape(-1) - 1).max() <= 1e-5
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        m = np.asarray(m_ref).reshape(-1, 1)
        atol = affine_atol(xs, gs, bs, 1e-5) + 2.0 ** -21 * (
            np.abs(m) * np.asarray(r_ref).reshape(-1, 1) * np.abs(gs))
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=atol, **_tol_fwd(dtype), what="y")
    assert_dx(to_np(dx), dx_ref, tolerance.dx_allowance(xs, dys, gs, 1e-5, dres=f32(drc)),
              _kind(dtype), f"route {_kind(dtype)} {rows}x{cols} dx + dres")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    yr, rs = rms_forward(lib, x, g, 1e-6)
    dxr, dw = rms_backward(lib, dy, x, rs, g)
    yr_ref, _ = norms.rms_norm_fwd(xs, gs, 1e-6)
    dxr_ref, dw_ref = norms.rms_norm_bwd(dys, xs, gs, 1e-6)
    if dtype == torch.float32:
        assert np.abs(to_np(yr) - yr_ref).max() <= 1e-5 * max(1, np.abs(yr_ref).max())
    else:
        assert_within_ulp(to_np(yr), yr_ref, 1.0, **_tol_fwd(dtype), what="rms y")
    assert_dx(to_np(dxr), dxr_ref, tolerance.dx_allowance(xs, dys, gs, 1e-6, rms=True),
              _kind(dtype), f"route {_kind(dtype)} {rows}x{cols} rms dx")
    assert_close_rel(to_np(dw), dw_ref, 1e-4, "dweight")


@pytest.mark.parametrize("kind,dtype,cols", [("ln", torch.bfloat16, 32768),
                                              ("rms", torch.float16, 28000),
                                              ("ln", torch.bfloat16, 24584)],
                         ids=["ln-bf16-32768", "rms-f16-28000", "ln-bf16-24584"])
def test_raw4_backward_many_rows(lib, monkeypatch, kind, dtype, cols):
    """16-bit LayerNorm / RMSNorm rows of 24577..32768 columns with at least 6 rows per CU take
    the backward raw tiles with 4 vectors per lane and no prefetched row (1600 rows: 6-7 per
    block; 28000 / 24584 columns: the last vectors partly past the row).  dx within 1 ulp of the
    C oracle, the parameter gradients to 1e-4, bitwise reproducible, and agreement with the two
    passes (FLN_BWD_NO_LDS)."""
    rows = 1600
    gen = torch.Generator().manual_seed(cols + 3)
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, dy = cuda(xc), cuda(gc), cuda(dyc)
    xs, gs, dys = f32(xc), f32(gc), f32(dyc)
    ulp_kind = "bf16" if dtype == torch.bfloat16 else "f16"
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, 1e-6)

        def run():
            dx, dw = rms_backward(lib, dy, x, rstd, g)
            return dx, dw, None
        dx_ref, dg_ref = c_oracle.rmsnorm_bwd(dys, xs, gs, 1e-6)
        db_ref = None
    else:
        _, mean, rstd = ln_forward(lib, x, g, None, 1e-5)

        def run():
            return ln_backward(lib, dy, x, mean, rstd, g)
        dx_ref, dg_ref, db_ref = c_oracle.layernorm_bwd(dys, xs, gs, 1e-5)
    dx, dg, db = run()
    al = _flavour_allowance(kind, xs, dys, gs)
    assert_dx(to_np(dx), dx_ref, al, ulp_kind, f"raw4 {kind} {ulp_kind} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    again = run()
    for a, c in zip((dx, dg, db), again):
        if a is not None:
            assert torch.equal(a, c)
    monkeypatch.setenv("FLN_BWD_NO_LDS", "1")
    capi.reload_tuning()
    two_pass = run()
    monkeypatch.delenv("FLN_BWD_NO_LDS")
    capi.reload_tuning()
    # Both are fp32 evaluations rounded once: each within its allowance of the exact value.
    assert_dx(to_np(dx), to_np(two_pass[0]), 2 * al, ulp_kind, "dx vs two passes")
    for a, c in zip((dg, db), two_pass[1:]):
        if a is not None:
            assert_close_rel(to_np(a), to_np(c), 1e-5, "parameter gradient vs two passes")


@pytest.mark.parametrize("kind", ["ln", "rms", "ln_dres", "gelu_tanh", "gelu_none"])
@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, 18432), (torch.float16, 16392),
                                        (torch.bfloat16, 17416), (torch.bfloat16, 20480),
                                        (torch.bfloat16, 19000), (torch.float16, 24576)],
                         ids=["bf16-18432", "f16-16392", "bf16-17416", "bf16-20480",
                              "bf16-19000", "f16-24576"])
def test_16bit_rows_past_16384_backward(lib, monkeypatch, kind, dtype, cols):
    """16-bit rows of 16385..18432 columns take the register backward with one row per
    768-thread block and 3 vectors per lane (the last ones partly past the row; gamma / beta
    parked in LDS for the residual and GELU flavours; 600 rows: several per block) for every
    flavour but fp16 with a residual gradient, which takes the LDS-staged backward with
    768-thread blocks; rows of 18433..24576 without a residual gradient take the raw tiles (3
    vectors per lane of a 1024-thread block, the row kept in the I/O type, GELU' looked up at
    each use; 19000 columns: the last vectors partly past the row); the residual flavour past
    18432 keeps the two passes.  Parity with the oracle, bitwise reproducible, and agreement with the two-pass
    backward (FLN_BWD_NO_LDS, which turns off the 768-thread register, raw-tile and LDS-staged
    kernels)."""
    rows = 600
    gen = torch.Generator().manual_seed(cols + 5 * len(kind))
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.2 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy, dr = cuda(xc), cuda(gc), cuda(bc), cuda(dyc), cuda(drc)
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    code = capi.dtype_code(x)
    p = capi.ptr
    ulp_kind = "bf16" if dtype == torch.bfloat16 else "f16"
    gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, 1e-6)
    else:
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        y = torch.empty_like(x)
        if kind.startswith("gelu"):
            capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd),
                                                      rows, cols, code, 1e-5, gm, capi.stream()))
        else:
            capi.check(lib.fln_layernorm_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                                 cols, code, 1e-5, capi.stream()))

    def run():
        if kind == "rms":
            dx, dw = rms_backward(lib, dy, x, rstd, g)
            return dx, dw, None
        if kind.startswith("gelu"):
            dx = torch.empty_like(x)
            dg = torch.empty(cols, device="cuda")
            db = torch.empty(cols, device="cuda")
            ws, n = workspace(lib, rows, cols, x)
            capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                       p(dx), p(dg), p(db), rows, cols, code,
                                                       capi.F32, gm, p(ws), n, capi.stream()))
            torch.cuda.synchronize()
            return dx, dg, db
        return ln_backward(lib, dy, x, mean, rstd, g, dres=dr if kind == "ln_dres" else None)

    dx, dg, db = run()
    if kind == "rms":
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, 1e-6)
    elif kind.startswith("gelu"):
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, kind[5:])
    else:
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
        if kind == "ln_dres":
            dx_ref = dx_ref + f32(drc)
    al = _flavour_allowance(kind, xs, dys, gs, bs, f32(drc))
    assert_dx(to_np(dx), dx_ref, al, ulp_kind, f"past 16384 {kind} {ulp_kind} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    again = run()
    for a, c in zip((dx, dg, db), again):
        if a is not None:
            assert torch.equal(a, c)
    monkeypatch.setenv("FLN_BWD_NO_LDS", "1")
    capi.reload_tuning()
    two_pass = run()
    monkeypatch.delenv("FLN_BWD_NO_LDS")
    capi.reload_tuning()
    # dx may differ by one rounding of the output type (row sums in another order): both are
    # within their fp32 allowance of the exact value; the fp32 parameter gradients agree to
    # fp32 summation-order error.
    assert_dx(to_np(dx), to_np(two_pass[0]), 2 * al, ulp_kind, "dx vs two passes")
    for a, c in zip((dg, db), two_pass[1:]):
        if a is not None:
            assert_close_rel(to_np(a), to_np(c), 1e-5, "parameter gradient vs two passes")


@pytest.mark.parametrize("kind,dtype,rows,cols", [
    ("ln", torch.bfloat16, 12, 262144), ("rms", torch.float16, 8, 300000),
    ("ln_dres", torch.float32, 16, 40000), ("gelu_tanh", torch.bfloat16, 8, 131072),
    ("ln", torch.bfloat16, 4, 100003), ("ln", torch.bfloat16, 4, 1048576),
    ("rms", torch.float32, 3, 524288)],
    ids=["ln-bf16-12x262144", "rms-f16-8x300000", "ln_dres-f32-16x40000",
         "gelu_tanh-bf16-8x131072", "ln-bf16-4x100003-scalar", "ln-bf16-4x1048576-one-block-row",
         "rms-f32-3x524288-one-block-row"])
def test_two_pass_backward_few_rows(lib, monkeypatch, kind, dtype, rows, cols):
    """Few very wide rows: the two-pass backward's row statistics split each row into up to 16
    column chunks of whole 2048-vector steps (so the statistics pass has blocks for every CU)
    and the column pass sums a row's splits in order (300000 fp16 columns: 10 chunks of 4096
    vectors, the last one 636; 100003 columns: the scalar path, 13 chunks; 131072 vectors: a
    column pass of one block row, which writes dgamma / dbeta itself).  Parity with the oracle,
    bitwise reproducible, and agreement with one block per row (FLN_BWD_STAT_SPLITS=1)."""
    gen = torch.Generator().manual_seed(cols + rows)
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.2 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy, dr = cuda(xc), cuda(gc), cuda(bc), cuda(dyc), cuda(drc)
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    code = capi.dtype_code(x)
    p = capi.ptr
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, 1e-6)

        def run():
            dx, dw = rms_backward(lib, dy, x, rstd, g)
            return dx, dw, None
        dx_ref, dg_ref = c_oracle.rmsnorm_bwd(dys, xs, gs, 1e-6)
        db_ref = None
    elif kind == "gelu_tanh":
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        y = torch.empty_like(x)
        capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd),
                                                  rows, cols, code, 1e-5, capi.GELU_TANH,
                                                  capi.stream()))

        def run():
            dx = torch.empty_like(x)
            dg = torch.empty(cols, device="cuda")
            db = torch.empty(cols, device="cuda")
            ws, n = workspace(lib, rows, cols, x)
            capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                       p(dx), p(dg), p(db), rows, cols, code,
                                                       capi.F32, capi.GELU_TANH, p(ws), n,
                                                       capi.stream()))
            return dx, dg, db
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, "tanh")
    else:
        _, mean, rstd = ln_forward(lib, x, g, None, 1e-5)
        dres = dr if kind == "ln_dres" else None

        def run():
            return ln_backward(lib, dy, x, mean, rstd, g, dres=dres)
        dx_ref, dg_ref, db_ref = c_oracle.layernorm_bwd(dys, xs, gs, 1e-5)
        if kind == "ln_dres":
            dx_ref = dx_ref + f32(drc)
    dx, dg, db = run()
    torch.cuda.synchronize()
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs, bs, f32(drc)),
              _kind(dtype), f"two-pass {kind} {_kind(dtype)} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    again = run()
    for a, c in zip((dx, dg, db), again):
        if a is not None:
            assert torch.equal(a, c)
    monkeypatch.setenv("FLN_BWD_STAT_SPLITS", "1")
    capi.reload_tuning()
    one = run()
    monkeypatch.delenv("FLN_BWD_STAT_SPLITS")
    capi.reload_tuning()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10 if dtype == torch.float16 else 1e-5
    af, cf = dx.float(), one[0].float()
    assert float((af - cf).abs().max()) <= 2 * ulp * max(1.0, float(cf.abs().max()))
    for a, c in zip((dg, db), one[1:]):
        if a is not None:
            assert_close_rel(to_np(a), to_np(c), 1e-5, "parameter gradient vs one block per row")


@pytest.mark.parametrize("kind", ["ln", "rms", "ln_dres", "gelu_none", "gelu_tanh"])
@pytest.mark.parametrize("dtype,cols", [(torch.float32, 20480), (torch.bfloat16, 24576),
                                        (torch.float16, 40000), (torch.bfloat16, 20001)],
                         ids=["f32-20480", "bf16-24576", "f16-40000", "bf16-20001-scalar"])
def test_two_pass_backward(lib, monkeypatch, kind, dtype, cols):
    """Rows past the register and LDS tiles take the two-pass backward (row statistics, then a
    column pass over row chunks; 257 rows: several chunks): parity with the oracle for every
    flavour, bitwise reproducible, and agreement with the looped kernel, which is also what a
    dx-only call without a workspace uses."""
    rows = 257
    gen = torch.Generator().manual_seed(cols + 11 * len(kind))
    xc = (torch.randn(rows, cols, generator=gen) * 2 + 0.5).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.2 * torch.randn(cols, generator=gen)).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    drc = torch.randn(rows, cols, generator=gen).to(dtype)
    x, g, b, dy, dr = cuda(xc), cuda(gc), cuda(bc), cuda(dyc), cuda(drc)
    xs, gs, bs, dys = f32(xc), f32(gc), f32(bc), f32(dyc)
    code = capi.dtype_code(x)
    p = capi.ptr
    if kind == "rms":
        _, rstd = rms_forward(lib, x, g, 1e-6)
        mean = None
    else:
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        y = torch.empty_like(x)
        if kind.startswith("gelu"):
            gm = capi.GELU_ERF if kind == "gelu_none" else capi.GELU_TANH
            capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd),
                                                      rows, cols, code, 1e-5, gm, capi.stream()))
        else:
            capi.check(lib.fln_layernorm_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                                 cols, code, 1e-5, capi.stream()))

    def run(params=True, with_ws=True):
        dx = torch.empty_like(x)
        dg = torch.empty(cols, device="cuda") if params else None
        db = torch.empty(cols, device="cuda") if params and kind != "rms" else None
        ws, n = workspace(lib, rows, cols, x)
        wsp, wsn = (p(ws), n) if with_ws else (None, 0)
        if kind == "rms":
            capi.check(lib.fln_rmsnorm_backward(p(dy), p(x), p(rstd), p(g), None, p(dx), p(dg),
                                                rows, cols, code, capi.F32, wsp, wsn,
                                                capi.stream()))
        elif kind.startswith("gelu"):
            capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                       p(dx), p(dg), p(db), rows, cols, code,
                                                       capi.F32, gm, wsp, wsn, capi.stream()))
        else:
            capi.check(lib.fln_layernorm_backward(p(dy), p(x), p(mean), p(rstd), p(g),
                                                  p(dr) if kind == "ln_dres" else None, p(dx),
                                                  p(dg), p(db), rows, cols, code, capi.F32, wsp,
                                                  wsn, capi.stream()))
        torch.cuda.synchronize()
        return dx, dg, db

    dx, dg, db = run()
    if kind == "rms":
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, 1e-6)
    elif kind.startswith("gelu"):
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, kind[5:])
    else:
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
        if kind == "ln_dres":
            dx_ref = dx_ref + f32(drc)
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs, bs, f32(drc)),
              _kind(dtype), f"two-pass {kind} {_kind(dtype)} {rows}x{cols} dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, "dgamma")
    if db is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, "dbeta")
    again = run()
    for a, c in zip((dx, dg, db), again):
        if a is not None:
            assert torch.equal(a, c)
    monkeypatch.setenv("FLN_BWD_NO_TWO_PASS", "1")
    capi.reload_tuning()
    looped = run()
    monkeypatch.delenv("FLN_BWD_NO_TWO_PASS")
    capi.reload_tuning()
    dx_nows, _, _ = run(params=False, with_ws=False)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10 if dtype == torch.float16 else 1e-5
    for a, c in zip((dx, dg, db, dx), looped + (dx_nows,)):
        if a is not None:
            af, cf = a.float(), c.float()
            assert float((af - cf).abs().max()) <= 2 * ulp * max(1.0, float(cf.abs().max()))


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(3, 12288), (5, 16384), (2, 32768), (4, 20480),
                                       (3, 40960), (300, 65536)])
def test_add_layernorm_wide_rows(lib, dtype, rows, cols):
    """Residual add + LayerNorm on rows of 12 to 16 waves and on the widest register tiles: h
    is the rounded sum, y the LayerNorm of h (same bar as the plain forward)."""
    gen = torch.Generator().manual_seed(rows * 17 + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, r, g, b = cuda(xc), cuda(rc), cuda(gc), cuda(bc)
    h, y = torch.empty_like(x), torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    p = capi.ptr
    capi.check(lib.fln_add_layernorm_forward(p(x), p(r), p(g), p(b), p(h), p(y), p(mean), p(rstd),
                                             rows, cols, capi.dtype_code(x), 1e-5, capi.stream()))
    torch.cuda.synchronize()
    h_ref = (xc.float() + rc.float()).to(dtype)
    assert torch.equal(h.cpu(), h_ref)
    hs = f32(h_ref)
    y_ref, _, _ = norms.layer_norm_fwd(hs, f32(gc), f32(bc), 1e-5)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - y_ref).max() <= 1e-5 * max(1, np.abs(y_ref).max())
    else:
        assert_within_ulp(to_np(y), y_ref, 1.0, atol=affine_atol(hs, f32(gc), f32(bc), 1e-5),
                          **_tol_fwd(dtype), what="y")


def test_add_rmsnorm_bf16(lib):
    gen = torch.Generator().manual_seed(21)
    xc = torch.randn(300, 4096, generator=gen).to(torch.bfloat16)
    rc = torch.randn(300, 4096, generator=gen).to(torch.bfloat16)
    wc = (1 + 0.02 * torch.randn(4096, generator=gen)).to(torch.bfloat16)
    x, r, wt = cuda(xc), cuda(rc), cuda(wc)
    y, h = torch.empty_like(x), torch.empty_like(x)
    rstd = torch.empty(300, device="cuda")
    capi.check(lib.fln_add_rmsnorm_forward(capi.ptr(x), capi.ptr(r), capi.ptr(wt), capi.ptr(h),
                                           capi.ptr(y), capi.ptr(rstd), 300, 4096, capi.BF16,
                                           1e-6, capi.stream()))
    assert torch.equal(h.cpu(), xc + rc)
    y_ref, h_ref, _ = norms.add_rms_norm_fwd(f32(xc), f32(rc), f32(wc), 1e-6, "bf16")
    assert_within_ulp(to_np(y), y_ref, 1.0, what="add_rms y")


def test_looped_fallback_matches_register_path(lib, monkeypatch):
    gen = torch.Generator().manual_seed(3)
    xc = torch.randn(40, 3072, generator=gen)
    gc = 1 + 0.1 * torch.randn(3072, generator=gen)
    x, g = cuda(xc), cuda(gc)
    y_reg, m_reg, r_reg = ln_forward(lib, x, g, g, 1e-5)
    monkeypatch.setenv("FLN_FORCE_LOOP", "1")
    capi.reload_tuning()
    y_loop, m_loop, r_loop = ln_forward(lib, x, g, g, 1e-5)
    monkeypatch.delenv("FLN_FORCE_LOOP")
    capi.reload_tuning()
    ref, _, _ = norms.layer_norm_fwd(xc.numpy(), gc.numpy(), gc.numpy(), 1e-5)
    assert np.abs(to_np(y_loop) - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.abs(to_np(y_reg) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_float64_forward(lib):
    gen = torch.Generator().manual_seed(4)
    xc = torch.randn(10, 777, generator=gen, dtype=torch.float64)
    gc = 1 + 0.1 * torch.randn(777, generator=gen, dtype=torch.float64)
    x, g = cuda(xc), cuda(gc)  # keep the device tensors alive across the launch
    y = torch.empty(10, 777, device="cuda", dtype=torch.float64)
    capi.check(lib.fln_layernorm(capi.ptr(x), capi.ptr(g), capi.ptr(g), capi.ptr(y), 10, 777,
                                 capi.F64, 1e-5, capi.stream()))
    ref, _, _ = norms.layer_norm_fwd(xc.numpy(), gc.numpy(), gc.numpy(), 1e-5)
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-12


def test_invalid_arguments_are_rejected_before_launch(lib):
    x = torch.zeros(4, 8, device="cuda")
    y = torch.empty_like(x)
    s = capi.stream()
    assert lib.fln_layernorm(capi.ptr(x), None, None, capi.ptr(y), -1, 8, capi.F32, 1e-5, s) == 1
    assert lib.fln_layernorm(None, None, None, capi.ptr(y), 4, 8, capi.F32, 1e-5, s) == 1
    assert lib.fln_layernorm(capi.ptr(x), None, None, capi.ptr(y), 4, 8, 99, 1e-5, s) == 1
    assert lib.fln_layernorm_gelu(capi.ptr(x), None, None, capi.ptr(y), 4, 8, capi.F32, 1e-5, 7,
                                  s) == 1
    mean = torch.zeros(4, device="cuda")
    dg = torch.empty(8, device="cuda")
    # dgamma requested without a workspace
    assert lib.fln_layernorm_backward(capi.ptr(x), capi.ptr(x), capi.ptr(mean), capi.ptr(mean),
                                      None, None, None, capi.ptr(dg), None, 4, 8, capi.F32,
                                      capi.F32, None, 0, s) == 1
    assert lib.fln_layernorm(capi.ptr(x), None, None, capi.ptr(y), 0, 8, capi.F32, 1e-5, s) == 0


# ------------------------------------------------------------------------------------------------
# The reference's own accuracy scenarios, through fln_layernorm (the reference's `layernorm`
# entry): its value ranges at 32 x 4096 with nn.LayerNorm's default affine (gamma 1, beta 0)
# (tests/publication_validation.py:205-214), its normalization check (:242-253) and its
# "wrong epsilon" case eps = 1e-12 (tests/break_kernel_test.py:39-41).  fp32 outputs against the
# float64 oracle at max-abs 1e-5; bf16 outputs within 1 bf16 ulp of it.
# ------------------------------------------------------------------------------------------------
def _reference_scenario(name, seed=2024):
    gen = torch.Generator().manual_seed(seed)
    if name == "mixed_range":  # half the row x1000, half x1e-3
        return torch.cat([torch.randn(32, 2048, generator=gen) * 1000,
                          torch.randn(32, 2048, generator=gen) * 1e-3], dim=1)
    scale = {"normal": 1.0, "large_values": 1000.0, "small_values": 1e-3, "near_zero": 1e-6}[name]
    return torch.randn(32, 4096, generator=gen) * scale


def _ln_plain(lib, x, eps):
    rows, cols = x.shape
    y = torch.empty_like(x)
    g = torch.ones(cols, dtype=x.dtype, device=x.device)
    b = torch.zeros(cols, dtype=x.dtype, device=x.device)
    capi.check(lib.fln_layernorm(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y), rows, cols,
                                 capi.dtype_code(x), eps, capi.stream()))
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("scenario", ["normal", "large_values", "small_values", "near_zero",
                                      "mixed_range"])
def test_reference_accuracy_scenarios(lib, scenario, dtype):
    xc = _reference_scenario(scenario).to(dtype)
    y = _ln_plain(lib, cuda(xc), 1e-5)
    ref, _, _ = norms.layer_norm_fwd(f32(xc), None, None, 1e-5)
    assert np.isfinite(to_np(y)).all()
    if dtype == torch.float32:
        err = np.abs(to_np(y) - ref).max()
        assert err <= 1e-5, f"{scenario}: max abs error {err:.3g}"
        # The reference publishes 4.77e-7 max-abs against nn.LayerNorm for the normal case
        # (publication_validation_results.json:176-182); torch's own fp32 kernel sits there too.
        ref_t = torch.nn.functional.layer_norm(xc, (4096,), None, None, 1e-5)
        assert (y.cpu() - ref_t).abs().max().item() <= 1e-5
    else:
        assert_within_ulp(to_np(y), ref, 1.0, what=f"{scenario} y")


def test_reference_normalization_check(lib):
    # publication_validation.py:242-253: with gamma 1 and beta 0 every row of the output has
    # mean 0 (|mean| < 1e-5) and biased std 1 (|std - 1| < 1e-3).
    gen = torch.Generator().manual_seed(7)
    x = cuda(torch.randn(32, 4096, generator=gen))
    y = _ln_plain(lib, x, 1e-5).double().cpu()
    assert y.mean(dim=-1).abs().max().item() < 1e-5
    assert (y.std(dim=-1, unbiased=False) - 1.0).abs().max().item() < 1e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("scenario", ["normal", "near_zero"])
def test_reference_epsilon_1e12(lib, scenario, dtype):
    # break_kernel_test.py:39-41 calls layernorm with eps = 1e-12.  With the near-zero rows
    # (variance ~1e-12) eps is no longer negligible against the variance: both terms matter.
    xc = _reference_scenario(scenario, seed=99).to(dtype)
    y = _ln_plain(lib, cuda(xc), 1e-12)
    ref, _, _ = norms.layer_norm_fwd(f32(xc), None, None, 1e-12)
    if dtype == torch.float32:
        assert np.abs(to_np(y) - ref).max() <= 1e-5
    else:
        assert_within_ulp(to_np(y), ref, 1.0, what=f"{scenario} eps=1e-12 y")


def _random_cases(n=240, seed=20261202):
    """Seeded shapes for test_random_shapes_against_the_oracle: the flavour cycles, the dtype is
    drawn, rows are log-uniform in 1..16384 and columns log-uniform in 1..70000; a third of the
    widths are rounded down to whole 16-byte vectors (of the 16-bit types), a third to 32-element
    blocks, the rest stay as drawn (the scalar path); at most 4 M elements per case.  Every fifth
    case passes x one element past a 16-byte boundary (the scalar path at any width)."""
    rng = np.random.default_rng(seed)
    kinds = ["ln", "rms", "gelu_tanh", "gelu_none", "add_ln", "ln_fp8", "add_rms_mx", "ln_dres",
             "add_rms", "rms_fp8", "add_ln_fp8", "ln_mx"]
    cases = []
    for i in range(n):
        kind = kinds[i % len(kinds)]
        dtype = DTYPES[int(rng.integers(3))]
        rows = int(np.exp(rng.uniform(0.0, np.log(16384.0))))
        cols = int(np.exp(rng.uniform(0.0, np.log(70000.0))))
        shape = int(rng.integers(3))
        if kind in ("add_rms_mx", "ln_mx") or shape == 1:
            cols = max(32, cols // 32 * 32)
        elif shape == 0:
            cols = max(8, cols // 8 * 8)
        rows = max(1, min(rows, 4_000_000 // cols))
        cases.append((kind, dtype, rows, cols, i % 5 == 4))
    return cases


RANDOM_CASES = _random_cases()


@pytest.mark.parametrize("kind,dtype,rows,cols,shifted", RANDOM_CASES,
                         ids=[f"{i}-{k}-{str(d)[6:]}-{r}x{c}{'-shifted' if sh else ''}"
                              for i, (k, d, r, c, sh) in enumerate(RANDOM_CASES)])
def test_random_shapes_against_the_oracle(lib, kind, dtype, rows, cols, shifted):
    """Seeded random shapes through whatever route the dispatcher picks for them (register
    tiles, odd tiles, LDS-staged, split, streamed, scalar path; the register, LDS and two-pass
    backwards): LayerNorm, RMSNorm and LN + GELU (both forms) forward and backward, the
    LayerNorm backward with a residual gradient, residual + LayerNorm / RMSNorm, LN -> fp8,
    RMSNorm -> fp8, residual + LN -> fp8, LN -> MXFP8 and residual + RMSNorm -> MXFP8 forwards,
    each against the oracle's bar for its dtype."""
    gen = torch.Generator().manual_seed(rows * 65537 + cols)
    xc = (torch.randn(rows, cols, generator=gen) * 1.5 + 0.25).to(dtype)
    rc = torch.randn(rows, cols, generator=gen).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    x, r, dy, g, b = cuda(xc), cuda(rc), cuda(dyc), cuda(gc), cuda(bc)
    if shifted:  # x one element past a 16-byte boundary
        xbuf = torch.empty(rows * cols + 1, dtype=dtype, device="cuda")
        xbuf[1:] = x.flatten()
        x = xbuf[1:].view(rows, cols)
    xs, rs, dys, gs, bs = f32(xc), f32(rc), f32(dyc), f32(gc), f32(bc)
    io = _kind(dtype)
    p = capi.ptr
    code = capi.dtype_code(x)
    what = f"{kind} {io} {rows}x{cols}{' shifted' if shifted else ''}"

    def check_y(y, y_ref, xin, bias=True, approximate=None):
        al = affine_atol(xin, gs, bs, 1e-5, approximate) if bias else 0.0
        if dtype == torch.float32:
            bar = 1e-5 * max(1.0, np.abs(y_ref).max()) + al
            assert (np.abs(to_np(y) - y_ref) <= bar).all(), what
        else:
            assert_within_ulp(to_np(y), y_ref, 1.0, atol=al, kind=io, what=what + " y")

    def check_h(h):
        assert np.array_equal(to_np(h), to_np(xc + rc)), what + " h bit-exact"

    if kind in ("ln", "ln_dres"):
        y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
        dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g, dres=r if kind == "ln_dres" else None)
        y_ref, m_ref, r_ref = norms.layer_norm_fwd(xs, gs, bs, 1e-5)
        check_y(y, y_ref, xs)
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5, what + " rstd"
        dx_ref, dg_ref, db_ref = norms.layer_norm_bwd(dys, xs, gs, 1e-5)
        if kind == "ln_dres":
            dx_ref = dx_ref + rs
    elif kind == "rms":
        y, rstd = rms_forward(lib, x, g, 1e-6)
        dx, dg = rms_backward(lib, dy, x, rstd, g)
        db = None
        y_ref, r_ref = norms.rms_norm_fwd(xs, gs, 1e-6)
        check_y(y, y_ref, xs, bias=False)
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5, what + " rstd"
        dx_ref, dg_ref = norms.rms_norm_bwd(dys, xs, gs, 1e-6)
        db_ref = None
    elif kind.startswith("gelu"):
        form = kind[5:]
        gm = capi.GELU_ERF if form == "none" else capi.GELU_TANH
        y = torch.empty_like(x)
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                                  cols, code, 1e-5, gm, capi.stream()))
        dx = torch.empty_like(x)
        dg = torch.empty(cols, device="cuda")
        db = torch.empty(cols, device="cuda")
        ws, n = workspace(lib, rows, cols, x)
        capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                   p(dx), p(dg), p(db), rows, cols, code,
                                                   capi.F32, gm, p(ws), n, capi.stream()))
        check_y(y, norms.layer_norm_gelu_fwd(xs, gs, bs, 1e-5, form), xs, approximate=form)
        dx_ref, dg_ref, db_ref = norms.layer_norm_gelu_bwd(dys, xs, gs, bs, 1e-5, form)
    elif kind == "add_ln":
        h = torch.empty_like(x)
        y = torch.empty_like(x)
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        capi.check(lib.fln_add_layernorm_forward(p(x), p(r), p(g), p(b), p(h), p(y), p(mean),
                                                 p(rstd), rows, cols, code, 1e-5, capi.stream()))
        check_h(h)
        y_ref, h_ref, _, r_ref = norms.add_layer_norm_fwd(xs, rs, gs, bs, 1e-5, io)
        check_y(y, y_ref, h_ref)
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5, what + " rstd"
        return
    elif kind == "add_rms":
        h = torch.empty_like(x)
        y = torch.empty_like(x)
        rstd = torch.empty(rows, device="cuda")
        capi.check(lib.fln_add_rmsnorm_forward(p(x), p(r), p(g), p(h), p(y), p(rstd), rows, cols,
                                               code, 1e-6, capi.stream()))
        check_h(h)
        y_ref, h_ref, r_ref = norms.add_rms_norm_fwd(xs, rs, gs, 1e-6, io)
        check_y(y, y_ref, h_ref, bias=False)
        assert np.abs(to_np(rstd) / r_ref - 1).max() <= 1e-5, what + " rstd"
        return
    elif kind in ("rms_fp8", "add_ln_fp8"):
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        s = torch.empty(rows, device="cuda")
        if kind == "rms_fp8":
            capi.check(lib.fln_rmsnorm_fp8_forward(p(x), p(g), p(q), p(s), None, rows, cols, code,
                                                   1e-6, capi.stream()))
            q_ref, s_ref = c_oracle.rmsnorm_fp8(xs, gs, 1e-6)
            t_ref = _scaled(norms.rms_norm_fwd(xs, gs, 1e-6)[0])
            s_atol = None
        else:
            h = torch.empty_like(x)
            capi.check(lib.fln_add_layernorm_fp8_forward(p(x), p(r), p(g), p(b), p(h), p(q), p(s),
                                                         None, None, rows, cols, code, 1e-5,
                                                         capi.stream()))
            check_h(h)
            q_ref, s_ref, h_ref = norms.add_layer_norm_fp8_fwd(xs, rs, gs, bs, 1e-5, io)
            t_ref = _scaled(norms.layer_norm_fwd(h_ref, gs, bs, 1e-5)[0])
            s_atol = affine_atol(h_ref, gs, bs, 1e-5).max(axis=1) / 448.0
        assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, what, t_ref=t_ref, s_atol=s_atol)
        return
    elif kind == "ln_mx":
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        sc = torch.empty(rows, cols // 32, device="cuda", dtype=torch.uint8)
        capi.check(_mx_call(lib, "ln", x, r, g, b, q, sc, None, rows, cols, code))
        q_ref, sc_ref, y_ref = _mx_ref("ln", xs, rs, gs, bs, io)
        assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, sc_ref, y_ref, what)
        return
    elif kind == "ln_fp8":
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        s = torch.empty(rows, device="cuda")
        capi.check(lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(s), None, None, rows,
                                                 cols, code, 1e-5, capi.stream()))
        q_ref, s_ref = c_oracle.layernorm_fp8(xs, gs, bs, 1e-5)
        assert_fp8_close(q.cpu().numpy(), to_np(s), q_ref, s_ref, what,
                         t_ref=_scaled(norms.layer_norm_fwd(xs, gs, bs, 1e-5)[0]),
                         s_atol=affine_atol(xs, gs, bs, 1e-5).max(axis=1) / 448.0)
        return
    else:
        h = torch.empty_like(x)
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        sc = torch.empty(rows, cols // 32, device="cuda", dtype=torch.uint8)
        capi.check(_mx_call(lib, "add_rms", x, r, g, b, q, sc, h, rows, cols, code))
        check_h(h)
        q_ref, sc_ref, y_ref = _mx_ref("add_rms", xs, rs, gs, bs, io)
        assert_mx_close(q.cpu().numpy(), sc.cpu().numpy(), q_ref, sc_ref, y_ref, what)
        return
    assert_dx(to_np(dx), dx_ref, _flavour_allowance(kind, xs, dys, gs, bs, rs), io, what + " dx")
    assert_close_rel(to_np(dg), dg_ref, 1e-4, what + " dgamma")
    if db_ref is not None:
        assert_close_rel(to_np(db), db_ref, 1e-4, what + " dbeta")


NONFINITE_CASES = [(4096, 4096, torch.bfloat16), (1024, 3072, torch.bfloat16),
                   (64, 40960, torch.bfloat16), (8, 65536, torch.float32), (100, 1023, torch.float16),
                   (300, 768, torch.float32), (400, 131072, torch.bfloat16)]


@pytest.mark.parametrize("rows,cols,dtype", NONFINITE_CASES,
                         ids=[f"{r}x{c}-{str(d)[6:]}" for r, c, d in NONFINITE_CASES])
@pytest.mark.parametrize("op", ["ln", "rms", "ln_fp8", "rms_mx"])
def test_non_finite_inputs_stay_in_their_rows(lib, op, rows, cols, dtype):
    """A NaN in row 3 and an infinity in row 5 (register tiles, odd tiles, the LDS-staged,
    streamed and split forwards, the scalar path): every other row's outputs are bitwise those of
    the same call without them, the call reports no error, and rows 3 and 5 are what the float64
    oracle makes of them.  LayerNorm: an infinity makes the mean infinite and every centred value
    NaN or infinite, so y is NaN throughout.  RMSNorm: an infinity makes rstd 0, so y is zero but
    NaN (inf * 0) at the infinity.  Both rows' statistics are unusable (oracle.norms.unusable_rows),
    so their fp8 row scale is NaN (torch's amax of y gives the same) and every MX block scale of
    theirs 0xFF, E8M0's NaN."""
    if op == "rms_mx" and cols % 32:
        pytest.skip("MX blocks need a multiple of 32 columns")
    gen = torch.Generator().manual_seed(rows + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bad = xc.clone()
    r5 = min(5, rows - 1)
    bad[3, cols // 3] = float("nan")
    bad[r5, cols - 1] = float("inf")
    g, b = cuda(gc), cuda(bc)
    p = capi.ptr
    code = capi.dtype_code(g)

    def run(xh):
        x = cuda(xh)
        if op == "ln":
            y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
            return [y.float().cpu(), torch.stack([mean, rstd], 1).cpu()]
        if op == "rms":
            y, rstd = rms_forward(lib, x, g, 1e-6)
            return [y.float().cpu(), rstd[:, None].cpu()]
        q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
        if op == "ln_fp8":
            s = torch.empty(rows, device="cuda")
            capi.check(lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(s), None, None,
                                                     rows, cols, code, 1e-5, capi.stream()))
            return [q.cpu(), s[:, None].cpu()]
        sc = torch.empty(rows, cols // 32, device="cuda", dtype=torch.uint8)
        capi.check(lib.fln_rmsnorm_mxfp8_forward(p(x), p(g), p(q), p(sc), None, rows, cols,
                                                 code, 1e-6, capi.stream()))
        return [q.cpu(), sc.cpu()]

    clean, dirty = run(xc), run(bad)
    torch.cuda.synchronize()
    keep = torch.ones(rows, dtype=torch.bool)
    keep[3] = keep[r5] = False
    for c_out, d_out in zip(clean, dirty):
        assert torch.equal(c_out[keep], d_out[keep]), f"{op}: a clean row changed"
    rr = [3, r5]
    xs, gs, bs = bad[rr].double().numpy(), gc.double().numpy(), bc.double().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        if op == "ln":
            y_ref = norms.layer_norm_fwd(xs, gs, bs, 1e-5)[0]
        elif op == "rms":
            y_ref = norms.rms_norm_fwd(xs, gs, 1e-6)[0]
        elif op == "ln_fp8":
            s_ref = norms.layer_norm_fp8_fwd(xs, gs, bs, 1e-5)[1]
        else:
            q_ref, sc_ref = norms.rms_norm_mxfp8_fwd(xs, gs, 1e-6)
    if op in ("ln", "rms"):
        y = dirty[0][rr]
        assert torch.equal(y.isnan(), torch.from_numpy(np.isnan(y_ref))), op
        assert torch.equal(y[~y.isnan()].double(), torch.from_numpy(y_ref[~np.isnan(y_ref)])), op
        if op == "ln":  # rstd NaN for both rows; the mean NaN or infinite
            assert torch.isnan(dirty[1][rr][:, 1]).all(), (op, dirty[1][rr])
            assert not torch.isfinite(dirty[1][rr][:, 0]).any(), (op, dirty[1][rr])
        else:           # rstd NaN for the NaN row, 1 / sqrt(inf) = 0 for the infinity's
            assert torch.isnan(dirty[1][3, 0]) and dirty[1][r5, 0] == 0, (op, dirty[1][rr])
    elif op == "ln_fp8":
        assert np.isnan(s_ref).all() and torch.isnan(dirty[1][rr]).all(), (op, dirty[1][rr])
    else:
        assert np.array_equal(dirty[1][rr].numpy(), sc_ref), (dirty[1][rr], sc_ref)
        live = np.repeat(sc_ref != 0xFF, 32, axis=1)  # blocks under a NaN scale are NaN anyway
        got, want = dirty[0][rr].numpy()[live], q_ref[live]
        # the zeros of the infinity's row: +0 or -0 codes (0x00 / 0x80) read as the same zero
        assert np.array_equal(norms.fp8_e4m3fn_decode(got), norms.fp8_e4m3fn_decode(want)), \
            (op, np.unique(got), np.unique(want))

NONFINITE_BWD_CASES = [(4096, 4096, torch.bfloat16), (64, 40960, torch.bfloat16),
                       (100, 1023, torch.float16), (300, 768, torch.float32)]


@pytest.mark.parametrize("rows,cols,dtype", NONFINITE_BWD_CASES,
                         ids=[f"{r}x{c}-{str(d)[6:]}" for r, c, d in NONFINITE_BWD_CASES])
@pytest.mark.parametrize("op", ["ln", "rms"])
def test_non_finite_rows_in_the_backward(lib, op, rows, cols, dtype):
    """The backward of a batch with a NaN in row 3 and an infinity in row 5, fed the forward's
    own statistics: dx of every other row is bitwise that of the clean batch; dx of rows 3 and 5
    is NaN wherever the float64 oracle's is; dγ / dw is NaN in every column (row 3's x̂ is NaN
    throughout) while dβ, a plain sum of dy, is bitwise the clean batch's (the non-finite rows
    leak into no other reduction)."""
    gen = torch.Generator().manual_seed(3 * rows + cols)
    xc = torch.randn(rows, cols, generator=gen).to(dtype)
    dyc = torch.randn(rows, cols, generator=gen).to(dtype)
    gc = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bc = (0.1 * torch.randn(cols, generator=gen)).to(dtype)
    bad = xc.clone()
    r5 = min(5, rows - 1)
    bad[3, cols // 3] = float("nan")
    bad[r5, cols - 1] = float("inf")
    g, b, dy = cuda(gc), cuda(bc), cuda(dyc)
    print(f"[non-finite bwd] {op} {rows}x{cols} {dtype}", flush=True)

    def run(xh):
        x = cuda(xh)
        if op == "ln":
            _, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
            dx, dg, db = ln_backward(lib, dy, x, mean, rstd, g)
            return dx.float().cpu(), dg.cpu(), db.cpu()
        _, rstd = rms_forward(lib, x, g, 1e-6)
        dx, dw = rms_backward(lib, dy, x, rstd, g)
        return dx.float().cpu(), dw.cpu(), None

    (dxc, dgc, dbc), (dxd, dgd, dbd) = run(xc), run(bad)
    torch.cuda.synchronize()
    keep = torch.ones(rows, dtype=torch.bool)
    keep[3] = keep[r5] = False
    assert torch.equal(dxc[keep], dxd[keep]), f"{op}: dx of a clean row changed"
    rr = [3, r5]
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        if op == "ln":
            dx_ref = norms.layer_norm_bwd(dyc[rr].double().numpy(), bad[rr].double().numpy(),
                                          gc.double().numpy(), 1e-5)[0]
        else:
            dx_ref = norms.rms_norm_bwd(dyc[rr].double().numpy(), bad[rr].double().numpy(),
                                        gc.double().numpy(), 1e-6)[0]
    assert torch.equal(dxd[rr].isnan(), torch.from_numpy(np.isnan(dx_ref))), op
    assert torch.isnan(dgd).all(), (op, dgd)
    if op == "ln":
        assert torch.equal(dbc, dbd), "dβ changed"
