"""GPU tests of the reference-facing API: the `fused_layernorm` package (modules, autograd,
functional ops, torch.compile) and the `fused_layernorm_cuda` binding.

The plan follows the reference's tests/test_layernorm.py (forward over its batch/hidden/dtype
list, 3-D input, no affine, backward, gradient accumulation, epsilon sweep, extreme values,
memory, functional interface, determinism, edge cases) and tests/edge_cases.py (its size list),
but every expectation here is PyTorch on the CPU in float64 rather than PyTorch on the same GPU.
Tolerances: fp32 forward max-abs 1e-5 (the reference's own rtol/atol 1e-5); fp32 gradients
rtol = atol = 1e-4 (the reference's grad tolerances); bf16/fp16 outputs within 1 ulp of the
float64 result plus, where y cancels, the fp32 evaluation allowance of y
(oracle.tolerance.y_allowance: the affine step's roundings and the fp32 row mean's shift of x̂).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from helpers import assert_fp8_close, assert_within_ulp, to_np
from oracle import norms, tolerance

import fused_layernorm as fl
import fused_layernorm_cuda

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu(gpu_available):
    torch.manual_seed(0)


def ref_ln(x, shape, w=None, b=None, eps=1e-5):
    """float64 CPU LayerNorm."""
    f = lambda t: None if t is None else t.detach().double().cpu()
    return F.layer_norm(f(x), shape, f(w), f(b), eps)


def check_out(y, ref, dtype, x=None, w=None, b=None, eps=1e-5, shape=None):
    got, r = to_np(y).astype(np.float64), ref.numpy()
    if dtype == torch.float32:
        assert np.abs(got - r).max() <= 1e-5
        return
    atol = 0.0
    if x is not None:
        atol = tolerance.y_allowance(to_np(x), None if w is None else to_np(w),
                                     None if b is None else to_np(b), eps)
    assert_within_ulp(got, r, 1.0, atol=atol, kind="bf16" if dtype == torch.bfloat16 else "f16",
                      what="y")


def make_ln(hidden, dtype=torch.float32, affine=True, bias=True):
    ln = fl.FusedLayerNorm(hidden, elementwise_affine=affine, bias=bias).to(DEV, dtype)
    if affine:
        with torch.no_grad():
            ln.weight.copy_(1 + 0.1 * torch.randn(hidden))
            if ln.bias is not None:
                ln.bias.copy_(0.1 * torch.randn(hidden))
    return ln


# ------------------------------------------------------------------------------------------------
# The reference's test plan.
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("batch,hidden,dtype", [
    (1, 768, torch.float32), (8, 768, torch.float32), (32, 1024, torch.float32),
    (64, 2048, torch.float32), (128, 4096, torch.float32), (1, 768, torch.float16),
    (32, 1024, torch.float16), (64, 2048, torch.float16), (32, 1024, torch.bfloat16),
    (128, 4096, torch.bfloat16)])
def test_forward_correctness(batch, hidden, dtype):
    x = torch.randn(batch, hidden, device=DEV, dtype=dtype)
    ln = make_ln(hidden, dtype)
    y = ln(x)
    assert y.dtype == dtype and y.shape == x.shape
    check_out(y, ref_ln(x, (hidden,), ln.weight, ln.bias), dtype, x, ln.weight, ln.bias,
              shape=(hidden,))


@pytest.mark.parametrize("batch,seq,hidden", [(2, 128, 768), (4, 256, 1024), (8, 512, 2048),
                                              (1, 1024, 4096)])
def test_3d_input(batch, seq, hidden):
    x = torch.randn(batch, seq, hidden, device=DEV)
    ln = make_ln(hidden)
    y = ln(x)
    assert y.shape == x.shape
    check_out(y, ref_ln(x, (hidden,), ln.weight, ln.bias), torch.float32)


@pytest.mark.parametrize("hidden,affine", [(768, True), (768, False), (1024, True),
                                           (1024, False)])
def test_no_affine_parameters(hidden, affine):
    x = torch.randn(16, hidden, device=DEV)
    ln = make_ln(hidden, affine=affine)
    assert (ln.weight is None) == (not affine)
    check_out(ln(x), ref_ln(x, (hidden,), ln.weight, ln.bias), torch.float32)


def _grads_f64(x, w, b, dy, shape, eps=1e-5):
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = None if w is None else w.detach().double().cpu().requires_grad_(True)
    bd = None if b is None else b.detach().double().cpu().requires_grad_(True)
    F.layer_norm(xd, shape, wd, bd, eps).backward(dy.double().cpu())
    return xd.grad, None if w is None else wd.grad, None if b is None else bd.grad


@pytest.mark.parametrize("batch,hidden", [(16, 768), (32, 1024), (64, 2048)])
def test_backward_correctness(batch, hidden):
    x = torch.randn(batch, hidden, device=DEV, requires_grad=True)
    ln = make_ln(hidden)
    dy = torch.randn(batch, hidden, device=DEV)
    ln(x).backward(dy)
    gx, gw, gb = _grads_f64(x, ln.weight, ln.bias, dy, (hidden,))
    for got, ref in ((x.grad, gx), (ln.weight.grad, gw), (ln.bias.grad, gb)):
        torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("shape,dtype,affine,bias", [
    ((32, 768), torch.float32, True, True), ((4, 9, 1024), torch.bfloat16, True, True),
    ((2, 3, 5, 2048), torch.float16, True, False), ((4096,), torch.float32, False, False),
    ((64, 4096), torch.bfloat16, True, True)],
    ids=["2d-f32", "3d-bf16", "4d-f16-nobias", "1d-f32-noaffine", "2d-bf16"])
@pytest.mark.parametrize("grads", ["all", "params", "input"])
def test_module_eager_path_matches_the_autograd_function(shape, dtype, affine, bias, grads):
    """FusedLayerNorm's eager forward runs autograd in C++ (fused_layernorm_cuda.
    layer_norm_autograd) instead of the Python FusedLayerNormFunction + operator call: the same
    kernels, so output and every gradient are bitwise identical to the Python path
    (FusedLayerNormFunction on the rows), for any rank, with or without affine parameters,
    for each combination of tensors requiring grad, and on a non-contiguous input."""
    hidden = shape[-1]
    ln = make_ln(hidden, dtype, affine=affine, bias=bias)
    base = torch.randn(*shape[:-1], 2 * hidden, device=DEV).to(dtype)
    x = base[..., ::2]  # non-contiguous
    dy = torch.randn(shape, device=DEV).to(dtype)
    need_x = grads in ("all", "input")
    for p in ln.parameters():
        p.requires_grad_(grads in ("all", "params"))
    xa = x.detach().clone().requires_grad_(need_x)
    ya = ln(xa)
    assert ya.requires_grad == (need_x or (affine and grads in ("all", "params")))
    if ya.requires_grad:
        ya.backward(dy)
    ga = [t.grad.clone() if t is not None and t.grad is not None else None
          for t in (xa, ln.weight, ln.bias)]
    for p in ln.parameters():
        p.grad = None
    xb = x.detach().contiguous().reshape(-1, hidden).requires_grad_(need_x)
    yb = fl.FusedLayerNormFunction.apply(xb, (hidden,), ln.weight, ln.bias, ln.eps)
    if yb.requires_grad:
        yb.backward(dy.reshape(-1, hidden))
    gb = [xb.grad.reshape(shape) if xb.grad is not None else None,
          ln.weight.grad if ln.weight is not None else None,
          ln.bias.grad if ln.bias is not None else None]
    assert torch.equal(ya.detach(), yb.detach().reshape(shape))
    for name, a, b in zip(("dx", "dweight", "dbias"), ga, gb):
        assert (a is None) == (b is None), name
        if a is not None:
            assert torch.equal(a, b), name
    check_out(ya, ref_ln(x, (hidden,), ln.weight, ln.bias), dtype, x, ln.weight, ln.bias,
              shape=(hidden,))


@pytest.mark.parametrize("shape,dtype,affine", [
    ((32, 768), torch.float32, True), ((4, 9, 4096), torch.bfloat16, True),
    ((2, 3, 2048), torch.float16, False)], ids=["2d-f32", "3d-bf16", "3d-f16-noaffine"])
def test_rms_module_eager_path_matches_the_operator(shape, dtype, affine):
    """FusedRMSNorm's eager forward runs autograd in C++ (fused_layernorm_cuda.
    rms_norm_autograd): output and gradients bitwise identical to the torch.compile-visible
    operator path (fused_layernorm::rms_norm_fwd with its registered autograd)."""
    hidden = shape[-1]
    m = fl.FusedRMSNorm(hidden, eps=1e-6, elementwise_affine=affine).to(DEV, dtype)
    if affine:
        with torch.no_grad():
            m.weight.copy_(1 + 0.1 * torch.randn(hidden))
    x = torch.randn(shape, device=DEV).to(dtype)
    dy = torch.randn(shape, device=DEV).to(dtype)
    xa = x.clone().requires_grad_(True)
    ya = m(xa)
    ya.backward(dy)
    ga = (xa.grad.clone(), m.weight.grad.clone() if affine else None)
    if affine:
        m.weight.grad = None
    xb = x.clone().reshape(-1, hidden).requires_grad_(True)
    yb, _ = torch.ops.fused_layernorm.rms_norm_fwd(xb, m.weight, 1e-6)
    yb.backward(dy.reshape(-1, hidden))
    assert torch.equal(ya.detach(), yb.detach().reshape(shape))
    assert torch.equal(ga[0], xb.grad.reshape(shape))
    if affine:
        assert torch.equal(ga[1], m.weight.grad)


def test_module_eager_path_rejects_mismatched_shapes():
    ln = make_ln(768)
    with pytest.raises(RuntimeError, match="normalized_shape"):
        ln(torch.randn(4, 1024, device=DEV))
    with pytest.raises(RuntimeError):
        fl.fused_layer_norm(torch.randn(4, 768, device=DEV), (768,), torch.ones(512, device=DEV))


def test_gradient_accumulation():
    x = torch.randn(32, 1024, device=DEV, requires_grad=True)
    ln = make_ln(1024)
    dy = torch.randn(32, 1024, device=DEV)
    ln(x).backward(dy)
    g1 = (x.grad.clone(), ln.weight.grad.clone(), ln.bias.grad.clone())
    ln(x).backward(dy)
    for acc, once in zip((x.grad, ln.weight.grad, ln.bias.grad), g1):
        assert torch.equal(acc, 2 * once)  # same kernels, same order: exactly twice


@pytest.mark.parametrize("eps", [1e-5, 1e-6, 1e-7, 1e-8])
def test_different_epsilon(eps):
    x = torch.randn(32, 768, device=DEV)
    ln = fl.FusedLayerNorm(768, eps=eps).to(DEV)
    check_out(ln(x), ref_ln(x, (768,), ln.weight, ln.bias, eps), torch.float32)


@pytest.mark.parametrize("case", ["tiny_const", "huge_const", "small_var", "large_var",
                                  "large_mean"])
def test_numerical_stability(case):
    b, h = 16, 768
    x = {"tiny_const": torch.full((b, h), 1e-8), "huge_const": torch.full((b, h), 1e8),
         "small_var": torch.randn(b, h) * 1e-4, "large_var": torch.randn(b, h) * 1e4,
         "large_mean": torch.randn(b, h) + 1e4}[case].to(DEV)
    ln = make_ln(h)
    y = ln(x)
    assert torch.isfinite(y).all()
    ref = ref_ln(x, (h,), ln.weight, ln.bias)
    # The fp32 bar, plus the fp32 spacing of the row mean, which any fp32 implementation
    # carries (a 1e4 offset is only known to ~1e-3 in fp32): 4 ulp(mean) * rstd * max|gamma|
    # (the sum's rounding is ~1.5 ulp(mean) at 768 columns).  The two-pass variance keeps the
    # offset harmless where E[x^2] - mean^2 would not.  Constant rows (variance 0) map to beta.
    xd = x.double().cpu()
    mean, var = xd.mean(-1, keepdim=True), xd.var(-1, unbiased=False, keepdim=True)
    allow = (2.0 ** -21 * mean.abs() / torch.sqrt(var + 1e-5)
             * ln.weight.abs().max().item()).numpy()
    err = np.abs(to_np(y) - ref.numpy())
    assert (err <= 1e-5 * max(1.0, ref.abs().max().item()) + allow).all(), err.max()


def test_memory_efficiency():
    x = torch.randn(64, 4096, device=DEV)
    ln_t, ln_f = nn.LayerNorm(4096).to(DEV), fl.FusedLayerNorm(4096).to(DEV)

    def peak(mod):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        start = torch.cuda.memory_allocated()
        with torch.no_grad():
            mod(x)
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - start

    peak(ln_f)  # first call loads the kernels
    # The fused forward allocates y plus fp32 mean/rstd and nothing else.
    assert peak(ln_f) <= x.numel() * 4 + 2 * 64 * 4 + 4096
    assert peak(ln_f) <= peak(ln_t) + 2 * 64 * 4 + 4096


def test_functional_interface():
    x = torch.randn(32, 1024, device=DEV)
    w, b = 1 + 0.1 * torch.randn(1024, device=DEV), 0.1 * torch.randn(1024, device=DEV)
    check_out(fl.fused_layer_norm(x, (1024,), w, b, 1e-5), ref_ln(x, (1024,), w, b),
              torch.float32)
    check_out(fl.layer_norm(x, (1024,), w, b, 1e-5), ref_ln(x, (1024,), w, b), torch.float32)


@pytest.mark.parametrize("seed", range(5))
def test_deterministic(seed):
    torch.manual_seed(seed)
    x = torch.randn(257, 2048, device=DEV, requires_grad=True)
    ln = make_ln(2048)
    dy = torch.randn(257, 2048, device=DEV)
    outs = []
    for _ in range(3):
        x.grad = None
        ln.zero_grad()
        y = ln(x)
        y.backward(dy)
        outs.append((y.detach().clone(), x.grad.clone(), ln.weight.grad.clone(),
                     ln.bias.grad.clone()))
    for o in outs[1:]:
        for a, c in zip(outs[0], o):
            assert torch.equal(a, c)


@pytest.mark.parametrize("batch,hidden", [
    (1, 768), (32, 1), (2, 16384),                                      # test_edge_cases
    (1, 1), (1, 17), (1000, 1), (1, 100000), (512, 512), (1, 32767),    # edge_cases.py list
    (1, 65536), (13, 13), (1, 4095), (1, 4097)])
def test_edge_cases(batch, hidden):
    x = torch.randn(batch, hidden, device=DEV)
    ln = nn.LayerNorm(hidden).to(DEV)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(hidden))
        ln.bias.copy_(0.1 * torch.randn(hidden))
    y = fused_layernorm_cuda.layernorm(x, ln.weight, ln.bias, 1e-5)
    assert y.shape == x.shape
    ref = ref_ln(x, (hidden,), ln.weight, ln.bias).numpy()
    assert np.abs(to_np(y) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    if hidden == 1:
        assert torch.equal(y, ln.bias.detach().expand_as(y))


# ------------------------------------------------------------------------------------------------
# The binding (fused_layernorm_cuda), reference names and argument meaning.
# ------------------------------------------------------------------------------------------------
def test_binding_layernorm_keyword_and_positional():
    x = torch.randn(8, 768, device=DEV)
    w, b = torch.ones(768, device=DEV), torch.zeros(768, device=DEV)
    y1 = fused_layernorm_cuda.layernorm(x, w, b, 1e-5)
    y2 = fused_layernorm_cuda.layernorm(x, w, b, eps=1e-5)
    assert torch.equal(y1, y2)
    check_out(y1, ref_ln(x, (768,)), torch.float32)


@pytest.mark.parametrize("approximate", ["tanh", "none"])
def test_binding_layernorm_gelu(approximate):
    x = torch.randn(17, 1023, device=DEV)
    w, b = 1 + 0.1 * torch.randn(1023, device=DEV), 0.1 * torch.randn(1023, device=DEV)
    if approximate == "tanh":
        y = fused_layernorm_cuda.layernorm_gelu(x, w, b, 1e-5)  # the reference's default: tanh
    else:
        y = fused_layernorm_cuda.layernorm_gelu(x, w, b, 1e-5, approximate="none")
    ref = F.gelu(ref_ln(x, (1023,), w, b), approximate=approximate)
    assert np.abs(to_np(y) - ref.numpy()).max() <= 1e-5


@pytest.mark.parametrize("mask", [[True, True, True], [True, False, False],
                                  [False, True, True], [True, True, False]])
def test_binding_forward_backward_output_mask(mask):
    x = torch.randn(64, 1024, device=DEV)
    w, b = 1 + 0.1 * torch.randn(1024, device=DEV), 0.1 * torch.randn(1024, device=DEV)
    out, mean, rstd = fused_layernorm_cuda.forward(x, w, b, 1e-5)
    assert mean.dtype == torch.float32 and rstd.dtype == torch.float32
    check_out(out, ref_ln(x, (1024,), w, b), torch.float32)
    dy = torch.randn_like(x)
    dx, dw, db = fused_layernorm_cuda.backward(dy, x, mean, rstd, w, b, mask)
    gx, gw, gb = _grads_f64(x, w, b, dy, (1024,))
    for want, got, ref in zip(mask, (dx, dw, db), (gx, gw, gb)):
        if not want:
            assert got is None
        else:
            torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4)


def test_binding_forward_without_affine_and_utilities():
    x = torch.randn(4, 512, device=DEV)
    out, mean, rstd = fused_layernorm_cuda.forward(x)
    check_out(out, ref_ln(x, (512,)), torch.float32)
    assert fused_layernorm_cuda.__version__ == "1.0.0"
    assert isinstance(fused_layernorm_cuda.__cuda_version__, int)
    assert fused_layernorm_cuda.get_memory_usage(32, 768) > 0
    assert isinstance(fused_layernorm_cuda.get_performance_hints(32, 768), str)


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_layer_norm_gelu_autograd(approximate):
    x = torch.randn(96, 2048, device=DEV, requires_grad=True)
    w = (1 + 0.1 * torch.randn(2048, device=DEV)).requires_grad_(True)
    b = (0.2 * torch.randn(2048, device=DEV)).requires_grad_(True)
    dy = torch.randn(96, 2048, device=DEV)
    y = fl.layer_norm_gelu(x, (2048,), w, b, 1e-5, approximate=approximate)
    y.backward(dy)
    xd, wd, bd = (t.detach().double().cpu().requires_grad_(True) for t in (x, w, b))
    yr = F.gelu(F.layer_norm(xd, (2048,), wd, bd, 1e-5), approximate=approximate)
    yr.backward(dy.double().cpu())
    assert np.abs(to_np(y) - yr.detach().numpy()).max() <= 1e-5
    for got, ref in ((x.grad, xd.grad), (w.grad, wd.grad), (b.grad, bd.grad)):
        torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------------------------------------
# New operators on the same kernels: RMSNorm, residual add, fp8.
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_module_forward_backward(dtype):
    x = torch.randn(128, 4096, device=DEV, dtype=dtype, requires_grad=True)
    m = fl.FusedRMSNorm(4096, eps=1e-6).to(DEV, dtype)
    with torch.no_grad():
        m.weight.copy_(1 + 0.1 * torch.randn(4096))
    dy = torch.randn(128, 4096, device=DEV, dtype=dtype)
    y = m(x)
    y.backward(dy)
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = m.weight.detach().double().cpu().requires_grad_(True)
    yr = F.rms_norm(xd, (4096,), wd, 1e-6)
    yr.backward(dy.double().cpu())
    if dtype == torch.float32:
        assert np.abs(to_np(y) - yr.detach().numpy()).max() <= 1e-5
        torch.testing.assert_close(x.grad.double().cpu(), xd.grad, rtol=1e-4, atol=1e-4)
    else:
        assert_within_ulp(to_np(y), yr.detach().numpy(), 1.0, what="rms y")
        assert_within_ulp(to_np(x.grad), xd.grad.numpy(), 1.0,
                          atol=2.0 ** -12 * xd.grad.abs().max().item(), what="rms dx")
    g = wd.grad.numpy()
    assert np.abs(to_np(m.weight.grad) - g).max() <= 1e-2 * np.abs(g).max()  # bf16-stored dw


def test_add_layer_norm_forward_and_gradients():
    x = torch.randn(64, 2048, device=DEV, requires_grad=True)
    r = torch.randn(64, 2048, device=DEV, requires_grad=True)
    w, b = 1 + 0.1 * torch.randn(2048, device=DEV), 0.1 * torch.randn(2048, device=DEV)
    y, h = fl.add_layer_norm(x, r, (2048,), w, b, 1e-5)
    assert torch.equal(h, x + r)
    check_out(y, ref_ln(h, (2048,), w, b), torch.float32)
    dy, dh = torch.randn_like(y), torch.randn_like(h)
    (y * dy).sum().add_((h * dh).sum()).backward()
    hd = (x.detach() + r.detach()).double().cpu().requires_grad_(True)
    F.layer_norm(hd, (2048,), w.double().cpu(), b.double().cpu(), 1e-5).backward(
        dy.double().cpu())
    expect = hd.grad + dh.double().cpu()  # h = x + r feeds both outputs
    torch.testing.assert_close(x.grad.double().cpu(), expect, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(r.grad.double().cpu(), expect, rtol=1e-4, atol=1e-4)


def test_add_rms_norm_forward():
    x = torch.randn(32, 4096, device=DEV, dtype=torch.bfloat16)
    r = torch.randn(32, 4096, device=DEV, dtype=torch.bfloat16)
    w = (1 + 0.02 * torch.randn(4096, device=DEV)).to(torch.bfloat16)
    y, h = fl.add_rms_norm(x, r, (4096,), w, 1e-6)
    assert torch.equal(h, x + r)
    ref = F.rms_norm(h.double().cpu(), (4096,), w.double().cpu(), 1e-6)
    assert_within_ulp(to_np(y), ref.numpy(), 1.0, what="add rms y")


def test_layer_norm_fp8_output_type_and_values():
    x = torch.randn(96, 7168, device=DEV, dtype=torch.bfloat16)
    w = (1 + 0.05 * torch.randn(7168, device=DEV)).to(torch.bfloat16)
    b = (0.05 * torch.randn(7168, device=DEV)).to(torch.bfloat16)
    q, scale = fl.layer_norm_fp8(x, (7168,), w, b, 1e-5)
    assert q.dtype == torch.float8_e4m3fn and scale.dtype == torch.float32
    q_ref, s_ref = norms.layer_norm_fp8_fwd(to_np(x), to_np(w), to_np(b), 1e-5)
    assert_fp8_close(q.view(torch.uint8).cpu().numpy(), to_np(scale), q_ref, s_ref, "fp8")
    deq = q.float() * scale[:, None]
    ref = ref_ln(x, (7168,), w, b)
    assert (deq.double().cpu() - ref).abs().max().item() <= 2.0 ** -3 * ref.abs().max().item()


@pytest.mark.parametrize("norm", ["rms", "ln"])
def test_residual_fp8_functional_and_gradient_pass_through(norm):
    """(codes, scale, h) from the fused residual ops; only h is differentiable, and its
    gradient reaches both addends unchanged (h = x + r)."""
    x = torch.randn(64, 4096, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    r = torch.randn(64, 4096, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = (1 + 0.05 * torch.randn(4096, device=DEV)).to(torch.bfloat16)
    if norm == "rms":
        q, scale, h = fl.add_rms_norm_fp8(x, r, (4096,), w, 1e-6)
        q_ref, s_ref, _ = norms.add_rms_norm_fp8_fwd(to_np(x), to_np(r), to_np(w), 1e-6)
    else:
        b = (0.05 * torch.randn(4096, device=DEV)).to(torch.bfloat16)
        q, scale, h = fl.add_layer_norm_fp8(x, r, (4096,), w, b, 1e-5)
        q_ref, s_ref, _ = norms.add_layer_norm_fp8_fwd(to_np(x), to_np(r), to_np(w), to_np(b),
                                                       1e-5)
    assert q.dtype == torch.float8_e4m3fn and not q.requires_grad and not scale.requires_grad
    assert torch.equal(h, (x + r).detach())
    assert_fp8_close(q.view(torch.uint8).cpu().numpy(), to_np(scale), q_ref, s_ref, norm)
    dh = torch.randn_like(h)
    (h * dh).sum().backward()
    assert torch.equal(x.grad, dh) and torch.equal(r.grad, dh)


def test_mxfp8_functional_dtypes_dequantization_and_pass_through():
    x = torch.randn(4, 32, 2048, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    r = torch.randn(4, 32, 2048, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = (1 + 0.05 * torch.randn(2048, device=DEV)).to(torch.bfloat16)
    q, sc, h = fl.add_rms_norm_mxfp8(x, r, (2048,), w, 1e-6)
    assert q.dtype == torch.float8_e4m3fn and sc.dtype == torch.float8_e8m0fnu
    assert q.shape == x.shape and sc.shape == (4, 32, 64)
    deq = (q.float().view(4, 32, 64, 32) * sc.float()[..., None]).view(4, 32, 2048)
    ref = F.rms_norm(h.detach().double().cpu(), (2048,), w.double().cpu(), 1e-6)
    # e4m3: within 2^-3 of the value, or of the block's subnormal step / saturation
    x_blk = sc.float().cpu().double()[..., None].expand(4, 32, 64, 32).reshape(4, 32, 2048)
    err = (deq.double().cpu() - ref).abs()
    bound = ref.abs() * 2 ** -3 + x_blk * 2 ** -9 + (ref.abs() - 448 * x_blk).clamp(min=0)
    assert (err <= bound).all()
    dh = torch.randn_like(h)
    (h * dh).sum().backward()
    assert torch.equal(x.grad, dh) and torch.equal(r.grad, dh)
    q2, sc2 = fl.layer_norm_mxfp8(x.detach(), 2048, w, None, 1e-5)
    q3, sc3 = fl.rms_norm_mxfp8(x.detach(), 2048, w, 1e-6)
    assert sc2.shape == sc3.shape == (4, 32, 64)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        fl.rms_norm_mxfp8(torch.randn(2, 48, device=DEV), 48)


def test_rms_norm_fp8_functional():
    x = torch.randn(4, 16, 2048, device=DEV, dtype=torch.bfloat16)
    w = (1 + 0.05 * torch.randn(2048, device=DEV)).to(torch.bfloat16)
    q, scale = fl.rms_norm_fp8(x, (2048,), w, 1e-6)
    assert q.shape == x.shape and scale.shape == (4, 16)
    q_ref, s_ref = norms.rms_norm_fp8_fwd(to_np(x).reshape(-1, 2048), to_np(w), 1e-6)
    assert_fp8_close(q.view(torch.uint8).reshape(-1, 2048).cpu().numpy(),
                     to_np(scale).reshape(-1), q_ref, s_ref, "rms fp8")


# ------------------------------------------------------------------------------------------------
# torch.compile and operator registration.
# ------------------------------------------------------------------------------------------------
def test_torch_compile_matches_eager():
    torch._dynamo.reset()
    model = nn.Sequential(nn.Linear(512, 1024), fl.FusedLayerNorm(1024), nn.GELU(),
                          nn.Linear(1024, 512), fl.FusedRMSNorm(512, eps=1e-6)).to(DEV)
    x = torch.randn(64, 512, device=DEV, requires_grad=True)
    y_e = model(x)
    y_e.sum().backward()
    g_e = x.grad.clone()
    x.grad = None
    compiled = torch.compile(model, backend="aot_eager")
    y_c = compiled(x)
    y_c.sum().backward()
    # Same kernels in the same order; only the surrounding GEMMs could pick another algorithm.
    torch.testing.assert_close(y_c, y_e, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(x.grad, g_e, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("op,args", [
    ("layer_norm_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                                torch.randn(256, device=DEV, requires_grad=True),
                                torch.randn(256, device=DEV, requires_grad=True), 1e-5)),
    ("rms_norm_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                              torch.randn(256, device=DEV, requires_grad=True), 1e-6)),
    ("add_layer_norm_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                                    torch.randn(8, 256, device=DEV, requires_grad=True),
                                    torch.randn(256, device=DEV), torch.randn(256, device=DEV),
                                    1e-5)),
    ("layer_norm_gelu_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                                     torch.randn(256, device=DEV, requires_grad=True),
                                     torch.randn(256, device=DEV, requires_grad=True), 1e-5,
                                     "tanh")),
    ("add_rms_norm_fp8_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                                      torch.randn(8, 256, device=DEV, requires_grad=True),
                                      torch.randn(256, device=DEV), 1e-6)),
    ("rms_norm_fp8_fwd", lambda: (torch.randn(8, 256, device=DEV),
                                  torch.randn(256, device=DEV), 1e-6)),
    ("add_rms_norm_mxfp8_fwd", lambda: (torch.randn(8, 256, device=DEV, requires_grad=True),
                                        torch.randn(8, 256, device=DEV, requires_grad=True),
                                        torch.randn(256, device=DEV), 1e-6)),
    ("layer_norm_mxfp8_fwd", lambda: (torch.randn(8, 256, device=DEV),
                                      torch.randn(256, device=DEV), None, 1e-5)),
])
def test_opcheck(op, args):
    # opcheck's AOT-dispatch check sums every output into a loss, and torch has no sum for
    # float8 tensors: the fp8 ops get the schema, fake-tensor and autograd-registration checks.
    utils = ("test_schema", "test_autograd_registration", "test_faketensor") \
        if "fp8" in op else ("test_schema", "test_autograd_registration", "test_faketensor",
                             "test_aot_dispatch_dynamic")
    torch.library.opcheck(getattr(torch.ops.fused_layernorm, op), args(), test_utils=utils)


# ------------------------------------------------------------------------------------------------
# HIP graph capture of the C-ABI calls (launch-bound callers replay a captured graph).
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,dtype", [
    (1000, 4096, torch.bfloat16),   # register tiles forward and backward
    (64, 18432, torch.bfloat16),    # RAW forward tiles; 768-thread LDS-staged backward
    (48, 32768, torch.bfloat16),    # RAW forward tiles; two-pass backward (row sums, column pass)
    (40, 16384, torch.float32),     # fp32 LDS-staged backward
    (6, 131072, torch.bfloat16),    # split forward (3 launches); two-pass backward, split sums
    (6, 131073, torch.bfloat16),    # streamed wide-row forward (unaligned rows); two-pass
    (0, 4096, torch.float32),       # empty batch: the backward zero-fills dgamma / dbeta
], ids=["registers", "lds768", "two_pass", "lds_fp32", "split", "wide", "empty"])
def test_forward_backward_in_a_hip_graph_match_eager_on_every_replay(rows, cols, dtype):
    """LayerNorm forward + backward (stage 1 and column reduction) captured once per kernel
    route, replayed with new data copied into the static inputs and the outputs overwritten
    between replays, with eager work and synchronizations in between; every replay must equal
    the eager result bit for bit.  No entry point records a memset node (an empty batch's
    parameter gradients are zeroed by a kernel)."""
    import capi
    from gpu_calls import ln_backward, ln_forward, workspace

    lib = capi.load()
    code = capi.dtype_code(torch.empty(0, dtype=dtype))
    xs = torch.empty(rows, cols, device=DEV, dtype=dtype)
    dys = torch.empty_like(xs)
    g = (1 + 0.1 * torch.randn(cols, device=DEV)).to(dtype)
    b = (0.1 * torch.randn(cols, device=DEV)).to(dtype)
    y, dx = torch.empty_like(xs), torch.empty_like(xs)
    mean = torch.empty(rows, device=DEV)
    rstd = torch.empty(rows, device=DEV)
    dg = torch.empty(cols, device=DEV)
    db = torch.empty(cols, device=DEV)
    ws, nws = workspace(lib, rows, cols, xs)
    p = capi.ptr

    def calls():
        st = capi.stream()
        capi.check(lib.fln_layernorm_forward(p(xs), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                             cols, code, 1e-5, st))
        capi.check(lib.fln_layernorm_backward(p(dys), p(xs), p(mean), p(rstd), p(g), None,
                                              p(dx), p(dg), p(db), rows, cols, code, capi.F32,
                                              p(ws), nws, st))

    xs.normal_()
    dys.normal_()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()  # warm-up outside the capture (per-device caches)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    for k in range(4):
        torch.manual_seed(100 + k)
        x_new = torch.randn(rows, cols, device=DEV).to(dtype)
        dy_new = torch.randn(rows, cols, device=DEV).to(dtype)
        xs.copy_(x_new)
        dys.copy_(dy_new)
        for out in (y, dx, mean, rstd, dg, db):
            out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        y_e, m_e, r_e = ln_forward(lib, x_new, g, b, 1e-5)
        dx_e, dg_e, db_e = ln_backward(lib, dy_new, x_new, m_e, r_e, g)
        torch.cuda.synchronize()
        for name, got, ref in (("y", y, y_e), ("mean", mean, m_e), ("rstd", rstd, r_e),
                               ("dx", dx, dx_e), ("dgamma", dg, dg_e), ("dbeta", db, db_e)):
            assert torch.equal(got, ref), f"replay {k}: {name} differs from eager"
        if rows == 0:
            assert not dg.any() and not db.any()


@pytest.mark.parametrize("rows,cols,dtype", [
    (8192, 4096, torch.bfloat16), (32768, 7168, torch.bfloat16), (32, 768, torch.float32),
    (17, 1023, torch.float32), (64, 4096, torch.float32), (1, 100000, torch.float32),
    (16384, 8192, torch.bfloat16), (5, 5120, torch.float16), (64, 12288, torch.bfloat16),
    (64, 16384, torch.float16), (64, 32768, torch.bfloat16), (64, 16384, torch.float32),
    (3, 20000, torch.float32), (64, 65536, torch.bfloat16), (5, 65544, torch.bfloat16),
    (7, 32772, torch.float32), (3, 40001, torch.float16), (2, 131072, torch.bfloat16),
    (16384, 2560, torch.bfloat16), (8192, 6656, torch.bfloat16), (16384, 3328, torch.float32),
    (2048, 100000, torch.float32), (63, 65536, torch.bfloat16), (300, 262144, torch.bfloat16),
    (64, 98304, torch.bfloat16), (512, 131072, torch.bfloat16), (64, 40960, torch.float32),
    (64, 65536, torch.float32)])
def test_optimal_config_matches_the_dispatcher(rows, cols, dtype, capfd, monkeypatch):
    """functional.get_optimal_config reports the plan of the C-ABI query fln_forward_plan; the
    dispatcher's own trace of the launch it made (FLN_DEBUG_GEOMETRY=1, one stderr line per
    launch) must name the same route and geometry (register route: waves per row, vectors per
    lane, exact tiling; every route: threads per block)."""
    import re
    import capi
    x = torch.randn(rows, cols, device=DEV, dtype=dtype)
    w = torch.ones(cols, device=DEV, dtype=dtype)
    capfd.readouterr()
    monkeypatch.setenv("FLN_DEBUG_GEOMETRY", "1")
    capi.reload_tuning()
    fused_layernorm_cuda.layernorm(x, w, w, 1e-5)
    torch.cuda.synchronize()
    monkeypatch.delenv("FLN_DEBUG_GEOMETRY")
    capi.reload_tuning()
    line = capfd.readouterr().err.strip().splitlines()[-1]
    cfg = fl.functional.get_optimal_config(rows, cols, dtype)
    m = re.search(r"-> (\S+) wpr=(\d+) vpl=(\d+) exact=(\d) threads=(\d+)", line)
    assert m, line
    assert m[1] == cfg["route"], line
    assert int(m[5]) == cfg["threads_per_block"], line
    if cfg["register_resident"]:
        assert (int(m[2]), int(m[3]), bool(int(m[4]))) == (
            cfg["waves_per_row"], cfg["vectors_per_lane"], cfg["exact_tiling"]), line


# ------------------------------------------------------------------------------------------------
# Model-level drop-in: module swap inside transformer blocks, eager and torch.compile.
# ------------------------------------------------------------------------------------------------
class _TinyLM(nn.Module):
    def __init__(self, vocab=1000, d=256, layers=2):
        super().__init__()
        self.emb = nn.Embedding(vocab, d)
        self.blocks = nn.ModuleList(
            nn.TransformerEncoderLayer(d_model=d, nhead=8, dim_feedforward=4 * d, dropout=0.0,
                                       batch_first=True, norm_first=True)
            for _ in range(layers))
        self.norm = nn.LayerNorm(d)
        self.head = nn.Linear(d, vocab)

    def forward(self, tokens):
        h = self.emb(tokens)
        for blk in self.blocks:
            h = blk(h)
        return self.head(self.norm(h))


@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
def test_transformer_logits_and_gradients_after_module_swap(compiled):
    """End-to-end parity: a transformer whose nn.LayerNorm modules are swapped for the fused
    ones (replace_layernorm_modules) gives the same logits and parameter gradients as the
    original (fp32; the norms differ only in summation order, so 1e-4 relative to the largest
    logit / gradient).  Train mode: torch's eval fast path would call its own fused encoder op
    and bypass the norm modules."""
    import copy
    torch.manual_seed(0)
    ref = _TinyLM().to(DEV).train()
    fused = fl.replace_layernorm_modules(copy.deepcopy(ref))
    assert all(isinstance(b.norm1, fl.FusedLayerNorm) for b in fused.blocks)
    run = torch.compile(fused, backend="aot_eager") if compiled else fused
    if compiled:
        torch._dynamo.reset()
    tokens = torch.randint(0, 1000, (8, 128), device=DEV)
    target = torch.randint(0, 1000, (8, 128), device=DEV)
    logits_ref = ref(tokens)
    logits = run(tokens)
    scale = logits_ref.abs().max().item()
    assert (logits - logits_ref).abs().max().item() <= 1e-4 * scale
    F.cross_entropy(logits_ref.flatten(0, 1), target.flatten()).backward()
    F.cross_entropy(logits.flatten(0, 1), target.flatten()).backward()
    for (name, p_ref), (_, p) in zip(ref.named_parameters(), fused.named_parameters()):
        g_ref = p_ref.grad
        tol = 1e-4 * max(g_ref.abs().max().item(), 1e-12)
        assert (p.grad - g_ref).abs().max().item() <= tol, name


def _module_cases(n=48, seed=4321):
    """Seeded FusedLayerNorm calls: rank 1-4, hidden sizes from 1 to 12288, leading dims 1-8,
    fp32 / bf16 / fp16, with or without weight and bias, contiguous or every-other-column views."""
    rng = np.random.default_rng(seed)
    hiddens = [1, 7, 64, 768, 1000, 1024, 2048, 3072, 4096, 5120, 8192, 12288]
    cases = []
    for _ in range(n):
        rank = int(rng.integers(1, 5))
        hidden = int(rng.choice(hiddens))
        lead = tuple(int(v) for v in rng.integers(1, 9, size=rank - 1))
        dtype = (torch.float32, torch.bfloat16, torch.float16)[int(rng.integers(3))]
        affine = bool(rng.integers(4) > 0)
        bias = affine and bool(rng.integers(4) > 0)
        strided = bool(rng.integers(2))
        cases.append((lead + (hidden,), dtype, affine, bias, strided))
    return cases


MODULE_CASES = _module_cases()


@pytest.mark.parametrize("shape,dtype,affine,bias,strided", MODULE_CASES,
                         ids=[f"{i}-{'x'.join(map(str, c[0]))}-{str(c[1])[6:]}"
                              f"{'-noaffine' if not c[2] else '-nobias' if not c[3] else ''}"
                              f"{'-strided' if c[4] else ''}" for i, c in enumerate(MODULE_CASES)])
def test_module_random_shapes(shape, dtype, affine, bias, strided):
    """FusedLayerNorm over seeded random ranks, widths, dtypes, affine flags and strided views:
    the output against torch's float64 LayerNorm on the CPU (the bars of check_out), and for
    fp32 the gradients of x, weight and bias against float64 autograd at the reference's
    gradient tolerance (rtol = atol = 1e-4, tests/test_layernorm.py:34-35)."""
    hidden = shape[-1]
    ln = make_ln(hidden, dtype, affine=affine, bias=bias)
    gen = torch.Generator().manual_seed(int(np.prod(shape)) * 7 + len(shape) * 3 +
                                        (torch.float32, torch.bfloat16, torch.float16).index(dtype))
    full = torch.randn(*shape[:-1], 2 * hidden, generator=gen) * 1.5 + 0.25
    x = (full[..., ::2] if strided else full[..., :hidden].contiguous()).to(DEV, dtype)
    x.requires_grad_(dtype == torch.float32)
    y = ln(x)
    check_out(y, ref_ln(x, (hidden,), ln.weight, ln.bias), dtype, x, ln.weight, ln.bias,
              shape=(hidden,))
    if dtype != torch.float32:
        return
    dy = torch.randn(shape, generator=gen).to(DEV)
    y.backward(dy)
    gx, gw, gb = _grads_f64(x, ln.weight, ln.bias, dy, (hidden,))
    torch.testing.assert_close(x.grad.double().cpu(), gx, rtol=1e-4, atol=1e-4)
    if affine:
        torch.testing.assert_close(ln.weight.grad.double().cpu(), gw, rtol=1e-4, atol=1e-4)
    if bias:
        torch.testing.assert_close(ln.bias.grad.double().cpu(), gb, rtol=1e-4, atol=1e-4)
