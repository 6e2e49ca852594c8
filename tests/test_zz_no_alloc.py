"""GPU test of fln_layernorm_backward_noalloc (the backward entry point that allocates nothing: its
workspace is a fixed per-device scratch array): called through the C ABI, its dx / dgamma / dbeta
must equal fln_layernorm_backward's (same kernels and geometry, a caller-allocated workspace)
bit for bit, on consecutive calls of decreasing size (the scratch keeps the previous call's
contents), and a call that needs more than the scratch holds is refused before any launch."""
from __future__ import annotations

import pytest
import torch

import capi
from gpu_calls import ln_backward, ln_forward

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(gpu_available):
    return capi.load()


def _inputs(rows, cols, dtype, seed, dres=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, cols, generator=g, device="cuda").to(dtype)
    dy = torch.randn(rows, cols, generator=g, device="cuda").to(dtype)
    gamma = (1 + 0.1 * torch.randn(cols, generator=g, device="cuda")).to(dtype)
    beta = (0.1 * torch.randn(cols, generator=g, device="cuda")).to(dtype)
    r = torch.randn(rows, cols, generator=g, device="cuda").to(dtype) if dres else None
    return x, dy, gamma, beta, r


def _noalloc(lib, dy, x, mean, rstd, g, dres=None, want_dbeta=True):
    rows, cols = x.shape
    dx = torch.full_like(x, float("nan"))
    dg = torch.full((cols,), float("nan"), device="cuda")
    db = torch.full((cols,), float("nan"), device="cuda") if want_dbeta else None
    rc = lib.fln_layernorm_backward_noalloc(
        capi.ptr(dy), capi.ptr(x), capi.ptr(mean), capi.ptr(rstd), capi.ptr(g), capi.ptr(dres),
        capi.ptr(dx), capi.ptr(dg), capi.ptr(db), rows, cols, capi.dtype_code(x), capi.F32,
        capi.stream())
    return rc, dx, dg, db


@pytest.mark.parametrize("cases", [
    # (rows, cols, dtype, residual gradient, dbeta wanted): a large call, then smaller ones
    # (12 x 65536: the two-pass backward with its row statistics split into column chunks).
    [(16384, 8192, torch.bfloat16, False, True), (8192, 4096, torch.bfloat16, False, True),
     (1000, 2048, torch.bfloat16, True, True), (12, 65536, torch.bfloat16, False, True),
     (37, 768, torch.float32, False, False)],
])
def test_noalloc_backward_equals_workspace_backward(lib, cases):
    for k, (rows, cols, dtype, with_dres, want_dbeta) in enumerate(cases):
        print(f"[no-alloc] case {k}: {rows} x {cols} {dtype} dres={with_dres}", flush=True)
        x, dy, gamma, beta, r = _inputs(rows, cols, dtype, 100 + k, with_dres)
        _, mean, rstd = ln_forward(lib, x, gamma, beta, 1e-5)
        dx_ref, dg_ref, db_ref = ln_backward(lib, dy, x, mean, rstd, gamma, dres=r)
        rc, dx, dg, db = _noalloc(lib, dy, x, mean, rstd, gamma, dres=r, want_dbeta=want_dbeta)
        capi.check(rc)
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_ref), f"dx differs (case {k})"
        assert torch.equal(dg, dg_ref), f"dgamma differs (case {k})"
        if want_dbeta:
            assert torch.equal(db, db_ref), f"dbeta differs (case {k})"


def test_noalloc_backward_refuses_calls_past_its_scratch(lib):
    # 4096 x 20480 bf16: one LDS-staged block per CU, 2 x 256 partial rows of 20480 fp32
    # columns = 40 MiB > 32 MiB of scratch.  Refused before any launch: outputs untouched.
    rows, cols = 4096, 20480
    x, dy, gamma, beta, _ = _inputs(rows, cols, torch.bfloat16, 7)
    _, mean, rstd = ln_forward(lib, x, gamma, beta, 1e-5)
    torch.cuda.synchronize()
    rc, dx, dg, db = _noalloc(lib, dy, x, mean, rstd, gamma)
    torch.cuda.synchronize()
    assert rc == capi.ERR_TOO_LARGE
    assert "scratch" in lib.fln_error_string(rc).decode()
    assert torch.isnan(dx.float()).all() and torch.isnan(dg).all() and torch.isnan(db).all()
    # The same shape without parameter gradients needs no partial rows and runs.
    dx2 = torch.empty_like(x)
    capi.check(lib.fln_layernorm_backward_noalloc(
        capi.ptr(dy), capi.ptr(x), capi.ptr(mean), capi.ptr(rstd), capi.ptr(gamma), None,
        capi.ptr(dx2), None, None, rows, cols, capi.BF16, capi.F32, capi.stream()))
    dx_ref, _, _ = ln_backward(lib, dy, x, mean, rstd, gamma, want_params=False)
    torch.cuda.synchronize()
    assert torch.equal(dx2, dx_ref)
