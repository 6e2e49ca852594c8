"""C-ABI call wrappers shared by the GPU tests: torch tensors (or None) in, raw device pointers
and torch's current HIP stream passed to libfln.so, exactly as a non-Python caller would."""
from __future__ import annotations

import numpy as np
import torch

import capi
from helpers import to_np


def cuda(t):
    return None if t is None else t.to("cuda")


def f32(t):
    return None if t is None else to_np(t).astype(np.float32)


def ln_forward(lib, x, g, b, eps, stats=True):
    rows, cols = x.numel() // x.shape[-1], x.shape[-1]
    y = torch.empty_like(x)
    mean = torch.empty(rows, device=x.device, dtype=torch.float32) if stats else None
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32) if stats else None
    capi.check(lib.fln_layernorm_forward(capi.ptr(x), capi.ptr(g), capi.ptr(b), capi.ptr(y),
                                         capi.ptr(mean), capi.ptr(rstd), rows, cols,
                                         capi.dtype_code(x), eps, capi.stream()))
    return y, mean, rstd


def rms_forward(lib, x, w, eps):
    rows, cols = x.numel() // x.shape[-1], x.shape[-1]
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    capi.check(lib.fln_rmsnorm_forward(capi.ptr(x), capi.ptr(w), capi.ptr(y), capi.ptr(rstd),
                                       rows, cols, capi.dtype_code(x), eps, capi.stream()))
    return y, rstd


def workspace(lib, rows, cols, x):
    n = lib.fln_backward_workspace_bytes(rows, cols, capi.dtype_code(x))
    return torch.empty(max(1, (n + 3) // 4), device=x.device, dtype=torch.float32), n


def ln_backward(lib, dy, x, mean, rstd, g, want_params=True, dres=None, dparam_f32=True):
    rows, cols = x.numel() // x.shape[-1], x.shape[-1]
    dx = torch.empty_like(x)
    pdt = torch.float32 if dparam_f32 else x.dtype
    dg = torch.empty(cols, device=x.device, dtype=pdt) if want_params else None
    db = torch.empty(cols, device=x.device, dtype=pdt) if want_params else None
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_layernorm_backward(
        capi.ptr(dy), capi.ptr(x), capi.ptr(mean), capi.ptr(rstd), capi.ptr(g), capi.ptr(dres),
        capi.ptr(dx), capi.ptr(dg), capi.ptr(db), rows, cols, capi.dtype_code(x),
        capi.F32 if dparam_f32 else capi.dtype_code(x), capi.ptr(ws), n, capi.stream()))
    return dx, dg, db


def rms_backward(lib, dy, x, rstd, w, dres=None):
    rows, cols = x.numel() // x.shape[-1], x.shape[-1]
    dx = torch.empty_like(x)
    dw = torch.empty(cols, device=x.device, dtype=torch.float32) if w is not None else None
    ws, n = workspace(lib, rows, cols, x)
    capi.check(lib.fln_rmsnorm_backward(
        capi.ptr(dy), capi.ptr(x), capi.ptr(rstd), capi.ptr(w), capi.ptr(dres), capi.ptr(dx),
        capi.ptr(dw), rows, cols, capi.dtype_code(x), capi.F32, capi.ptr(ws), n, capi.stream()))
    return dx, dw
