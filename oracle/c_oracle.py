"""ctypes wrapper of the C oracle (oracle/fln_oracle.c) -- test infrastructure only.

``load()`` builds ``oracle/liboracle.so`` with make if it is missing (gcc is present both here
and on the GPU box) and returns the library; the wrappers take numpy float32 arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
_lib = None

_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    src = os.path.join(HERE, "fln_oracle.c")
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "liboracle.so"], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(LIB)
        lib.orc_layernorm_fwd.argtypes = [_fp, _fp, _fp, _i64, _i64, ctypes.c_double, _fp, _dp, _dp]
        lib.orc_rmsnorm_fwd.argtypes = [_fp, _fp, _i64, _i64, ctypes.c_double, _fp, _dp]
        lib.orc_layernorm_bwd.argtypes = [_fp, _fp, _fp, _i64, _i64, ctypes.c_double, _fp, _dp, _dp]
        lib.orc_rmsnorm_bwd.argtypes = [_fp, _fp, _fp, _i64, _i64, ctypes.c_double, _fp, _dp]
        lib.orc_fp8_e4m3fn.argtypes = [ctypes.c_double]
        lib.orc_fp8_e4m3fn.restype = ctypes.c_uint8
        lib.orc_layernorm_fp8.argtypes = [_fp, _fp, _fp, _i64, _i64, ctypes.c_double, _u8p, _fp]
        lib.orc_rmsnorm_fp8.argtypes = [_fp, _fp, _i64, _i64, ctypes.c_double, _u8p, _fp]
        _lib = lib
    return _lib


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def layernorm_fwd(x, gamma=None, beta=None, eps=1e-5):
    x, g, b = _f32(x), _f32(gamma), _f32(beta)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    mean = np.empty(rows, np.float64)
    rstd = np.empty(rows, np.float64)
    load().orc_layernorm_fwd(_p(x, _fp), _p(g, _fp), _p(b, _fp), rows, cols, eps, _p(y, _fp),
                             _p(mean, _dp), _p(rstd, _dp))
    return y, mean, rstd


def rmsnorm_fwd(x, weight=None, eps=1e-6):
    x, w = _f32(x), _f32(weight)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    rstd = np.empty(rows, np.float64)
    load().orc_rmsnorm_fwd(_p(x, _fp), _p(w, _fp), rows, cols, eps, _p(y, _fp), _p(rstd, _dp))
    return y, rstd


def layernorm_bwd(dy, x, gamma=None, eps=1e-5):
    dy, x, g = _f32(dy), _f32(x), _f32(gamma)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    dx = np.empty_like(x)
    dg = np.empty(cols, np.float64)
    db = np.empty(cols, np.float64)
    load().orc_layernorm_bwd(_p(dy, _fp), _p(x, _fp), _p(g, _fp), rows, cols, eps, _p(dx, _fp),
                             _p(dg, _dp), _p(db, _dp))
    return dx, dg, db


def rmsnorm_bwd(dy, x, weight=None, eps=1e-6):
    dy, x, w = _f32(dy), _f32(x), _f32(weight)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    dx = np.empty_like(x)
    dw = np.empty(cols, np.float64)
    load().orc_rmsnorm_bwd(_p(dy, _fp), _p(x, _fp), _p(w, _fp), rows, cols, eps, _p(dx, _fp),
                           _p(dw, _dp))
    return dx, dw


def fp8_encode_scalar(v: float) -> int:
    return int(load().orc_fp8_e4m3fn(float(v)))


def layernorm_fp8(x, gamma=None, beta=None, eps=1e-5):
    x, g, b = _f32(x), _f32(gamma), _f32(beta)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    q = np.empty(x.shape, np.uint8)
    scale = np.empty(rows, np.float32)
    load().orc_layernorm_fp8(_p(x, _fp), _p(g, _fp), _p(b, _fp), rows, cols, eps, _p(q, _u8p),
                             _p(scale, _fp))
    return q, scale


def rmsnorm_fp8(x, weight=None, eps=1e-6):
    x, w = _f32(x), _f32(weight)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    q = np.empty(x.shape, np.uint8)
    scale = np.empty(rows, np.float32)
    load().orc_rmsnorm_fp8(_p(x, _fp), _p(w, _fp), rows, cols, eps, _p(q, _u8p), _p(scale, _fp))
    return q, scale
