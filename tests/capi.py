"""ctypes view of libfln.so's C ABI (include/fused_layernorm.h) for the tests.

Wrappers take torch tensors (or None) and pass raw device pointers plus the current HIP stream,
exactly as a non-Python caller of the C ABI would.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "fused-layernorm-cuda-operator_amd")
LIB_PATH = os.path.join(PKG, "libfln.so")
HEADER = os.path.join(ROOT, "include", "fused_layernorm.h")

F32, BF16, F16, F64, F8E4M3FN = 0, 1, 2, 3, 4
ERR_INVALID, ERR_TOO_LARGE = 1, -2
GELU_NONE, GELU_ERF, GELU_TANH = 0, 1, 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

SIGNATURES = {
    "fln_layernorm": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp], _i32),
    "fln_layernorm_gelu": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _i32, _vp], _i32),
    "fln_layernorm_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp], _i32),
    "fln_layernorm_gelu_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _i32,
                                    _vp], _i32),
    "fln_layernorm_gelu_backward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                     _i32, _i32, _i32, _vp, _sz, _vp], _i32),
    "fln_backward_workspace_bytes": ([_i64, _i64, _i32], _sz),
    "fln_layernorm_backward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32,
                                _i32, _vp, _sz, _vp], _i32),
    "fln_layernorm_backward_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                        _i32, _i32, _vp], _i32),
    "fln_rmsnorm_forward": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp], _i32),
    "fln_rmsnorm_backward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp,
                              _sz, _vp], _i32),
    "fln_add_layernorm_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32,
                                   _f32, _vp], _i32),
    "fln_add_rmsnorm_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp],
                                _i32),
    "fln_layernorm_fp8_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32,
                                   _vp], _i32),
    "fln_rmsnorm_fp8_forward": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp], _i32),
    "fln_add_layernorm_fp8_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                       _i32, _f32, _vp], _i32),
    "fln_add_rmsnorm_fp8_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32,
                                     _vp], _i32),
    "fln_layernorm_mxfp8_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32,
                                     _vp], _i32),
    "fln_rmsnorm_mxfp8_forward": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _vp], _i32),
    "fln_add_rmsnorm_mxfp8_forward": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32,
                                       _f32, _vp], _i32),
    "fln_fp8_e4m3fn_encode": ([_vp, _vp, _i64, _vp], _i32),
    "fln_forward_plan": ([_i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp], _i32),
    "fln_get_memory_usage": ([_i32, _i32, _i32], _i64),
    "fln_get_performance_hints": ([_i32, _i32, ctypes.c_char_p, _sz], _i32),
    "fln_version": ([], ctypes.c_char_p),
    "fln_hip_version": ([], _i32),
    "fln_error_string": ([_i32], ctypes.c_char_p),
    "fln_reload_tuning": ([], None),
}


def declared_functions():
    """Names of the functions declared in include/fused_layernorm.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fln_[a-z0-9_]+)\s*\(", text)))


_lib = None


def load():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def reload_tuning():
    """Make libfln re-read its FLN_* environment knobs (read once per process otherwise); call
    after setting or clearing one."""
    load().fln_reload_tuning()


def dtype_code(t):
    import torch
    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16,
            torch.float64: F64}[t.dtype]


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def check(rc):
    if rc != 0:
        raise RuntimeError(f"libfln error {rc}: {load().fln_error_string(rc).decode()}")
