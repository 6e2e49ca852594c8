"""Utilities of the reference's fused_layernorm/functional.py, kept with the same names.

``check_input_dtype_and_device`` (:13-44), ``get_optimal_config`` (:47-74),
``benchmark_config`` (:77-129), ``LayerNormProfiler`` and the global profiler helpers
(:132-213).  ``get_optimal_config`` reports the launch plan this library's dispatcher takes on
MI355X (kernel route, waves per row, vectors per lane), queried from the dispatcher itself,
instead of the reference's CUDA-capability heuristics; the benchmark times with HIP events on
the current stream.
"""
from __future__ import annotations

import statistics
from typing import Optional, Tuple

import torch

from .layernorm import FusedLayerNormFunction, fused_layernorm_cuda

__all__ = [
    "FusedLayerNormFunction", "check_input_dtype_and_device", "get_optimal_config",
    "benchmark_config", "LayerNormProfiler", "enable_profiling", "disable_profiling",
    "get_profiler",
]


def check_input_dtype_and_device(input: torch.Tensor, weight: Optional[torch.Tensor] = None,
                                 bias: Optional[torch.Tensor] = None) -> None:
    """Raise RuntimeError unless input/weight/bias are GPU tensors on one device with one dtype
    (same messages as the reference, functional.py:13-44)."""
    if not input.is_cuda:
        raise RuntimeError("FusedLayerNorm requires CUDA tensors")
    for name, t in (("Weight", weight), ("Bias", bias)):
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a CUDA tensor")
        if t.device != input.device:
            raise RuntimeError(f"{name} and input must be on the same device")
        if t.dtype != input.dtype:
            raise RuntimeError(f"{name} and input must have the same dtype")


_DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3}
_ROUTES = {-1: "none", 0: "registers", 1: "lds", 2: "lds+registers", 3: "wide", 4: "split",
           5: "loop"}
_GELU_CODES = {None: 0, "none": 1, "tanh": 2}


def get_optimal_config(batch_size: int, hidden_size: int,
                       dtype: torch.dtype = torch.float32, num_cus: Optional[int] = None,
                       fp8: int = 0, residual: bool = False,
                       approximate: Optional[str] = None) -> dict:
    """Forward launch plan the HIP dispatcher takes for a contiguous, 16-byte aligned
    [batch_size, hidden_size] input, with the reference's keys (reference
    fused_layernorm/functional.py:47-72) and this library's geometry.

    The plan comes from the dispatcher itself (the C-ABI query ``fln_forward_plan``, the same
    function that decides the launches, under the same FLN_* knobs), so there is no second copy
    of the rule here.  ``num_cus``: the CU count to plan for (default: the current device's, or
    256 -- MI355X -- without a GPU).  ``fp8`` (0, 1 per-row scale, 2 MXFP8), ``residual`` and
    ``approximate`` (GELU form, None for no GELU) select the flavour."""
    if dtype not in _DTYPE_CODES:
        raise ValueError(f"unsupported dtype {dtype}")
    if num_cus is None:
        num_cus = 0 if torch.cuda.is_available() else 256
    route, vec, wpr, vpl, exact, threads = fused_layernorm_cuda.forward_plan(
        batch_size, hidden_size, _DTYPE_CODES[dtype], fp8, residual,
        _GELU_CODES[approximate], num_cus)
    name = _ROUTES[route]
    return {
        "use_mixed_precision": dtype in (torch.float16, torch.bfloat16),
        "threads_per_block": threads,
        "enable_persistent_kernel": name in ("registers", "lds", "lds+registers", "wide"),
        "use_vectorized_load": vec > 1,
        "use_tensor_cores": False,  # bandwidth-bound: no MFMA on this path
        "route": name,
        "waves_per_row": wpr if name == "registers" else None,
        "vector_elems": vec,
        "vectors_per_lane": vpl if name == "registers" else None,
        "exact_tiling": bool(exact),
        "register_resident": name == "registers",
        "lds_staged": name in ("lds", "lds+registers"),
        "lds_registers": name == "lds+registers",
        "threads_lds": threads if name in ("lds", "lds+registers") else None,
        "wide_streamed": name == "wide",
        "split_rows": name == "split",
    }


def benchmark_config(input_shape: Tuple[int, ...], num_iterations: int = 100,
                     warmup_iterations: int = 10, dtype: torch.dtype = torch.float32) -> dict:
    """Forward and forward+backward wall time of FusedLayerNormFunction (reference
    functional.py:77-129), timed with HIP events on the current stream."""
    device = torch.cuda.current_device()
    x = torch.randn(input_shape, device=device, dtype=dtype)
    x2 = x.reshape(-1, input_shape[-1])
    ns = (input_shape[-1],)
    weight = torch.ones(ns, device=device, dtype=dtype, requires_grad=True)
    bias = torch.zeros(ns, device=device, dtype=dtype, requires_grad=True)
    for _ in range(warmup_iterations):
        FusedLayerNormFunction.apply(x2, ns, weight, bias, 1e-5)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(num_iterations):
        out = FusedLayerNormFunction.apply(x2, ns, weight, bias, 1e-5)
    end.record()
    torch.cuda.synchronize()
    forward_time = start.elapsed_time(end) / num_iterations
    grad = torch.randn_like(out)
    start.record()
    for _ in range(num_iterations):
        out = FusedLayerNormFunction.apply(x2, ns, weight, bias, 1e-5)
        out.backward(grad)
    end.record()
    torch.cuda.synchronize()
    backward_time = start.elapsed_time(end) / num_iterations
    return {
        "forward_time_ms": forward_time,
        "backward_time_ms": backward_time,
        "total_time_ms": forward_time + backward_time,
        "throughput_gb_s": (x.numel() * x.element_size() * 2) / (forward_time * 1e6),
    }


class LayerNormProfiler:
    """Collects (batch, hidden, forward ms, backward ms) records and summarises them
    (reference functional.py:132-194)."""

    def __init__(self):
        self.profiles = []
        self.enabled = False

    def start(self):
        self.enabled = True
        self.profiles = []

    def stop(self):
        self.enabled = False
        return self.analyze_profiles()

    def record(self, batch_size: int, hidden_size: int, forward_time: float,
               backward_time: float):
        if self.enabled:
            self.profiles.append({
                "batch_size": batch_size, "hidden_size": hidden_size,
                "forward_time_ms": forward_time, "backward_time_ms": backward_time,
                "total_time_ms": forward_time + backward_time,
            })

    def analyze_profiles(self) -> dict:
        if not self.profiles:
            return {}

        def summary(vals):
            return {"mean_ms": statistics.mean(vals),
                    "std_ms": statistics.stdev(vals) if len(vals) > 1 else 0,
                    "min_ms": min(vals), "max_ms": max(vals)}

        return {
            "num_calls": len(self.profiles),
            "forward": summary([p["forward_time_ms"] for p in self.profiles]),
            "backward": summary([p["backward_time_ms"] for p in self.profiles]),
            "total": summary([p["total_time_ms"] for p in self.profiles]),
        }


_profiler = LayerNormProfiler()


def enable_profiling():
    _profiler.start()


def disable_profiling():
    return _profiler.stop()


def get_profiler():
    return _profiler
