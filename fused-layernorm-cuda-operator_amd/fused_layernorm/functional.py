"""Utilities of the reference's fused_layernorm/functional.py, kept with the same names.

``check_input_dtype_and_device`` (:13-44), ``get_optimal_config`` (:47-74),
``benchmark_config`` (:77-129), ``LayerNormProfiler`` and the global profiler helpers
(:132-213).  ``get_optimal_config`` reports the geometry this library actually uses on MI355X
(waves per row, vectors per lane) instead of the reference's CUDA-capability heuristics; the
benchmark times with HIP events on the current stream.
"""
from __future__ import annotations

import math
import statistics
from typing import Optional, Tuple

import torch

from .layernorm import FusedLayerNormFunction

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


def _next_pow2(v: int) -> int:
    p = 1
    while p < v:
        p <<= 1
    return p


def get_optimal_config(batch_size: int, hidden_size: int,
                       dtype: torch.dtype = torch.float32, num_cus: int = 256) -> dict:
    """Forward launch geometry the HIP dispatcher picks for a [batch_size, hidden_size] input
    (aligned, contiguous), plus the reference's keys (functional.py:61-72)."""
    es = torch.empty((), dtype=dtype).element_size()
    vec = 16 // es if (hidden_size * es) % 16 == 0 else 1
    nvec = hidden_size // vec
    cap = 16 if vec == 1 else 32 // vec
    per_lane = lambda w: -(-nvec // (64 * w))  # noqa: E731
    wpr = 1
    while per_lane(wpr) > cap and wpr < 16:
        wpr *= 2
    register_resident = per_lane(wpr) <= cap
    while register_resident and batch_size * wpr < 4 * num_cus and wpr < 16 and \
            nvec > 64 * wpr * 2:
        wpr *= 2
    return {
        "use_mixed_precision": dtype in (torch.float16, torch.bfloat16),
        "threads_per_block": 256 if wpr <= 4 else 64 * wpr,
        "enable_persistent_kernel": False,
        "use_vectorized_load": vec > 1,
        "use_tensor_cores": False,  # bandwidth-bound: no MFMA on this path
        "waves_per_row": wpr,
        "vector_elems": vec,
        "vectors_per_lane": _next_pow2(per_lane(wpr)) if register_resident else None,
        "register_resident": register_resident,
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
