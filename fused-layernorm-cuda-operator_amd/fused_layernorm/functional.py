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


def _forward_geometry(rows: int, nvec: int, cap: int, wide_cap: int, max_cap: int,
                      vec_path: bool, num_cus: int):
    """The forward dispatcher's geometry rule (csrc/fln_forward_impl.h, fwd_geometry): the
    fewest power-of-two waves per row that keep <= cap vectors per lane for rows of up to 4
    waves and <= wide_cap beyond (max_cap when nothing narrower fits 16 waves); on the vector
    path an exact (mask-free) non-power-of-two tiling within the same caps when one exists;
    more waves per row (up to 4) while the grid holds fewer than 4 waves per CU.
    Returns (loop, wpr, vpl, exact, threads)."""
    per_lane = lambda w: -(-nvec // (64 * w))  # noqa: E731
    cap_of = lambda w: cap if w <= 4 else wide_cap  # noqa: E731
    wpr = 1
    while per_lane(wpr) > cap_of(wpr) and wpr < 16:
        wpr *= 2
    widest = per_lane(wpr) > cap_of(wpr)
    if widest and per_lane(wpr) > max_cap:
        return True, 0, 0, False, 1024
    fits = lambda w, v: v <= (max_cap if widest else cap_of(w))  # noqa: E731
    vpl = _next_pow2(per_lane(wpr))
    exact = nvec == vpl * 64 * wpr
    if vec_path and not exact:
        top = max_cap if widest else max(cap, wide_cap)
        v = _next_pow2(top) // 2 if _next_pow2(top) > top else top
        # exact tilings of one vector per lane only when rows are too few to fill the device
        min_v = 1 if rows * wpr < 4 * num_cus else 2
        while v >= min_v:
            w = nvec // (64 * v)
            if nvec % (64 * v) == 0 and w <= 16 and fits(w, v):
                wpr, vpl, exact = w, v, True
                break
            v >>= 1
    while rows * wpr < 4 * num_cus and wpr * 2 <= 4:  # few rows: up to 4 waves per row
        if exact and vpl >= 2:
            wpr, vpl = wpr * 2, vpl // 2
        elif not exact and nvec > 64 * wpr * 2:
            wpr *= 2
            vpl = _next_pow2(per_lane(wpr))
        else:
            break
    threads = 256 if 4 % wpr == 0 else 64 * wpr
    return False, wpr, vpl, vec_path and exact, threads


def get_optimal_config(batch_size: int, hidden_size: int,
                       dtype: torch.dtype = torch.float32, num_cus: int = 256) -> dict:
    """Forward launch geometry the HIP dispatcher picks for a [batch_size, hidden_size] input
    (16-byte aligned, contiguous; default tuning), plus the reference's keys
    (reference fused_layernorm/functional.py:47-72).  ``num_cus`` is the device's CU count
    (256 on MI355X)."""
    es = torch.empty((), dtype=dtype).element_size()
    vv = 16 // es
    vec_path = hidden_size % vv == 0
    vec = vv if vec_path else 1
    nvec = hidden_size // vec
    max_cap = 32 // vv if vec_path else 16
    cap = min(max(32, vec) // vec, max_cap)
    wide_cap = min(16 // vv if vec_path else 8, cap)
    raw_cap = wide_cap if (vec_path and vv < 8) else max_cap  # RAW tiles: 16-bit types only
    loop, wpr, vpl, exact, threads = _forward_geometry(batch_size, nvec, cap, wide_cap, raw_cap,
                                                       vec_path, num_cus)
    # Rows past the register tiles: parked in LDS (vector path, <= 8 vectors per thread of a
    # 1024-thread block; LayerNorm keeps half of the row in registers up to twice that), else
    # streamed by the wide-row kernel (rows under 2 GiB).  Few rows split over several blocks
    # each: fewer than a quarter of the CUs where a kernel parked in LDS would run, fewer than
    # 4 per CU where the streamed one would.
    lds = loop and vec_path and nvec <= 8 * 1024
    lds_reg = loop and vec_path and nvec <= 16 * 1024
    wide = loop and not lds and hidden_size * es < 2 ** 31
    max_rows = num_cus // 4 - 1 if (lds or lds_reg) else 4 * num_cus - 1
    split = loop and vec_path and batch_size <= max_rows and hidden_size * es < 2 ** 31
    return {
        "use_mixed_precision": dtype in (torch.float16, torch.bfloat16),
        "threads_per_block": threads,
        "enable_persistent_kernel": not loop or lds or wide,  # persistent grid-stride rows
        "use_vectorized_load": vec > 1,
        "use_tensor_cores": False,  # bandwidth-bound: no MFMA on this path
        "waves_per_row": wpr if not loop else None,
        "vector_elems": vec,
        "vectors_per_lane": vpl if not loop else None,
        "exact_tiling": exact,
        "register_resident": not loop,
        "lds_staged": lds and not split,
        "threads_lds": 1024 if lds and not split else None,
        "wide_streamed": wide and not split,
        "split_rows": split,
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
