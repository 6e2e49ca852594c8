"""Seeded workloads of the benchmark configurations and their algorithmic byte model.

Inputs are generated on the CPU with ``torch.Generator().manual_seed(seed)`` (float32, then cast
to the I/O dtype), so a CPU checker and the GPU see bit-identical inputs.  Seed plan: config k
uses seed k for x, k+100 for gamma / weight, k+200 for beta, k+300 for dy and k+400 for the
residual; the 8192 x 4096 fwd+bwd headline reuses config 3's seeds.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    op: str                 # layer_norm | layer_norm_gelu | add_layer_norm | rms_norm_fwd_bwd |
    #                         layer_norm_fwd_bwd | layer_norm_fp8 | add_rms_norm_fp8 |
    #                         layer_norm_gelu_fwd_bwd | add_rms_norm_mxfp8
    rows: int
    cols: int
    dtype: torch.dtype
    seed: int
    eps: float
    gamma: Optional[Tuple[float, float]] = (1.0, 0.1)  # (mean, std) or None
    beta: Optional[Tuple[float, float]] = (0.0, 0.1)
    approximate: str = "none"
    outlier_channels: int = 0
    outlier_scale: float = 1.0
    extra: Dict[str, object] = field(default_factory=dict)


WORKLOADS: Dict[str, Workload] = {w.name: w for w in [
    Workload("c1_ln_fwd_fp32_32x768", "layer_norm", 32, 768, torch.float32, 1, 1e-5),
    Workload("c2_ln_gelu_fp32_17x1023", "layer_norm_gelu", 17, 1023, torch.float32, 2, 1e-5),
    Workload("c2_ln_gelu_fp32_64x4096", "layer_norm_gelu", 64, 4096, torch.float32, 2, 1e-5),
    Workload("c3_add_ln_fwd_bf16_8192x4096", "add_layer_norm", 8192, 4096, torch.bfloat16, 3,
             1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("c4_rms_fwd_bwd_bf16_16384x8192", "rms_norm_fwd_bwd", 16384, 8192, torch.bfloat16,
             4, 1e-6, (1.0, 0.02), None),
    Workload("c5_ln_fp8_bf16_32768x7168", "layer_norm_fp8", 32768, 7168, torch.bfloat16, 5,
             1e-5, (1.0, 0.05), (0.0, 0.05), outlier_channels=7, outlier_scale=20.0),
    # Residual add + RMSNorm -> fp8 at C5's shape (the pre-norm feeding an fp8 GEMM).
    Workload("c6_add_rms_fp8_bf16_32768x7168", "add_rms_norm_fp8", 32768, 7168, torch.bfloat16,
             6, 1e-6, (1.0, 0.05), None, outlier_channels=7, outlier_scale=20.0),
    # Residual add + RMSNorm -> OCP MXFP8 (E4M3 codes + E8M0 scales per 32 elements).
    Workload("c7_add_rms_mxfp8_bf16_32768x7168", "add_rms_norm_mxfp8", 32768, 7168,
             torch.bfloat16, 6, 1e-6, (1.0, 0.05), None, outlier_channels=7,
             outlier_scale=20.0),
    # LayerNorm + GELU (tanh, the reference's form) forward + fused backward, headline shape.
    Workload("ln_gelu_fwd_bwd_bf16_8192x4096", "layer_norm_gelu_fwd_bwd", 8192, 4096,
             torch.bfloat16, 7, 1e-5, (1.0, 0.02), (0.0, 0.02), approximate="tanh"),
    # The same with the exact (erf) GELU, torch.nn.GELU's default.
    Workload("ln_gelu_erf_fwd_bwd_bf16_8192x4096", "layer_norm_gelu_fwd_bwd", 8192, 4096,
             torch.bfloat16, 7, 1e-5, (1.0, 0.02), (0.0, 0.02), approximate="none"),
    Workload("ln_fwd_bwd_bf16_8192x4096", "layer_norm_fwd_bwd", 8192, 4096, torch.bfloat16, 3,
             1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("rms_fwd_bwd_bf16_8192x4096", "rms_norm_fwd_bwd", 8192, 4096, torch.bfloat16, 3,
             1e-6, (1.0, 0.02), None),
    # Wide rows (profiled, not benchmark lines): the RAW-tile forward with the 768-thread
    # register backward (3 vectors per lane), and with the backward's raw tiles at 20480; the
    # LDS-staged forward with half of each row in registers and the two-pass backward at 131072;
    # the GELU backward with gamma / beta in LDS.
    Workload("wide_ln_fwd_bwd_bf16_4096x18432", "layer_norm_fwd_bwd", 4096, 18432,
             torch.bfloat16, 8, 1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("wide_ln_fwd_bwd_bf16_4096x20480", "layer_norm_fwd_bwd", 4096, 20480,
             torch.bfloat16, 8, 1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("wide_ln_fwd_bwd_bf16_512x131072", "layer_norm_fwd_bwd", 512, 131072,
             torch.bfloat16, 9, 1e-5, (1.0, 0.02), (0.0, 0.02)),
    # Few very wide rows: the split forward (each row over 64 blocks) and the two-pass backward
    # with the row statistics split into column chunks.
    Workload("few_rows_ln_fwd_bwd_bf16_64x1048576", "layer_norm_fwd_bwd", 64, 1048576,
             torch.bfloat16, 11, 1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("wide_ln_gelu_erf_fwd_bwd_bf16_4096x16384", "layer_norm_gelu_fwd_bwd", 4096, 16384,
             torch.bfloat16, 10, 1e-5, (1.0, 0.02), (0.0, 0.02), approximate="none"),
    # Narrow rows (profiled, not benchmark lines): where the backward's column reduction is a
    # fixed cost of a short call.
    Workload("narrow_ln_fwd_bwd_bf16_16384x768", "layer_norm_fwd_bwd", 16384, 768,
             torch.bfloat16, 11, 1e-5, (1.0, 0.02), (0.0, 0.02)),
    Workload("narrow_ln_fwd_bwd_bf16_16384x2048", "layer_norm_fwd_bwd", 16384, 2048,
             torch.bfloat16, 12, 1e-5, (1.0, 0.02), (0.0, 0.02)),
]}


def _randn(shape, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def make_inputs(w: Workload, rows: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """CPU tensors x, [residual], [gamma], [beta], [dy] for workload ``w``.  ``rows`` < w.rows
    returns the leading rows of the same full-size draw (identical values)."""
    x = _randn((w.rows, w.cols), w.seed)
    if w.outlier_channels:
        g = torch.Generator().manual_seed(w.seed)
        idx = torch.randperm(w.cols, generator=g)[: w.outlier_channels]
        x[:, idx] *= w.outlier_scale
    out = {"x": x}
    if w.gamma is not None:
        out["gamma"] = w.gamma[0] + w.gamma[1] * _randn((w.cols,), w.seed + 100)
    if w.beta is not None:
        out["beta"] = w.beta[0] + w.beta[1] * _randn((w.cols,), w.seed + 200)
    if w.op in ("layer_norm_fwd_bwd", "rms_norm_fwd_bwd", "layer_norm_gelu_fwd_bwd"):
        out["dy"] = _randn((w.rows, w.cols), w.seed + 300)
    if w.op in ("add_layer_norm", "add_rms_norm_fp8", "add_rms_norm_mxfp8"):
        out["residual"] = _randn((w.rows, w.cols), w.seed + 400)
    out = {k: v.to(w.dtype) for k, v in out.items()}
    if rows is not None and rows < w.rows:
        out = {k: (v[:rows].contiguous() if v.dim() == 2 else v) for k, v in out.items()}
    return out


def algorithmic_bytes(w: Workload, rows: Optional[int] = None) -> Dict[str, int]:
    """Bytes the op must move (reads + writes of its tensors; no workspace), per launch group:
    'fwd', 'bwd' (where applicable) and 'total'.  Stage-1 partial buffers of the backward are
    workspace and excluded."""
    m = w.rows if rows is None else rows
    n = w.cols
    es = torch.empty((), dtype=w.dtype).element_size()
    act = m * n * es
    params = n * es * ((w.gamma is not None) + (w.beta is not None))
    stats = m * 4
    if w.op in ("layer_norm", "layer_norm_gelu"):
        fwd = 2 * act + params
        return {"fwd": fwd, "total": fwd}
    if w.op == "add_layer_norm":
        fwd = 4 * act + params
        return {"fwd": fwd, "total": fwd}
    if w.op == "layer_norm_fp8":
        fwd = act + m * n + stats + params
        return {"fwd": fwd, "total": fwd}
    if w.op == "add_rms_norm_fp8":
        fwd = 3 * act + m * n + stats + params  # x, r read; h, codes, scale written
        return {"fwd": fwd, "total": fwd}
    if w.op == "add_rms_norm_mxfp8":
        fwd = 3 * act + m * n + m * (n // 32) + params  # x, r read; h, codes, E8M0 written
        return {"fwd": fwd, "total": fwd}
    if w.op == "layer_norm_gelu_fwd_bwd":
        fwd = 2 * act + params + 2 * stats
        bwd = 3 * act + params + 2 * stats + 2 * n * 4  # gamma and beta both read
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}
    if w.op == "layer_norm_fwd_bwd":
        fwd = 2 * act + params + 2 * stats
        bwd = 3 * act + n * es + 2 * stats + 2 * n * 4
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}
    if w.op == "rms_norm_fwd_bwd":
        fwd = 2 * act + params + stats
        bwd = 3 * act + n * es + stats + n * 4
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}
    raise ValueError(w.op)
