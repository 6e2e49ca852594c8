"""``torch.library`` integration of the fused normalization operators.

The operator schemas and their GPU implementations are registered by the compiled extension
(namespace ``fused_layernorm``).  This module adds what torch.compile and autograd need on top:
fake (meta) implementations, so the ops trace with FakeTensors, and autograd formulas that route
the backward through the HIP backward kernels.  It also provides the functional entry points
(``layer_norm``, ``rms_norm``, ``add_layer_norm``, ...), which accept any leading shape and
normalize over the trailing ``normalized_shape`` dimensions.

No reference counterpart: the reference registers no custom ops; its only autograd hook is the
Function in fused_layernorm/layernorm.py:31-109.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple, Union

import torch

from ._ext import load as _load_ext

_ext = _load_ext()  # registers the schemas and the GPU kernels
_ops = torch.ops.fused_layernorm

__all__ = [
    "layer_norm", "layer_norm_gelu", "rms_norm", "add_layer_norm", "add_rms_norm",
    "layer_norm_fp8", "rms_norm_fp8", "add_layer_norm_fp8", "add_rms_norm_fp8",
    "layer_norm_mxfp8", "rms_norm_mxfp8", "add_rms_norm_mxfp8",
]


def _stat_shape(x: torch.Tensor):
    return tuple(x.shape[:-1]) if x.dim() > 1 else (1,)


# ---------------------------------------------------------------------------------------------
# Fake implementations (shape/dtype propagation only).
# ---------------------------------------------------------------------------------------------
@torch.library.register_fake("fused_layernorm::layer_norm_fwd")
def _ln_fwd_fake(input, weight, bias, eps):
    s = _stat_shape(input)
    return (torch.empty_like(input), input.new_empty(s, dtype=torch.float32),
            input.new_empty(s, dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::layer_norm_bwd")
def _ln_bwd_fake(grad_out, input, mean, rstd, weight, bias, output_mask, grad_extra):
    e = input.new_empty((0,))
    return (torch.empty_like(input) if output_mask[0] else e,
            torch.empty_like(weight) if (output_mask[1] and weight is not None) else e,
            torch.empty_like(bias) if (output_mask[2] and bias is not None) else e)


@torch.library.register_fake("fused_layernorm::layer_norm_gelu_fwd")
def _ln_gelu_fake(input, weight, bias, eps, approximate):
    st = _stat_shape(input)
    return (torch.empty_like(input), input.new_empty(st, dtype=torch.float32),
            input.new_empty(st, dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::layer_norm_gelu_bwd")
def _ln_gelu_bwd_fake(grad_out, input, mean, rstd, weight, bias, approximate, output_mask):
    return _ln_bwd_fake(grad_out, input, mean, rstd, weight, bias, output_mask, None)


@torch.library.register_fake("fused_layernorm::rms_norm_fwd")
def _rms_fwd_fake(input, weight, eps):
    return torch.empty_like(input), input.new_empty(_stat_shape(input), dtype=torch.float32)


@torch.library.register_fake("fused_layernorm::rms_norm_bwd")
def _rms_bwd_fake(grad_out, input, rstd, weight, output_mask, grad_extra):
    e = input.new_empty((0,))
    return (torch.empty_like(input) if output_mask[0] else e,
            torch.empty_like(weight) if (output_mask[1] and weight is not None) else e)


@torch.library.register_fake("fused_layernorm::add_layer_norm_fwd")
def _add_ln_fake(input, residual, weight, bias, eps):
    s = _stat_shape(input)
    return (torch.empty_like(input), torch.empty_like(input),
            input.new_empty(s, dtype=torch.float32), input.new_empty(s, dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::add_rms_norm_fwd")
def _add_rms_fake(input, residual, weight, eps):
    return (torch.empty_like(input), torch.empty_like(input),
            input.new_empty(_stat_shape(input), dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::layer_norm_fp8_fwd")
def _ln_fp8_fake(input, weight, bias, eps):
    return (torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device),
            input.new_empty(_stat_shape(input), dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::rms_norm_fp8_fwd")
def _rms_fp8_fake(input, weight, eps):
    return (torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device),
            input.new_empty(_stat_shape(input), dtype=torch.float32))


@torch.library.register_fake("fused_layernorm::add_layer_norm_fp8_fwd")
def _add_ln_fp8_fake(input, residual, weight, bias, eps):
    return (torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device),
            input.new_empty(_stat_shape(input), dtype=torch.float32), torch.empty_like(input))


def _mx_fake(input):
    assert input.shape[-1] % 32 == 0, "MX fp8 output needs a multiple of 32 columns"
    return (torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device),
            torch.empty((*input.shape[:-1], input.shape[-1] // 32), dtype=torch.float8_e8m0fnu,
                        device=input.device))


@torch.library.register_fake("fused_layernorm::layer_norm_mxfp8_fwd")
def _ln_mx_fake(input, weight, bias, eps):
    return _mx_fake(input)


@torch.library.register_fake("fused_layernorm::rms_norm_mxfp8_fwd")
def _rms_mx_fake(input, weight, eps):
    return _mx_fake(input)


@torch.library.register_fake("fused_layernorm::add_rms_norm_mxfp8_fwd")
def _add_rms_mx_fake(input, residual, weight, eps):
    return (*_mx_fake(input), torch.empty_like(input))


@torch.library.register_fake("fused_layernorm::add_rms_norm_fp8_fwd")
def _add_rms_fp8_fake(input, residual, weight, eps):
    return (torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device),
            input.new_empty(_stat_shape(input), dtype=torch.float32), torch.empty_like(input))


# ---------------------------------------------------------------------------------------------
# Autograd formulas.
# ---------------------------------------------------------------------------------------------
def _ln_setup(ctx, inputs, output):
    input, weight, bias, _eps = inputs
    _, mean, rstd = output
    ctx.save_for_backward(input, weight, bias, mean, rstd)
    ctx.mark_non_differentiable(mean, rstd)


def _ln_backward(ctx, gy, _gmean, _grstd):
    input, weight, bias, mean, rstd = ctx.saved_tensors
    mask = [bool(ctx.needs_input_grad[0]),
            weight is not None and bool(ctx.needs_input_grad[1]),
            bias is not None and bool(ctx.needs_input_grad[2])]
    dx, dw, db = _ops.layer_norm_bwd(gy.contiguous(), input, mean, rstd, weight, bias, mask, None)
    return (dx if mask[0] else None, dw if mask[1] else None, db if mask[2] else None, None)


torch.library.register_autograd("fused_layernorm::layer_norm_fwd", _ln_backward,
                                setup_context=_ln_setup)


def _rms_setup(ctx, inputs, output):
    input, weight, _eps = inputs
    _, rstd = output
    ctx.save_for_backward(input, weight, rstd)
    ctx.mark_non_differentiable(rstd)


def _rms_backward(ctx, gy, _grstd):
    input, weight, rstd = ctx.saved_tensors
    mask = [bool(ctx.needs_input_grad[0]), weight is not None and bool(ctx.needs_input_grad[1])]
    dx, dw = _ops.rms_norm_bwd(gy.contiguous(), input, rstd, weight, mask, None)
    return (dx if mask[0] else None, dw if mask[1] else None, None)


torch.library.register_autograd("fused_layernorm::rms_norm_fwd", _rms_backward,
                                setup_context=_rms_setup)


def _ln_gelu_setup(ctx, inputs, output):
    input, weight, bias, _eps, approximate = inputs
    _, mean, rstd = output
    ctx.save_for_backward(input, weight, bias, mean, rstd)
    ctx.approximate = approximate
    ctx.mark_non_differentiable(mean, rstd)


def _ln_gelu_backward(ctx, gy, _gmean, _grstd):
    input, weight, bias, mean, rstd = ctx.saved_tensors
    mask = [bool(ctx.needs_input_grad[0]),
            weight is not None and bool(ctx.needs_input_grad[1]),
            bias is not None and bool(ctx.needs_input_grad[2])]
    dx, dw, db = _ops.layer_norm_gelu_bwd(gy.contiguous(), input, mean, rstd, weight, bias,
                                          ctx.approximate, mask)
    return (dx if mask[0] else None, dw if mask[1] else None, db if mask[2] else None, None,
            None)


torch.library.register_autograd("fused_layernorm::layer_norm_gelu_fwd", _ln_gelu_backward,
                                setup_context=_ln_gelu_setup)


def _add_ln_setup(ctx, inputs, output):
    _input, _residual, weight, bias, _eps = inputs
    _, h, mean, rstd = output
    ctx.save_for_backward(h, weight, bias, mean, rstd)
    ctx.mark_non_differentiable(mean, rstd)


def _add_ln_backward(ctx, gy, gh, _gmean, _grstd):
    # y = LN(h), h = x + r: dL/dh = LN'(gy) + gh, and dL/dx = dL/dr = dL/dh.
    h, weight, bias, mean, rstd = ctx.saved_tensors
    need_h = bool(ctx.needs_input_grad[0] or ctx.needs_input_grad[1])
    mask = [need_h, weight is not None and bool(ctx.needs_input_grad[2]),
            bias is not None and bool(ctx.needs_input_grad[3])]
    if gy is None:
        gy = torch.zeros_like(h)
    dh, dw, db = _ops.layer_norm_bwd(gy.contiguous(), h, mean, rstd, weight, bias, mask,
                                     None if gh is None else gh.contiguous())
    dh = dh if need_h else None
    return (dh if ctx.needs_input_grad[0] else None, dh if ctx.needs_input_grad[1] else None,
            dw if mask[1] else None, db if mask[2] else None, None)


torch.library.register_autograd("fused_layernorm::add_layer_norm_fwd", _add_ln_backward,
                                setup_context=_add_ln_setup)


def _add_rms_setup(ctx, inputs, output):
    _input, _residual, weight, _eps = inputs
    _, h, rstd = output
    ctx.save_for_backward(h, weight, rstd)
    ctx.mark_non_differentiable(rstd)


def _add_rms_backward(ctx, gy, gh, _grstd):
    h, weight, rstd = ctx.saved_tensors
    need_h = bool(ctx.needs_input_grad[0] or ctx.needs_input_grad[1])
    mask = [need_h, weight is not None and bool(ctx.needs_input_grad[2])]
    if gy is None:
        gy = torch.zeros_like(h)
    dh, dw = _ops.rms_norm_bwd(gy.contiguous(), h, rstd, weight, mask,
                               None if gh is None else gh.contiguous())
    dh = dh if need_h else None
    return (dh if ctx.needs_input_grad[0] else None, dh if ctx.needs_input_grad[1] else None,
            dw if mask[1] else None, None)


torch.library.register_autograd("fused_layernorm::add_rms_norm_fwd", _add_rms_backward,
                                setup_context=_add_rms_setup)


# The fp8 outputs (codes, scales) are not differentiable; the residual sum h = x + r is, and
# its gradient passes through to both addends.
def _fp8_residual_setup(ctx, inputs, output):
    q, scale, _h = output
    ctx.mark_non_differentiable(q, scale)


def _fp8_residual_backward(ctx, _gq, _gscale, gh):
    n_rest = 3 if len(ctx.needs_input_grad) == 5 else 2  # (weight, bias, eps) or (weight, eps)
    return (gh if ctx.needs_input_grad[0] else None, gh if ctx.needs_input_grad[1] else None,
            *([None] * n_rest))


torch.library.register_autograd("fused_layernorm::add_layer_norm_fp8_fwd",
                                _fp8_residual_backward, setup_context=_fp8_residual_setup)
torch.library.register_autograd("fused_layernorm::add_rms_norm_fp8_fwd",
                                _fp8_residual_backward, setup_context=_fp8_residual_setup)
torch.library.register_autograd("fused_layernorm::add_rms_norm_mxfp8_fwd",
                                _fp8_residual_backward, setup_context=_fp8_residual_setup)


# ---------------------------------------------------------------------------------------------
# Functional entry points.
# ---------------------------------------------------------------------------------------------
ShapeLike = Union[int, Sequence[int], torch.Size]


def _norm_shape(normalized_shape: ShapeLike) -> Tuple[int, ...]:
    if isinstance(normalized_shape, int):
        return (normalized_shape,)
    return tuple(int(s) for s in normalized_shape)


def _flatten(input: torch.Tensor, normalized_shape: ShapeLike):
    ns = _norm_shape(normalized_shape)
    if len(ns) == 0 or tuple(input.shape[input.dim() - len(ns):]) != ns:
        raise RuntimeError(
            f"Given normalized_shape={list(ns)}, expected input with shape [*, "
            f"{', '.join(str(s) for s in ns)}], but got input of size {list(input.shape)}")
    n = math.prod(ns)
    return input.reshape(-1, n).contiguous(), n


def _flat_param(p: Optional[torch.Tensor]):
    return None if p is None else p.reshape(-1)


def layer_norm(input: torch.Tensor, normalized_shape: ShapeLike,
               weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
               eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm with torch.nn.functional.layer_norm semantics (weight / bias independent)."""
    x, _ = _flatten(input, normalized_shape)
    y, _, _ = _ops.layer_norm_fwd(x, _flat_param(weight), _flat_param(bias), eps)
    return y.view(input.shape)


def layer_norm_gelu(input: torch.Tensor, normalized_shape: ShapeLike,
                    weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                    eps: float = 1e-5, approximate: str = "tanh") -> torch.Tensor:
    """GELU(LayerNorm(x)); approximate='tanh' is the reference's fused GELU, 'none' the exact
    erf form.  Differentiable: the backward recomputes the GELU input from the saved row
    statistics and folds GELU' into the fused LayerNorm backward."""
    x, _ = _flatten(input, normalized_shape)
    y, _, _ = _ops.layer_norm_gelu_fwd(x, _flat_param(weight), _flat_param(bias), eps,
                                       approximate)
    return y.view(input.shape)


def rms_norm(input: torch.Tensor, normalized_shape: ShapeLike,
             weight: Optional[torch.Tensor] = None, eps: Optional[float] = None) -> torch.Tensor:
    """RMSNorm with torch.nn.functional.rms_norm semantics (eps=None -> finfo(dtype).eps)."""
    if eps is None:
        eps = torch.finfo(input.dtype).eps
    ns = _norm_shape(normalized_shape)
    if len(ns) == 1 and not torch.compiler.is_compiling():
        # Eager: autograd in C++ around the kernels (FusedRMSNorm's hot path).
        return _ext.rms_norm_autograd(input, ns[0], weight, eps)
    x, _ = _flatten(input, normalized_shape)
    y, _ = _ops.rms_norm_fwd(x, _flat_param(weight), eps)
    return y.view(input.shape)


def add_layer_norm(input: torch.Tensor, residual: torch.Tensor, normalized_shape: ShapeLike,
                   weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                   eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused residual add + LayerNorm -> (LayerNorm(h), h) with h = input + residual."""
    x, _ = _flatten(input, normalized_shape)
    r, _ = _flatten(residual, normalized_shape)
    y, h, _, _ = _ops.add_layer_norm_fwd(x, r, _flat_param(weight), _flat_param(bias), eps)
    return y.view(input.shape), h.view(input.shape)


def add_rms_norm(input: torch.Tensor, residual: torch.Tensor, normalized_shape: ShapeLike,
                 weight: Optional[torch.Tensor] = None, eps: float = 1e-6
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused residual add + RMSNorm -> (RMSNorm(h), h) with h = input + residual."""
    x, _ = _flatten(input, normalized_shape)
    r, _ = _flatten(residual, normalized_shape)
    y, h, _ = _ops.add_rms_norm_fwd(x, r, _flat_param(weight), eps)
    return y.view(input.shape), h.view(input.shape)


def layer_norm_fp8(input: torch.Tensor, normalized_shape: ShapeLike,
                   weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                   eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm quantized to OCP fp8 e4m3fn -> (codes as torch.float8_e4m3fn, per-row float32
    scale); dequantize with codes.float() * scale[..., None]."""
    x, _ = _flatten(input, normalized_shape)
    q, scale = _ops.layer_norm_fp8_fwd(x, _flat_param(weight), _flat_param(bias), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), scale.view(lead if lead else (1,))


def rms_norm_fp8(input: torch.Tensor, normalized_shape: ShapeLike,
                 weight: Optional[torch.Tensor] = None, eps: float = 1e-6
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm quantized to OCP fp8 e4m3fn -> (codes, per-row float32 scale)."""
    x, _ = _flatten(input, normalized_shape)
    q, scale = _ops.rms_norm_fp8_fwd(x, _flat_param(weight), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), scale.view(lead if lead else (1,))


def add_layer_norm_fp8(input: torch.Tensor, residual: torch.Tensor, normalized_shape: ShapeLike,
                       weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                       eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused residual add + LayerNorm -> fp8: (codes, per-row scale, h = input + residual).
    Gradients flow through h only (to input and residual)."""
    x, _ = _flatten(input, normalized_shape)
    r, _ = _flatten(residual, normalized_shape)
    q, scale, h = _ops.add_layer_norm_fp8_fwd(x, r, _flat_param(weight), _flat_param(bias), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), scale.view(lead if lead else (1,)), h.view(input.shape)


def add_rms_norm_fp8(input: torch.Tensor, residual: torch.Tensor, normalized_shape: ShapeLike,
                     weight: Optional[torch.Tensor] = None, eps: float = 1e-6
                     ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused residual add + RMSNorm -> fp8 (the pre-norm feeding an fp8 GEMM):
    (codes, per-row scale, h = input + residual).  Gradients flow through h only."""
    x, _ = _flatten(input, normalized_shape)
    r, _ = _flatten(residual, normalized_shape)
    q, scale, h = _ops.add_rms_norm_fp8_fwd(x, r, _flat_param(weight), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), scale.view(lead if lead else (1,)), h.view(input.shape)


def layer_norm_mxfp8(input: torch.Tensor, normalized_shape: ShapeLike,
                     weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                     eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm quantized to OCP MXFP8 E4M3 -> (codes float8_e4m3fn, E8M0 block scales
    float8_e8m0fnu [..., n / 32]); dequantize block-wise with codes.float() * scales.float()."""
    x, n = _flatten(input, normalized_shape)
    q, sc = _ops.layer_norm_mxfp8_fwd(x, _flat_param(weight), _flat_param(bias), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), sc.view(*lead, n // 32)


def rms_norm_mxfp8(input: torch.Tensor, normalized_shape: ShapeLike,
                   weight: Optional[torch.Tensor] = None, eps: float = 1e-6
                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm quantized to OCP MXFP8 E4M3 -> (codes, E8M0 block scales)."""
    x, n = _flatten(input, normalized_shape)
    q, sc = _ops.rms_norm_mxfp8_fwd(x, _flat_param(weight), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), sc.view(*lead, n // 32)


def add_rms_norm_mxfp8(input: torch.Tensor, residual: torch.Tensor, normalized_shape: ShapeLike,
                       weight: Optional[torch.Tensor] = None, eps: float = 1e-6
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused residual add + RMSNorm -> OCP MXFP8 E4M3: (codes, E8M0 block scales,
    h = input + residual).  Gradients flow through h only."""
    x, n = _flatten(input, normalized_shape)
    r, _ = _flatten(residual, normalized_shape)
    q, sc, h = _ops.add_rms_norm_mxfp8_fwd(x, r, _flat_param(weight), eps)
    lead = tuple(input.shape[:input.dim() - len(_norm_shape(normalized_shape))])
    return q.view(input.shape), sc.view(*lead, n // 32), h.view(input.shape)
