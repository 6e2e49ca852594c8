"""Fused LayerNorm module, autograd Function and functional API (reference-compatible names).

Drop-in for the reference's fused_layernorm/layernorm.py: ``FusedLayerNormFunction``
(:31-109), ``FusedLayerNorm`` (:112-231), ``fused_layer_norm`` (:234-266) and
``replace_torch_layernorm`` / ``restore_torch_layernorm`` (:269-280), with the same signatures,
state_dict keys and error behaviour.  Differences, all supersets of the reference:

* the forward and backward both run HIP kernels (the reference's Python package calls a
  ``forward``/``backward`` binding that is never built, and it has no backward kernel);
* inputs of any rank and multi-dimensional ``normalized_shape`` are handled by flattening to
  rows, where the reference falls back to torch.nn.functional.layer_norm for ranks other than
  2 and 3 (:189-193, :293-294);
* bfloat16 and float16 inputs are supported with float32 statistics.

The calls go through the ``torch.ops.fused_layernorm`` operators, so the module also works inside
``torch.compile``.  ``FusedRMSNorm`` / ``fused_rms_norm`` add RMSNorm on the same kernels.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn
from torch.autograd import Function
from torch.nn import Parameter

from . import ops as _fops
from ._ext import load as _load_ext

fused_layernorm_cuda = _load_ext()
_ops = torch.ops.fused_layernorm
_layer_norm_autograd = fused_layernorm_cuda.layer_norm_autograd
_compiling = torch.compiler.is_compiling


class FusedLayerNormFunction(Function):
    """Autograd Function for the fused LayerNorm (reference layernorm.py:31-109).

    forward(ctx, input, normalized_shape, weight=None, bias=None, eps=1e-5): input must be 2D
    and normalized_shape must equal (input.size(1),) -- a ValueError otherwise, as in the
    reference (:59-65).  Saves (input, weight, bias, mean, rstd) for backward (:76).
    backward returns (grad_input, None, grad_weight, grad_bias, None) (:109).
    """

    @staticmethod
    def forward(ctx, input: torch.Tensor, normalized_shape: Tuple[int, ...],
                weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                eps: float = 1e-5) -> torch.Tensor:
        if input.dim() != 2:
            raise ValueError(f"Expected 2D input, got {input.dim()}D")
        if len(normalized_shape) != 1 or normalized_shape[0] != input.size(1):
            raise ValueError(
                f"normalized_shape {normalized_shape} doesn't match input shape {input.shape}")
        input = input.contiguous()
        output, mean, rstd = _ops.layer_norm_fwd(input, weight, bias, eps)
        ctx.save_for_backward(input, weight, bias, mean, rstd)
        ctx.normalized_shape = normalized_shape
        ctx.eps = eps
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        input, weight, bias, mean, rstd = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        needs_input_grad = bool(ctx.needs_input_grad[0])
        needs_weight_grad = bool(ctx.needs_input_grad[2]) if weight is not None else False
        needs_bias_grad = bool(ctx.needs_input_grad[3]) if bias is not None else False
        mask = [needs_input_grad, needs_weight_grad, needs_bias_grad]
        grad_input, grad_weight, grad_bias = _ops.layer_norm_bwd(
            grad_output, input, mean, rstd, weight, bias, mask, None)
        return (grad_input if needs_input_grad else None, None,
                grad_weight if needs_weight_grad else None,
                grad_bias if needs_bias_grad else None, None)


def _as_shape(normalized_shape) -> Tuple[int, ...]:
    if isinstance(normalized_shape, int):
        return (normalized_shape,)
    return tuple(int(s) for s in normalized_shape)


def _apply_rows(input: torch.Tensor, normalized_shape: Tuple[int, ...],
                weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                eps: float) -> torch.Tensor:
    nd = len(normalized_shape)
    if nd == 0 or tuple(input.shape[input.dim() - nd:]) != normalized_shape:
        raise RuntimeError(
            f"Given normalized_shape={list(normalized_shape)}, expected input with shape "
            f"[*, {', '.join(str(s) for s in normalized_shape)}], but got input of size "
            f"{list(input.shape)}")
    n = math.prod(normalized_shape)
    x2 = input.reshape(-1, n)
    w = None if weight is None else weight.reshape(-1)
    b = None if bias is None else bias.reshape(-1)
    out = FusedLayerNormFunction.apply(x2, (n,), w, b, eps)
    return out.view(input.shape)


class FusedLayerNorm(nn.Module):
    """Drop-in replacement for torch.nn.LayerNorm (reference layernorm.py:112-231).

    Same constructor (normalized_shape int or tuple, eps, elementwise_affine, device, dtype),
    parameters ``weight`` (ones) and ``bias`` (zeros), hence the same state_dict keys as
    nn.LayerNorm.  ``bias=False`` is accepted as in nn.LayerNorm.
    """

    def __init__(self, normalized_shape: Union[int, Tuple[int, ...]], eps: float = 1e-5,
                 elementwise_affine: bool = True, bias: bool = True, device=None,
                 dtype=None) -> None:
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if self.elementwise_affine:
            self.weight = Parameter(torch.empty(self.normalized_shape, **factory_kwargs))
            if bias:
                self.bias = Parameter(torch.empty(self.normalized_shape, **factory_kwargs))
            else:
                self.register_parameter("bias", None)
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        if self.elementwise_affine:
            nn.init.ones_(self.weight)
            if self.bias is not None:
                nn.init.zeros_(self.bias)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if len(self.normalized_shape) == 1 and not _compiling():
            # Eager: autograd in C++ around the kernels (host cost close to nn.LayerNorm's).
            return _layer_norm_autograd(input, self.normalized_shape[0], self.weight, self.bias,
                                        self.eps)
        if input.dim() == 2 and len(self.normalized_shape) == 1:
            return FusedLayerNormFunction.apply(input, self.normalized_shape, self.weight,
                                                self.bias, self.eps)
        return _apply_rows(input, self.normalized_shape, self.weight, self.bias, self.eps)

    def extra_repr(self) -> str:
        return "{normalized_shape}, eps={eps}, elementwise_affine={elementwise_affine}".format(
            **self.__dict__)

    @torch.jit.unused
    def estimate_memory_usage(self, batch_size: int) -> int:
        """Byte estimate with the reference's formula (csrc/layernorm_cuda.cpp:144-164)."""
        hidden_size = math.prod(self.normalized_shape)
        use_mixed_precision = (self.weight.dtype in (torch.float16, torch.bfloat16)
                               if self.weight is not None else False)
        return fused_layernorm_cuda.get_memory_usage(batch_size, hidden_size,
                                                     use_mixed_precision)

    @torch.jit.unused
    def get_performance_hints(self, input_shape: Tuple[int, ...]) -> str:
        """Hints with the reference's thresholds (csrc/layernorm_cuda.cpp:167-195)."""
        if len(input_shape) >= 2:
            batch_size = (input_shape[0] if len(input_shape) == 2
                          else input_shape[0] * input_shape[1])
            hidden_size = input_shape[-1]
            return fused_layernorm_cuda.get_performance_hints(batch_size, hidden_size)
        return "Unable to analyze performance for given input shape"


def fused_layer_norm(input: torch.Tensor, normalized_shape: Tuple[int, ...],
                     weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                     eps: float = 1e-5) -> torch.Tensor:
    """Functional LayerNorm with F.layer_norm's signature (reference layernorm.py:234-266)."""
    ns = _as_shape(normalized_shape)
    if len(ns) == 1 and not _compiling():
        return _layer_norm_autograd(input, ns[0], weight, bias, eps)
    if input.dim() == 2 and len(ns) == 1 and ns[0] == input.size(1):
        return FusedLayerNormFunction.apply(input, ns, weight, bias, eps)
    return _apply_rows(input, ns, weight, bias, eps)


class FusedRMSNorm(nn.Module):
    """RMSNorm module with torch.nn.RMSNorm's constructor and state_dict (``weight``)."""

    def __init__(self, normalized_shape: Union[int, Tuple[int, ...]],
                 eps: Optional[float] = None, elementwise_affine: bool = True, device=None,
                 dtype=None) -> None:
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = Parameter(torch.empty(self.normalized_shape, **factory_kwargs))
        else:
            self.register_parameter("weight", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        if self.elementwise_affine:
            nn.init.ones_(self.weight)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        return _fops.rms_norm(input, self.normalized_shape, self.weight, self.eps)

    def extra_repr(self) -> str:
        return "{normalized_shape}, eps={eps}, elementwise_affine={elementwise_affine}".format(
            **self.__dict__)


def fused_rms_norm(input: torch.Tensor, normalized_shape, weight: Optional[torch.Tensor] = None,
                   eps: Optional[float] = None) -> torch.Tensor:
    """Functional RMSNorm with F.rms_norm's signature."""
    return _fops.rms_norm(input, normalized_shape, weight, eps)


def _fused_like(child: nn.Module) -> Optional[nn.Module]:
    """A fused module computing what `child` computes, sharing its Parameter objects."""
    if isinstance(child, nn.LayerNorm) and not isinstance(child, FusedLayerNorm):
        fused = FusedLayerNorm(child.normalized_shape, eps=child.eps,
                               elementwise_affine=False)
        fused.elementwise_affine = child.elementwise_affine
        fused.weight, fused.bias = child.weight, child.bias
        return fused
    rms_cls = getattr(nn, "RMSNorm", None)
    if rms_cls is not None and isinstance(child, rms_cls) and not isinstance(child, FusedRMSNorm):
        fused = FusedRMSNorm(child.normalized_shape, eps=child.eps, elementwise_affine=False)
        fused.elementwise_affine = child.elementwise_affine
        fused.weight = child.weight
        return fused
    return None


def replace_layernorm_modules(module: nn.Module) -> nn.Module:
    """Swap every nn.LayerNorm (and nn.RMSNorm) inside `module` for FusedLayerNorm
    (FusedRMSNorm) in place, sharing the same Parameter objects (optimizer state, state_dict
    keys and tying are unchanged); returns `module`.

    This is the working form of the reference README's replace_layernorm (README.md:103-122),
    whose setattr of a lambda onto an nn.Module child raises TypeError and whose lambda would
    hand 3-D activations to a kernel that reads only size(0) / size(1)."""
    for name, child in list(module.named_children()):
        fused = _fused_like(child)
        if fused is not None:
            setattr(module, name, fused)
        else:
            replace_layernorm_modules(child)
    return module


def replace_torch_layernorm():
    """Replace torch.nn.LayerNorm with FusedLayerNorm globally (reference layernorm.py:269-273)."""
    torch.nn.LayerNorm = FusedLayerNorm
    print("Successfully replaced torch.nn.LayerNorm with FusedLayerNorm")


def restore_torch_layernorm():
    """Restore the original torch.nn.LayerNorm (reference layernorm.py:276-280)."""
    import importlib
    torch.nn.LayerNorm = importlib.import_module("torch.nn.modules.normalization").LayerNorm
    print("Restored original torch.nn.LayerNorm")
