"""Fused LayerNorm / RMSNorm for AMD Instinct MI355X (gfx950).

Drop-in for the package of JonSnow1807/Fused-LayerNorm-CUDA-Operator (fused_layernorm/__init__.py):
the same exports (FusedLayerNorm, FusedLayerNormFunction, fused_layer_norm,
replace_torch_layernorm, restore_torch_layernorm) plus RMSNorm, residual-add and fp8-output
variants, all running hand-written HIP kernels.  Importing requires the built extension
(``python build.py`` next to this package); there is no silent fallback.
"""
from .layernorm import (FusedLayerNorm, FusedLayerNormFunction, FusedRMSNorm, fused_layer_norm,
                        fused_rms_norm, replace_layernorm_modules, replace_torch_layernorm,
                        restore_torch_layernorm)
from .ops import (add_layer_norm, add_layer_norm_fp8, add_rms_norm, add_rms_norm_fp8,
                  add_rms_norm_mxfp8, layer_norm, layer_norm_fp8, layer_norm_gelu,
                  layer_norm_mxfp8, rms_norm, rms_norm_fp8, rms_norm_mxfp8)
from . import functional

__version__ = "1.0.0"

__all__ = [
    "FusedLayerNorm",
    "FusedLayerNormFunction",
    "fused_layer_norm",
    "replace_torch_layernorm",
    "restore_torch_layernorm",
    "replace_layernorm_modules",
    "FusedRMSNorm",
    "fused_rms_norm",
    "layer_norm",
    "layer_norm_gelu",
    "rms_norm",
    "add_layer_norm",
    "add_rms_norm",
    "layer_norm_fp8",
    "rms_norm_fp8",
    "add_layer_norm_fp8",
    "add_rms_norm_fp8",
    "layer_norm_mxfp8",
    "rms_norm_mxfp8",
    "add_rms_norm_mxfp8",
    "functional",
]
