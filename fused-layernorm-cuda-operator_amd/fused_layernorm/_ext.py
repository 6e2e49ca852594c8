"""Loader of the compiled extension ``fused_layernorm_cuda`` (HIP kernels behind a torch binding).

The extension is built in-tree next to this package (``python build.py`` in the directory above).
There is no fallback: if it cannot be imported the package import fails loudly, as the
reference's does (fused_layernorm/layernorm.py:22-28).
"""
from __future__ import annotations

import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load():
    import torch  # noqa: F401  (the extension links against libtorch)
    try:
        import fused_layernorm_cuda  # type: ignore
    except ImportError:
        if _ROOT not in sys.path:
            sys.path.insert(0, _ROOT)
        try:
            import fused_layernorm_cuda  # type: ignore
        except ImportError as e:
            raise ImportError(
                "Cannot import fused_layernorm_cuda. Please ensure the HIP extension is built: "
                f"run `python {os.path.join(_ROOT, 'build.py')}`") from e
    return fused_layernorm_cuda


def library_path() -> str:
    """Path of the C-ABI library (libfln.so) the extension links against."""
    return os.path.join(_ROOT, "libfln.so")
