"""Installable build of the MI355X fused normalization library.

Drop-in for the reference's ``setup.py`` (setup.py:1-13), which builds the extension module
``fused_layernorm_cuda`` with ``CUDAExtension`` / nvcc and is installed with ``pip install -e .``
(README.md:78).  Here the same commands install the same two import names:

* ``fused_layernorm_cuda`` -- the torch binding (host C++, g++), linked against ``libfln.so``, the
  C-ABI library of the hand-written HIP kernels, compiled by hipcc with
  ``--offload-arch=gfx950`` (no hipify, no CUDA headers, no CUDA/HIP dual paths);
* ``fused_layernorm`` -- the Python package (``FusedLayerNorm``, ``functional``, ...).

``build_ext`` runs the hipcc / g++ recipe of ``fused-layernorm-cuda-operator_amd/build.py`` (its
objects are cached under ``_build/`` and rebuilt when a source is newer) and places
``libfln.so`` next to the extension, which finds it through its ``$ORIGIN`` run path.

    pip install --no-build-isolation -e .          # editable, as the reference's README
    pip install --no-build-isolation .             # into site-packages
    python setup.py build_ext --inplace            # in-tree only

``--no-build-isolation`` uses the torch that is installed (the binding compiles against its
headers); there is no package index on these machines.
"""
from __future__ import annotations

import importlib.util
import os
import shutil

from setuptools import Extension, setup
from setuptools.command.build_ext import build_ext

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = "fused-layernorm-cuda-operator_amd"


def _recipe():
    """fused-layernorm-cuda-operator_amd/build.py, loaded by path (no name clash with any
    installed ``build`` module)."""
    path = os.path.join(ROOT, PKG_DIR, "build.py")
    spec = importlib.util.spec_from_file_location("_fln_build_recipe", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class HipccBuildExt(build_ext):
    """Builds ``fused_layernorm_cuda`` with the hipcc recipe instead of setuptools' compiler."""

    def build_extension(self, ext: Extension) -> None:
        recipe = _recipe()
        recipe.build(verbose=bool(self.verbose), force=bool(self.force))
        built = os.path.join(recipe.HERE, recipe.EXT_NAME)
        lib = os.path.join(recipe.HERE, recipe.LIB_NAME)
        target = os.path.abspath(self.get_ext_fullpath(ext.name))
        if target != os.path.abspath(built):
            os.makedirs(os.path.dirname(target), exist_ok=True)
            shutil.copy2(built, target)
            shutil.copy2(lib, os.path.join(os.path.dirname(target), recipe.LIB_NAME))


setup(
    name="fused_layernorm_cuda",
    version="1.0.0",
    description="Fused LayerNorm / RMSNorm operators for AMD Instinct MI355X (gfx950), "
                "hand-written HIP kernels",
    package_dir={"": PKG_DIR},
    packages=["fused_layernorm"],
    ext_modules=[Extension("fused_layernorm_cuda", sources=[])],
    cmdclass={"build_ext": HipccBuildExt},
    python_requires=">=3.8",
    zip_safe=False,
)
