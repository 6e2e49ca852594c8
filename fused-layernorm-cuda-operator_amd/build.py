"""Build recipe for the MI355X fused normalization library.

Produces, next to this file:
  * ``libfln.so``  -- the C-ABI library (``include/fused_layernorm.h``): HIP kernels for gfx950
    compiled by hipcc directly (no hipify, no CUDA headers, no dual paths);
  * ``fused_layernorm_cuda<EXT_SUFFIX>`` -- the PyTorch binding, the drop-in for the reference's
    extension module of the same name (reference setup.py:6-10), linked against libfln.so;
  * ``libfln_stream.so`` -- streaming reference kernels (``include/fln_stream.h``) that bench.py
    times as the HBM ceiling of each access pattern (not part of the drop-in).

Run ``python build.py`` (or ``__graft_entry__.build()``).  Object files are cached under
``_build/`` and rebuilt when a source or header is newer.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("FLN_OFFLOAD_ARCH", "gfx950")

KERNEL_SOURCES = ["fln_forward.hip", "fln_forward_f32.hip", "fln_forward_bf16.hip",
                  "fln_forward_f16.hip", "fln_forward_f64.hip", "fln_backward.hip", "fln_host.hip"]
BINDING_SOURCE = "fln_torch.cpp"
HEADERS = ["fln_device.h", "fln_internal.h", "fln_forward_impl.h", "fln_gelu_table.h"]

# Packed-fp32 VALU ops are disabled for device code (the host pass warns that it does not know
# the feature; that warning is harmless).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-ffp-contract=fast",
]

LIB_NAME = "libfln.so"
STREAM_SOURCE = "fln_stream.hip"
STREAM_LIB_NAME = "libfln_stream.so"
EXT_NAME = "fused_layernorm_cuda" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")


def _newer(target: str, deps: list[str]) -> bool:
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        l for l in res.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose: bool = False, force: bool = False) -> str:
    """Compile the HIP kernels and link libfln.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    hdrs = [os.path.join(CSRC, h) for h in HEADERS] + [os.path.join(INCLUDE, "fused_layernorm.h")]
    objs, jobs = [], []
    for src in KERNEL_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD, src + ".o")
        objs.append(o)
        if force or _newer(o, [s] + hdrs):
            jobs.append([HIPCC, *DEVICE_FLAGS, "-I", INCLUDE, "-c", s, "-o", o])
    with ThreadPoolExecutor(max_workers=min(8, max(1, len(jobs)))) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    lib = os.path.join(HERE, LIB_NAME)
    if force or jobs or _newer(lib, objs):
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", lib], verbose)
    return lib


def build_stream_library(verbose: bool = False, force: bool = False) -> str:
    """Compile the streaming reference kernels into libfln_stream.so; returns its path."""
    src = os.path.join(CSRC, STREAM_SOURCE)
    deps = [src, os.path.join(CSRC, "fln_device.h"), os.path.join(INCLUDE, "fln_stream.h")]
    lib = os.path.join(HERE, STREAM_LIB_NAME)
    if force or _newer(lib, deps):
        _run([HIPCC, *DEVICE_FLAGS, "-I", INCLUDE, "-shared", src, "-o", lib], verbose)
    return lib


def build_binding(verbose: bool = False, force: bool = False) -> str:
    """Compile the torch binding (host C++ only) against libfln.so; returns its path."""
    import torch
    from torch.utils import cpp_extension as ce

    os.makedirs(BUILD, exist_ok=True)
    src = os.path.join(CSRC, BINDING_SOURCE)
    obj = os.path.join(BUILD, BINDING_SOURCE + ".o")
    out = os.path.join(HERE, EXT_NAME)
    lib = os.path.join(HERE, LIB_NAME)
    incs = ce.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                 os.path.join(ROCM, "include")]
    abi = int(torch.compiled_with_cxx11_abi())
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              "-DTORCH_EXTENSION_NAME=fused_layernorm_cuda", "-DTORCH_API_INCLUDE_EXTENSION_H"]
    if force or _newer(obj, [src, os.path.join(INCLUDE, "fused_layernorm.h")]):
        _run(["g++", *cflags, *[f"-I{i}" for i in incs], "-c", src, "-o", obj], verbose)
    if force or _newer(out, [obj, lib]):
        libdirs = ce.library_paths()
        _run(["g++", "-shared", obj, "-o", out, *[f"-L{d}" for d in libdirs],
              f"-L{HERE}", "-lfln", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
              "-lc10_hip", "-ltorch_hip", "-Wl,-rpath,$ORIGIN",
              *[f"-Wl,-rpath,{d}" for d in libdirs]], verbose)
    return out


def build(verbose: bool = False, force: bool = False) -> None:
    with ThreadPoolExecutor(max_workers=2) as ex:
        stream = ex.submit(build_stream_library, verbose, force)
        build_library(verbose, force)
        stream.result()
    build_binding(verbose, force)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, force="--force" in sys.argv)
    print("built", os.path.join(HERE, LIB_NAME), os.path.join(HERE, STREAM_LIB_NAME), "and",
          os.path.join(HERE, EXT_NAME))
