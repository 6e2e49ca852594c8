"""setup.py: the reference's install commands (`pip install -e .`, README.md:78; setup.py:1-13)
build and install the same two import names here, offline, with hipcc for gfx950.

CPU only: the installed extension is imported (not called) from the installed location in a
fresh interpreter, so the test proves where `fused_layernorm_cuda` and `fused_layernorm` come
from, that `libfln.so` travels with the extension, and that the reference's entry points exist.
"""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fused-layernorm-cuda-operator_amd")
PIP = [sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps", "--no-index",
       "--disable-pip-version-check", "-q"]

# Imported from the installed location: reports where each module came from and checks the
# reference's entry points (csrc/bindings.cpp:41-44, csrc/layernorm_cuda.cpp:198-237).
PROBE = """
import json, os, sys
import fused_layernorm_cuda as ext
import fused_layernorm as pkg
names = ["layernorm", "layernorm_gelu", "forward", "backward", "get_memory_usage",
         "get_performance_hints"]
print(json.dumps({"ext": os.path.realpath(ext.__file__), "pkg": os.path.realpath(pkg.__file__),
                  "version": ext.__version__, "missing": [n for n in names if not hasattr(ext, n)],
                  "classes": [n for n in ("FusedLayerNorm", "FusedLayerNormFunction",
                                          "fused_layer_norm", "replace_torch_layernorm",
                                          "restore_torch_layernorm") if hasattr(pkg, n)]}))
"""


def _env(extra_path=None):
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    if extra_path:
        env["PYTHONPATH"] = extra_path
    return env


def _probe(cwd, env, prelude=""):
    import json
    r = subprocess.run([sys.executable, "-c", prelude + PROBE], cwd=cwd, env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def _check(info, where):
    assert info["ext"].startswith(str(where)), info
    assert info["pkg"].startswith(str(where)), info
    assert info["version"] == "1.0.0"
    assert info["missing"] == []
    assert len(info["classes"]) == 5


def test_setup_build_ext_inplace():
    r = subprocess.run([sys.executable, "setup.py", "-q", "build_ext", "--inplace"], cwd=ROOT,
                       capture_output=True, text=True, timeout=1800)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    names = os.listdir(PKG)
    assert any(n.startswith("fused_layernorm_cuda") and n.endswith(".so") for n in names)
    assert "libfln.so" in names


def test_pip_install_places_the_extension_and_its_library(tmp_path):
    site = tmp_path / "site"
    r = subprocess.run(PIP + ["--target", str(site), ROOT], cwd=ROOT, capture_output=True,
                       text=True, timeout=1800)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert (site / "libfln.so").exists(), "libfln.so must sit beside the extension ($ORIGIN)"
    _check(_probe(tmp_path, _env(str(site))), site)


def test_pip_editable_install_resolves_to_the_source_tree(tmp_path):
    prefix = tmp_path / "prefix"
    site = prefix / "lib" / f"python{sys.version_info[0]}.{sys.version_info[1]}" / "site-packages"
    site.mkdir(parents=True)
    r = subprocess.run(PIP + ["--prefix", str(prefix), "-e", ROOT], cwd=ROOT,
                       env=_env(str(site)), capture_output=True, text=True, timeout=1800)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    # The .pth file of a develop install is read by site.addsitedir (as at interpreter start-up
    # for a real site-packages directory).
    info = _probe(tmp_path, _env(), prelude=f"import site; site.addsitedir({str(site)!r})\n")
    _check(info, os.path.realpath(PKG))
