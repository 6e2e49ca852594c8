"""pytest configuration: the `gpu` marker, import paths and shared fixtures.

Tests marked `gpu` need an MI355X (run on the GPU box); everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fused-layernorm-cuda-operator_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu_available():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return True


@pytest.fixture(autouse=True)
def _announce(request):
    # Name each test before it touches the GPU, so a run that dies mid-test still says which.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield
    # libfln reads its FLN_* knobs once; after monkeypatch has restored the environment (this
    # fixture is torn down after it), re-read them so no test leaves a knob set behind.
    import capi
    if capi._lib is not None:
        capi.reload_tuning()
