"""Host-side concurrency of the C ABI on the GPU: several threads of one fresh process, each on
its own HIP stream, start calling libfln at the same moment (every per-process cache cold) and
must get bit-for-bit the results of the same calls made one at a time (tests/threads_worker.py
runs in a child process so that its caches start cold whatever ran before it)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu


def test_concurrent_threads_from_a_cold_start(gpu_available):
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "threads_worker.py")
    print("[threads] child process: 6 threads x 3 rounds x 8 cases", flush=True)
    r = subprocess.run([sys.executable, "-u", script], capture_output=True, text=True,
                       timeout=280)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "threads ok" in r.stdout, r.stdout[-3000:]
