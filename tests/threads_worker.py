"""Child process of test_gpu_threads.py: several host threads, each on its own HIP stream, make
their first libfln calls at the same moment (cold per-process caches: the calling thread's
device, the tuning snapshot, cached kernel handles and occupancy, the GELU tables), then repeat
a mix of forward and backward calls; every thread's outputs must equal, bit for bit, the same
calls made afterwards one at a time on the default stream (the kernels' results depend only on
the shapes, never on the stream or the thread).  Prints "threads ok" on success."""
import os
import sys
import threading

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests"),
                os.path.join(ROOT, "fused-layernorm-cuda-operator_amd")]

import torch  # noqa: E402

import capi  # noqa: E402
from gpu_calls import ln_backward, ln_forward, rms_backward, rms_forward, workspace  # noqa: E402

# (flavour, dtype, rows, cols): register tiles, odd tiles, the scalar path, the split forward
# with the two-pass backward, GELU with its tables, the fp8 row scale, an fp32 halved tile,
# the 16-bit raw tiles.
CASES = [("ln", torch.bfloat16, 2048, 4096), ("rms", torch.float16, 1000, 768),
         ("ln", torch.float32, 300, 1023), ("ln", torch.bfloat16, 4, 65536),
         ("gelu", torch.bfloat16, 512, 7168), ("fp8", torch.bfloat16, 1024, 5120),
         ("rms", torch.float32, 2048, 4096), ("ln", torch.float16, 64, 20480)]
THREADS = 6
REPEATS = 3


def make_inputs(k, case):
    _, dtype, rows, cols = case
    gen = torch.Generator().manual_seed(1000 + k)
    t = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    return {"x": (t(rows, cols) + 0.3).to(dtype).cuda(), "dy": t(rows, cols).to(dtype).cuda(),
            "g": (1 + 0.1 * t(cols)).to(dtype).cuda(), "b": (0.1 * t(cols)).to(dtype).cuda()}


def run(lib, case, inp):
    kind, dtype, rows, cols = case
    x, dy, g, b = inp["x"], inp["dy"], inp["g"], inp["b"]
    p = capi.ptr
    if kind == "ln":
        y, mean, rstd = ln_forward(lib, x, g, b, 1e-5)
        return [y, mean, rstd, *ln_backward(lib, dy, x, mean, rstd, g)]
    if kind == "rms":
        y, rstd = rms_forward(lib, x, g, 1e-6)
        return [y, rstd, *rms_backward(lib, dy, x, rstd, g)]
    if kind == "gelu":
        y = torch.empty_like(x)
        mean = torch.empty(rows, device="cuda")
        rstd = torch.empty(rows, device="cuda")
        capi.check(lib.fln_layernorm_gelu_forward(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows,
                                                  cols, capi.dtype_code(x), 1e-5, capi.GELU_ERF,
                                                  capi.stream()))
        dx = torch.empty_like(x)
        dg = torch.empty(cols, device="cuda")
        db = torch.empty(cols, device="cuda")
        ws, n = workspace(lib, rows, cols, x)
        capi.check(lib.fln_layernorm_gelu_backward(p(dy), p(x), p(mean), p(rstd), p(g), p(b),
                                                   p(dx), p(dg), p(db), rows, cols,
                                                   capi.dtype_code(x), capi.F32, capi.GELU_ERF,
                                                   p(ws), n, capi.stream()))
        return [y, mean, rstd, dx, dg, db]
    q = torch.empty(rows, cols, device="cuda", dtype=torch.uint8)
    s = torch.empty(rows, device="cuda")
    capi.check(lib.fln_layernorm_fp8_forward(p(x), p(g), p(b), p(q), p(s), None, None, rows, cols,
                                             capi.dtype_code(x), 1e-5, capi.stream()))
    return [q, s]


def main():
    lib = capi.load()  # loads the library; no call into it before the threads start
    inputs = [make_inputs(k, c) for k, c in enumerate(CASES)]
    torch.cuda.synchronize()
    barrier = threading.Barrier(THREADS)
    results = [None] * THREADS
    errors = []

    def worker(t):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                order = list(range(len(CASES)))
                order = order[t % len(order):] + order[:t % len(order)]
                barrier.wait(timeout=60)
                outs = {}
                for _ in range(REPEATS):
                    for k in order:
                        outs[k] = run(lib, CASES[k], inputs[k])
                stream.synchronize()
            results[t] = outs
        except BaseException as e:  # reported by the main thread
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=240)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    reference = {k: run(lib, CASES[k], inputs[k]) for k in range(len(CASES))}
    torch.cuda.synchronize()
    for t in range(THREADS):
        for k, case in enumerate(CASES):
            for i, (got, ref) in enumerate(zip(results[t][k], reference[k])):
                assert torch.equal(got, ref), f"thread {t}, case {case}, output {i} differs"
    print(f"threads ok: {THREADS} threads x {REPEATS} rounds x {len(CASES)} cases", flush=True)


if __name__ == "__main__":
    main()
