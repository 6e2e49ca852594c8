"""Benchmark of the fused normalization hot path on one MI355X.

Default workload (the headline metric): LayerNorm forward + backward, bf16, 8192 x 4096 -- one
"step" is the forward (y, mean, rstd) plus the backward (dx, dgamma, dbeta) over one batch, with
inputs already resident in HBM.  The RMSNorm forward + backward at the same shape is timed the
same way and reported under "rms_fwd_bwd"; the benchmark configurations C1..C5, C6 / C7
(residual add + RMSNorm -> fp8 with per-row / OCP MX block scales at C5's shape) and LayerNorm +
GELU forward + backward at the headline shape are timed under "configs" (latency for the small
ones, GB/s for the large ones).

The kernels are called through the C ABI (libfln.so) on torch's current HIP stream, with every
output preallocated.  Inputs and outputs rotate over at least 4 buffer sets (>= 2 GiB in all,
8x the 256 MiB Infinity Cache), and a step runs the backward on the set half the rotation away
from the forward's, so no kernel finds its inputs in a cache from an earlier launch (as in
training, where a layer's backward comes long after its forward).

Prints ONE JSON line.  `value` = algorithmic bytes of one step / measured step time, in GB/s.
`roofline` covers the backward call (fln_layernorm_backward: stage-1 kernel + column
reduction), the larger of the two, timed with HIP events on its launch stream; its `traffic`
comes from two rocprofv3 counter passes (FETCH_SIZE, then WRITE_SIZE) over a child run of this
script (--kernel-loop), each scaled by what the counter reads for a device copy of known size.
`stream_ceilings` times hand-written streaming kernels (libfln_stream.so) of each access
pattern as the HBM ceiling the kernels are judged against (and, per bandwidth-bound config, at
that config's own tensor size: `configs[*].stream_ceiling`).  `reference_paths` times the
reference's own call paths with its own methods: the binding `fused_layernorm_cuda.layernorm`
at the shapes of its published latencies, the `FusedLayerNorm` module against nn.LayerNorm
at the shapes of its performance-regression test, and the binding at the shapes of its
large-row bandwidth table (fp32, with the 1R1W stream of the same size).  `cpu_baseline` times the reference's
CPU path (torch-CPU F.layer_norm + autograd backward, which the reference's module falls back to
off the GPU) on the full headline workload with the process's host threads; the C oracle
(oracle/fln_oracle.c, the "port") on a row sample is nested beside it.
"""
from __future__ import annotations

import argparse
import csv
import functools
import glob
import json
import os
import platform
import shutil
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "fused-layernorm-cuda-operator_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "HBM GB/s (% of peak) + µs/call, LN/RMSNorm fwd+bwd bf16 8192×4096"
HEADLINE = "ln_fwd_bwd_bf16_8192x4096"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 2 * 2 ** 30
CALIBRATION_COPY_BYTES = 256 * 2 ** 20
CONFIGS = ("c1_ln_fwd_fp32_32x768", "c2_ln_gelu_fp32_17x1023", "c2_ln_gelu_fp32_64x4096",
           "c3_add_ln_fwd_bf16_8192x4096", "c4_rms_fwd_bwd_bf16_16384x8192",
           "c5_ln_fp8_bf16_32768x7168", "c6_add_rms_fp8_bf16_32768x7168",
           "c7_add_rms_mxfp8_bf16_32768x7168", "ln_gelu_fwd_bwd_bf16_8192x4096",
           "ln_gelu_erf_fwd_bwd_bf16_8192x4096")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes (roofline.traffic = null)")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1..C7 timings")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the LayerNorm headline (no RMSNorm line, no configs); "
                         "used for per-kernel profiles")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate host time budget of the CPU baseline")
    ap.add_argument("--kernel-loop", metavar="WORKLOAD", default=None,
                    help="(profiling child) launch WORKLOAD's forward and backward --iters "
                         "times each, then a device copy of known size, and exit")
    ap.add_argument("--stream-loop", metavar="PAT:THREADS:BLOCKS_PER_CU:UNROLL:DEPTH,...",
                    default=None,
                    help="(profiling child) launch the streaming kernels of libfln_stream.so "
                         "(64 MiB per stream, rotating sets) --iters times per listed pattern and "
                         "launch shape, and exit")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--stream-bytes", type=int, default=64 << 20,
                    help="bytes per stream of --stream-loop (default 64 MiB)")
    ap.add_argument("--traffic-configs", action="store_true",
                    help="instead of the bench line: HBM traffic (two rocprofv3 counter passes "
                         "each) and call times of every bandwidth-bound config (C3..C7, LN+GELU)")
    ap.add_argument("--large-rows-only", action="store_true",
                    help="instead of the bench line: only the reference's large-row table "
                         "(reference_paths.large_rows_fp32), one JSON line; used for its "
                         "kernel profile")
    return ap.parse_args()


class _Recorder:
    """Stands in for the library while a call's arguments are built: records the bound call
    instead of making it."""

    def __init__(self, lib):
        self._lib, self.call = lib, None

    def __getattr__(self, name):
        fn = getattr(self._lib, name)

        def record(*args):
            self.call = functools.partial(fn, *args)
            return 0
        return record


class Runner:
    """Preallocated buffer sets + C-ABI launches for one workload.  Each (buffer set, stream)
    call is bound once (ctypes arguments built up front, as a C caller holds its pointers), so
    the timed loops measure the library and the launch, not Python argument conversion."""

    def __init__(self, lib, capi, torch, w, inputs):
        self.lib, self.capi, self.torch, self.w = lib, capi, torch, w
        dev = "cuda"
        x = inputs["x"]
        set_bytes = x.numel() * x.element_size() * (4 if ("dy" in inputs or
                                                         "residual" in inputs) else 2)
        self.nsets = min(16, max(4, -(-ROTATE_BYTES // set_bytes)))
        self.sets = []
        for k in range(self.nsets):
            s = {n: t.to(dev) for n, t in inputs.items()}
            if k > 0:  # distinct buffers, same values
                s = {n: t.clone() for n, t in s.items()}
            s["y"] = torch.empty_like(s["x"])
            if w.op in ("add_layer_norm", "add_rms_norm_fp8", "add_rms_norm_mxfp8"):
                s["h"] = torch.empty_like(s["x"])
            if w.op == "add_rms_norm_mxfp8":
                s["q"] = torch.empty(s["x"].shape, device=dev, dtype=torch.uint8)
                s["bscale"] = torch.empty(w.rows, w.cols // 32, device=dev, dtype=torch.uint8)
            if w.op in ("layer_norm_fp8", "add_rms_norm_fp8"):
                s["q"] = torch.empty(s["x"].shape, device=dev, dtype=torch.uint8)
                s["scale"] = torch.empty(w.rows, device=dev)
            s["mean"] = torch.empty(w.rows, device=dev)
            s["rstd"] = torch.empty(w.rows, device=dev)
            if "dy" in s:
                s["dx"] = torch.empty_like(s["x"])
            self.sets.append(s)
        self.rows, self.cols = w.rows, w.cols
        self.code = capi.dtype_code(self.sets[0]["x"])
        self.has_bwd = "dy" in inputs
        self.ws_bytes = lib.fln_backward_workspace_bytes(self.rows, self.cols, self.code)
        self.ws = torch.empty(max(1, self.ws_bytes // 4), device=dev)
        self.dg = torch.empty(self.cols, device=dev)
        self.db = torch.empty(self.cols, device=dev)
        self.i = 0
        self._calls = {}

    def _bound(self, kind, s, stream):
        key = (kind, id(s), stream.value if hasattr(stream, "value") else stream)
        call = self._calls.get(key)
        if call is None:
            lib, rec = self.lib, _Recorder(self.lib)
            self.lib = rec
            try:
                (self._fwd_args if kind == "fwd" else self._bwd_args)(s, stream)
            finally:
                self.lib = lib
            call = self._calls[key] = rec.call
        return call

    def fwd(self, s, stream):
        self.capi.check(self._bound("fwd", s, stream)())

    def bwd(self, s, stream):
        self.capi.check(self._bound("bwd", s, stream)())

    def _fwd_args(self, s, stream):
        c, p = self.capi, self.capi.ptr
        if self.w.op == "add_layer_norm":
            rc = self.lib.fln_add_layernorm_forward(
                p(s["x"]), p(s["residual"]), p(s.get("gamma")), p(s.get("beta")), p(s["h"]),
                p(s["y"]), None, None, self.rows, self.cols, self.code, self.w.eps, stream)
        elif self.w.op == "add_rms_norm_fp8":
            rc = self.lib.fln_add_rmsnorm_fp8_forward(
                p(s["x"]), p(s["residual"]), p(s.get("gamma")), p(s["h"]), p(s["q"]),
                p(s["scale"]), None, self.rows, self.cols, self.code, self.w.eps, stream)
        elif self.w.op == "add_rms_norm_mxfp8":
            rc = self.lib.fln_add_rmsnorm_mxfp8_forward(
                p(s["x"]), p(s["residual"]), p(s.get("gamma")), p(s["h"]), p(s["q"]),
                p(s["bscale"]), None, self.rows, self.cols, self.code, self.w.eps, stream)
        elif self.w.op == "layer_norm_fp8":
            rc = self.lib.fln_layernorm_fp8_forward(
                p(s["x"]), p(s.get("gamma")), p(s.get("beta")), p(s["q"]), p(s["scale"]), None,
                None, self.rows, self.cols, self.code, self.w.eps, stream)
        elif self.w.op in ("layer_norm", "layer_norm_gelu"):
            gelu = {"none": c.GELU_ERF, "tanh": c.GELU_TANH}[self.w.approximate]
            if self.w.op == "layer_norm":
                rc = self.lib.fln_layernorm(p(s["x"]), p(s.get("gamma")), p(s.get("beta")),
                                            p(s["y"]), self.rows, self.cols, self.code,
                                            self.w.eps, stream)
            else:
                rc = self.lib.fln_layernorm_gelu(p(s["x"]), p(s.get("gamma")), p(s.get("beta")),
                                                 p(s["y"]), self.rows, self.cols, self.code,
                                                 self.w.eps, gelu, stream)
        elif self.w.op == "layer_norm_gelu_fwd_bwd":
            rc = self.lib.fln_layernorm_gelu_forward(
                p(s["x"]), p(s.get("gamma")), p(s.get("beta")), p(s["y"]), p(s["mean"]),
                p(s["rstd"]), self.rows, self.cols, self.code, self.w.eps, self._gelu(), stream)
        elif self.w.op.startswith("rms"):
            rc = self.lib.fln_rmsnorm_forward(p(s["x"]), p(s.get("gamma")), p(s["y"]),
                                              p(s["rstd"]), self.rows, self.cols, self.code,
                                              self.w.eps, stream)
        else:
            rc = self.lib.fln_layernorm_forward(p(s["x"]), p(s.get("gamma")), p(s.get("beta")),
                                                p(s["y"]), p(s["mean"]), p(s["rstd"]),
                                                self.rows, self.cols, self.code, self.w.eps,
                                                stream)
        c.check(rc)

    def _bwd_args(self, s, stream):
        c, p = self.capi, self.capi.ptr
        if self.w.op == "layer_norm_gelu_fwd_bwd":
            rc = self.lib.fln_layernorm_gelu_backward(
                p(s["dy"]), p(s["x"]), p(s["mean"]), p(s["rstd"]), p(s.get("gamma")),
                p(s.get("beta")), p(s["dx"]), p(self.dg), p(self.db), self.rows, self.cols,
                self.code, c.F32, self._gelu(), p(self.ws), self.ws_bytes, stream)
        elif self.w.op.startswith("rms"):
            rc = self.lib.fln_rmsnorm_backward(p(s["dy"]), p(s["x"]), p(s["rstd"]),
                                               p(s.get("gamma")), None, p(s["dx"]), p(self.dg),
                                               self.rows, self.cols, self.code, c.F32,
                                               p(self.ws), self.ws_bytes, stream)
        else:
            rc = self.lib.fln_layernorm_backward(p(s["dy"]), p(s["x"]), p(s["mean"]),
                                                 p(s["rstd"]), p(s.get("gamma")), None,
                                                 p(s["dx"]), p(self.dg), p(self.db), self.rows,
                                                 self.cols, self.code, c.F32, p(self.ws),
                                                 self.ws_bytes, stream)
        c.check(rc)

    def _gelu(self):
        return {"none": self.capi.GELU_ERF, "tanh": self.capi.GELU_TANH}[self.w.approximate]

    def prime(self, stream):
        """One forward per set, so every set holds the statistics its backward reads."""
        for s in self.sets:
            self.fwd(s, stream)

    def step(self, stream):
        """Forward on set i, backward on set i + nsets / 2.  Every set a kernel reads was last
        touched nsets / 2 steps earlier (>= 1 GiB of other traffic since), never by the launch
        just before it: with the backward on set i + 1, the next step's forward would read the
        x that backward had just streamed through the Infinity Cache."""
        k = self.i
        self.i += 1
        self.fwd(self.sets[k % self.nsets], stream)
        if self.has_bwd:
            self.bwd(self.sets[(k + self.nsets // 2) % self.nsets], stream)

    def time_region(self, fn, n, stream_obj):
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream_obj)
        for _ in range(n):
            fn()
        e1.record(stream_obj)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms


def warm_clocks(fn, seconds=0.3):
    """Run `fn` back to back for `seconds` of wall time so the GPU leaves its idle clock state
    before anything is timed (the first ~100 ms of work run measurably slower)."""
    import torch
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_launch_group(runner, which, n, stream, stream_obj):
    """Average duration (ms) of one forward or backward call, rotating buffer sets."""
    it = [0]

    def one():
        s = runner.sets[it[0] % runner.nsets]
        it[0] += 1
        (runner.fwd if which == "fwd" else runner.bwd)(s, stream)

    for _ in range(3):
        one()
    return runner.time_region(one, n, stream_obj)


# ------------------------------------------------------------------------------------------------
# HBM traffic from hardware counters.
# ------------------------------------------------------------------------------------------------
def kernel_loop(args):
    """Profiling child: forward and backward of one workload --iters times each (after one
    forward per buffer set), then --iters copies of CALIBRATION_COPY_BYTES for the counter
    calibration."""
    import torch
    import capi
    from fused_layernorm.testing import WORKLOADS, make_inputs

    lib = capi.load()
    stream = capi.stream()
    w = WORKLOADS[args.kernel_loop]
    r = Runner(lib, capi, torch, w, make_inputs(w))
    r.prime(stream)
    for i in range(args.iters):
        r.fwd(r.sets[i % r.nsets], stream)
    if r.has_bwd:
        for i in range(args.iters):
            r.bwd(r.sets[i % r.nsets], stream)
    torch.cuda.synchronize()
    del r
    torch.cuda.empty_cache()
    a = torch.empty(CALIBRATION_COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda").normal_()
    b = torch.empty_like(a)
    for _ in range(args.iters):
        b.copy_(a)
    torch.cuda.synchronize()
    print("kernel loop done", flush=True)


def stream_loop(args):
    """Profiling child: --iters launches of each listed streaming kernel (pattern 0 1R1W, 1 2R1W,
    2 2R2W, 3 1R + half W) at the listed launch shape, --stream-bytes per stream (64 MiB by
    default) over rotating sets; the counter passes compare the normalization kernels with
    these."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(PKG, "libfln_stream.so"))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.fln_stream_run.argtypes = [i32, vp, vp, vp, vp, i64, i32, i32, i32, i32, i32, i32, vp]
    lib.fln_stream_run.restype = i32
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = lib.fln_stream_cu_count()
    nbytes = args.stream_bytes
    nsets = max(2, min(8, -(-ROTATE_BYTES // (4 * nbytes))))
    sets = [[torch.empty(nbytes // 4, dtype=torch.int32, device="cuda") for _ in range(4)]
            for _ in range(nsets)]
    for st4 in sets:
        for t in st4[:2]:
            t.random_(0, 2 ** 31 - 1)
    for spec in args.stream_loop.split(","):
        pat, thr, bpc, u, pd = (int(v) for v in spec.split(":"))
        for k in range(args.iters):
            a, b, c, d = sets[k % nsets]
            rc = lib.fln_stream_run(pat, a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(),
                                    nbytes, thr, bpc * cus, u, pd, 2, 2, sp)
            if rc != 0:
                raise RuntimeError(f"fln_stream_run {spec}: {rc}")
    torch.cuda.synchronize()
    print("stream loop done", flush=True)


def _counter_rows(outdir):
    files = glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True)
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def pmc_traffic(workload, iters=20):
    """Per-call HBM bytes of the forward and backward of `workload` from two rocprofv3 --pmc
    passes over `bench.py --kernel-loop`.  FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are each
    divided by what the same counter reads per byte of a device-to-device copy of known size
    (torch's copy kernel, CALIBRATION_COPY_BYTES read and written): on gfx950 FETCH_SIZE reads
    half the copied bytes and WRITE_SIZE all of them.  Returns (dict, None) or (None, reason)."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    base = os.path.join(ROOT, "gpurun_out")
    os.makedirs(base, exist_ok=True)
    work = tempfile.mkdtemp(prefix="bench_pmc_", dir=base)
    env = dict(os.environ, TMPDIR="/tmp")
    counts = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        outdir = os.path.join(work, counter)
        cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", counter, "--output-format", "csv",
               "-d", outdir, "-o", "pmc", "--", sys.executable, os.path.abspath(__file__),
               "--kernel-loop", workload, "--iters", str(iters)]
        print(f"bench.py: counter pass {counter}", file=sys.stderr, flush=True)
        with open(os.path.join(work, counter + ".log"), "w") as log:
            rc = subprocess.run(cmd, cwd="/tmp", env=env, stdout=log, stderr=subprocess.STDOUT)
        rows = _counter_rows(outdir)
        if not rows:
            return None, f"{counter} pass produced no counter rows (rc {rc.returncode})"
        rows = [r for r in rows if r.get("Counter_Name") == counter]
        rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0) or 0))
        counts[counter] = [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows]

    def avg_kib(counter, pred):
        vals = [v for name, v in counts[counter] if pred(name)]
        return statistics.fmean(vals) if vals else None

    def copy_kib(counter):
        # The calibration copies are the child's last `iters` copy dispatches (earlier ones
        # are the buffer-set clones).
        copies = [v for name, v in counts[counter] if "copy" in name.lower()][-iters:]
        return statistics.fmean(copies) if len(copies) == iters else None

    cal = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        kib = copy_kib(counter)
        if not kib:
            return None, f"no calibration copy found in the {counter} pass"
        cal[counter] = kib * 1024.0 / CALIBRATION_COPY_BYTES  # counted bytes per true byte

    def call_bytes(names):
        total = 0.0
        detail = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            b = 0.0
            for n in names:
                kib = avg_kib(counter, lambda k, n=n: n in k)
                if kib is None:
                    return None, None
                b += kib * 1024.0 / cal[counter]
            detail[counter.split("_")[0].lower()] = int(round(b))
            total += b
        return int(round(total)), detail

    fwd_total, fwd_detail = call_bytes(["fwd_reg_kernel"])
    bwd_total, bwd_detail = call_bytes(["bwd_reg_kernel", "col_reduce_kernel"])
    return {"fwd": fwd_total, "fwd_detail": fwd_detail, "bwd": bwd_total,
            "bwd_detail": bwd_detail,
            "calibration": {"FETCH_SIZE": round(cal["FETCH_SIZE"], 4),
                            "WRITE_SIZE": round(cal["WRITE_SIZE"], 4),
                            "copy_bytes": CALIBRATION_COPY_BYTES},
            "passes": f"rocprofv3 --pmc FETCH_SIZE | WRITE_SIZE -- bench.py --kernel-loop "
                      f"{workload} --iters {iters}"}, None


# ------------------------------------------------------------------------------------------------
# CPU baselines.
# ------------------------------------------------------------------------------------------------
def cpu_threads():
    """Host threads for the CPU baselines: the process's thread budget (OMP_NUM_THREADS, which
    the GPU boxes set to their CPU share), else every CPU the host reports."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    return max(1, n if n > 0 else (os.cpu_count() or 1))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(run, seconds, min_runs=3, warmup=2):
    for _ in range(warmup):
        run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def torch_cpu_baseline(w, seconds):
    """The reference's CPU path on the full workload: its module falls back to
    torch.nn.functional.layer_norm off the GPU (fused_layernorm/layernorm.py:189-193), here
    F.layer_norm (F.rms_norm for RMS) plus its autograd backward (dx, dgamma, dbeta) on torch-CPU,
    in the workload's dtype, on every host thread of the process's budget.  Full size: the
    tensors (64 MiB each at 8192 x 4096 bf16) exceed the host's last-level cache, as on the GPU."""
    import torch
    from fused_layernorm.testing import algorithmic_bytes, make_inputs

    threads = cpu_threads()
    torch.set_num_threads(threads)
    inp = make_inputs(w)
    x = inp["x"].requires_grad_(True)
    g = inp.get("gamma")
    b = inp.get("beta")
    params = [t.requires_grad_(True) for t in (g, b) if t is not None]
    dy = inp["dy"]
    rms = w.op.startswith("rms")

    def run():
        if rms:
            y = torch.nn.functional.rms_norm(x, (w.cols,), g, w.eps)
        else:
            y = torch.nn.functional.layer_norm(x, (w.cols,), g, b, w.eps)
        torch.autograd.grad(y, [x] + params, dy)

    med, n = _median_time(run, seconds)
    return {"value": round(algorithmic_bytes(w)["total"] / med / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "reference",
            "path": ("torch-CPU F.layer_norm / F.rms_norm + autograd: what the reference module "
                     "runs off the GPU (fused_layernorm/layernorm.py:189-193)"),
            "sample": (f"full {w.rows} x {w.cols} {str(w.dtype).replace('torch.', '')} step of "
                       f"{w.name} (the reference's CPU path: F.layer_norm + autograd backward of "
                       f"x, gamma, beta), median of {n} runs, {med * 1e3:.1f} ms per step"),
            "ms_per_step": round(med * 1e3, 2), "torch_threads": torch.get_num_threads(),
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count()}


def cpu_port_baseline(w, seconds):
    """The C oracle (oracle/fln_oracle.c: scalar C port, one thread, fp64 accumulation) on a
    bounded row sample of the workload."""
    from oracle import c_oracle
    from fused_layernorm.testing import algorithmic_bytes, make_inputs

    c_oracle.load()
    rows = 256
    inp = make_inputs(w, rows)
    f = {k: v.float().numpy() for k, v in inp.items()}
    rms = w.op.startswith("rms")

    def run():
        if rms:
            c_oracle.rmsnorm_fwd(f["x"], f.get("gamma"), w.eps)
            c_oracle.rmsnorm_bwd(f["dy"], f["x"], f.get("gamma"), w.eps)
        else:
            c_oracle.layernorm_fwd(f["x"], f.get("gamma"), f.get("beta"), w.eps)
            c_oracle.layernorm_bwd(f["dy"], f["x"], f.get("gamma"), w.eps)

    med, n = _median_time(run, seconds, warmup=1)
    return {
        "value": round(algorithmic_bytes(w, rows)["total"] / med / 1e9, 3), "unit": "GB/s",
        "cores": 1, "kind": "port",
        "sample": (f"{rows} of {w.rows} rows of the same seeded workload ({w.name}), "
                   f"C oracle fwd+bwd (fp64 accumulation), median of {n} runs "
                   f"({med * 1e3:.1f} ms per {rows}-row fwd+bwd)"),
        "ms_per_step_full_size_extrapolated": round(med * (w.rows / rows) * 1e3, 1),
    }


# Launch shapes of the streaming reference kernels timed for each access pattern: (threads,
# blocks per CU, 16-byte vectors per thread per tile, tiles of loads in flight), the best few of a
# sweep over 256-1024 threads, 1-8 blocks per CU, 1-4 vectors and 1-4 tiles on MI355X (all with
# non-temporal loads and stores, which beat the default policy for every pattern).
STREAM_SHAPES = {
    0: ((512, 1, 2, 1), (256, 2, 1, 2), (256, 4, 1, 1), (512, 2, 2, 2)),
    1: ((512, 1, 1, 1), (512, 1, 2, 1), (512, 1, 1, 2), (1024, 1, 1, 1)),
    2: ((256, 2, 1, 4), (256, 1, 2, 3), (512, 1, 1, 1), (256, 1, 1, 2)),
    3: ((512, 1, 1, 3), (256, 2, 1, 3), (512, 1, 2, 2), (512, 1, 4, 1)),
}
STREAM_NAMES = {0: "1r1w", 1: "2r1w", 2: "2r2w", 3: "1r_half_w"}
STREAM_MOVED = {0: 2.0, 1: 3.0, 2: 4.0, 3: 1.5}  # bytes moved per input-stream byte


def stream_ceilings(torch, nbytes, fwd_bytes=None, bwd_bytes=None, n=100, patterns=None):
    """HBM ceiling of each access pattern on this device: the streaming reference kernels of
    libfln_stream.so (include/fln_stream.h; raw buffer loads / stores, persistent grid, a ring of
    loads in flight: the normalization kernels' own idioms with nothing computed) over streams of
    `nbytes` each, rotating over >= 2 GiB, best launch shape of STREAM_SHAPES, HIP events on the
    launch stream.  The step ceiling is the headline step's algorithmic bytes with the forward's
    at the 1R1W rate and the backward's at the 2R1W rate.  `patterns`: the pattern numbers to
    time (default: all four)."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(PKG, "libfln_stream.so"))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.fln_stream_run.argtypes = [i32, vp, vp, vp, vp, i64, i32, i32, i32, i32, i32, i32, vp]
    lib.fln_stream_run.restype = i32
    st = torch.cuda.current_stream()
    sp = ctypes.c_void_p(st.cuda_stream)
    cus = lib.fln_stream_cu_count()
    nsets = max(4, -(-ROTATE_BYTES // (4 * nbytes)))
    sets = [[torch.empty(nbytes // 4, dtype=torch.int32, device="cuda") for _ in range(4)]
            for _ in range(nsets)]
    for st4 in sets:
        for t in st4[:2]:
            t.random_(0, 2 ** 31 - 1)
    res = {}
    for pat, shapes in STREAM_SHAPES.items():
        if patterns is not None and pat not in patterns:
            continue
        best = None
        for thr, bpc, u, pd in shapes:
            k = [0]

            def one():
                a, b, c, d = sets[k[0] % nsets]
                k[0] += 1
                rc = lib.fln_stream_run(pat, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                        d.data_ptr(), nbytes, thr, bpc * cus, u, pd, 2, 2, sp)
                if rc != 0:
                    raise RuntimeError(f"fln_stream_run pattern {pat}: {rc}")
            for _ in range(10):
                one()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(n):
                one()
            e1.record(st)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / n * 1e3
            rate = nbytes * STREAM_MOVED[pat] / (us * 1e-6) / 1e9
            if best is None or rate > best[0]:
                best = (rate, us, (thr, bpc, u, pd))
        res[STREAM_NAMES[pat] + "_gbs"] = round(best[0], 1)
        res[STREAM_NAMES[pat] + "_shape"] = {"threads": best[2][0], "blocks_per_cu": best[2][1],
                                             "vectors_per_thread": best[2][2],
                                             "tiles_in_flight": best[2][3],
                                             "us_per_call": round(best[1], 2)}
    del sets
    torch.cuda.empty_cache()
    if fwd_bytes is not None and "1r1w_gbs" in res and "2r1w_gbs" in res:
        step_s = fwd_bytes / (res["1r1w_gbs"] * 1e9) + bwd_bytes / (res["2r1w_gbs"] * 1e9)
        res["step_ceiling_gbs"] = round((fwd_bytes + bwd_bytes) / step_s / 1e9, 1)
        res["what"] = (f"libfln_stream.so kernels, {nbytes >> 20} MiB per stream (the headline's "
                       "tensor size), rotating >= 2 GiB, best of STREAM_SHAPES; step ceiling = "
                       "the step's algorithmic bytes at the 1R1W (forward) and 2R1W (backward) "
                       "rates")
    return res


# Access pattern of each bandwidth-bound config's calls and its per-stream size (the size of its
# largest input), for ceilings measured at the config's own size: (forward pattern, backward
# pattern or None, bytes per stream).  C6 / C7 (two reads, a full and a half-width write) have
# no stream kernel of their own pattern.
CONFIG_PATTERNS = {
    "c3_add_ln_fwd_bf16_8192x4096": (2, None, 8192 * 4096 * 2),
    "c4_rms_fwd_bwd_bf16_16384x8192": (0, 1, 16384 * 8192 * 2),
    "c5_ln_fp8_bf16_32768x7168": (3, None, 32768 * 7168 * 2),
    "ln_gelu_fwd_bwd_bf16_8192x4096": (0, 1, 8192 * 4096 * 2),
    "ln_gelu_erf_fwd_bwd_bf16_8192x4096": (0, 1, 8192 * 4096 * 2),
}


def config_ceiling(torch, name, fwd_bytes, bwd_bytes, cache):
    """Streaming ceiling (GB/s) of config `name`'s call pattern at its own tensor size: the
    forward's pattern rate, or for a forward + backward step the step's algorithmic bytes at the
    forward's and backward's pattern rates.  `cache` maps (pattern, bytes) -> GB/s."""
    fpat, bpat, nbytes = CONFIG_PATTERNS[name]
    want = [p for p in (fpat, bpat) if p is not None and (p, nbytes) not in cache]
    if want:
        r = stream_ceilings(torch, nbytes, patterns=want)
        for p in want:
            cache[(p, nbytes)] = r[STREAM_NAMES[p] + "_gbs"]
    if bpat is None:
        return cache[(fpat, nbytes)], STREAM_NAMES[fpat], nbytes
    t = fwd_bytes / (cache[(fpat, nbytes)] * 1e9) + bwd_bytes / (cache[(bpat, nbytes)] * 1e9)
    return ((fwd_bytes + bwd_bytes) / t / 1e9,
            f"{STREAM_NAMES[fpat]} + {STREAM_NAMES[bpat]}", nbytes)


# The reference's published small-shape latencies ("optimal": 500 back-to-back calls on one
# tensor, HIP/CUDA events; publication_validation_results.json:91-172, A100, ms per call).
PUBLICATION_OPTIMAL = (
    ("Tiny Batch", 1, 768, 0.021110784530639647, 0.01005568027496338),
    ("Small Batch", 8, 768, 0.021123071670532227, 0.010141695976257324),
    ("BERT", 32, 768, 0.021166080474853514, 0.010106880187988282),
    ("GPT-2 Small", 32, 1024, 0.021170175552368165, 0.01003110408782959),
    ("GPT-2 Medium", 32, 2048, 0.02207744026184082, 0.01009663963317871),
    ("GPT-3", 32, 4096, 0.02109235191345215, 0.009992192268371582),
    ("Large Batch", 64, 4096, 0.02105548858642578, 0.010108927726745605),
    ("XL Batch", 128, 4096, 0.021360639572143555, 0.010102784156799317),
    ("Odd Dims", 17, 1023, 0.024211456298828125, 0.010010623931884765),
    ("GPT-3 Large", 32, 12288, 0.024375295639038085, 0.01245798397064209),
)
# The reference's large-row forward table (benchmarks/results/final_benchmark_results.csv:2-7;
# rows = batch x seq_len, fp32, ms per call on its A100; no script in the reference produces it).
LARGE_ROWS = (
    ("GPT-3 Medium", 2048, 4096, 0.07, 0.049), ("GPT-3 Large", 2048, 4096, 0.07, 0.049),
    ("Custom-4K", 2048, 4096, 0.07, 0.049), ("GPT-3 XL", 2048, 5120, 0.087, 0.058),
    ("Custom-6K", 2048, 6144, 0.102, 0.069), ("Large Model", 1024, 8192, 0.069, 0.049),
)
A100_HBM_GBS = 1555.0  # A100 40 GB
# The reference's performance regression test: FusedLayerNorm >= 1.2x nn.LayerNorm
# (tests/test_layernorm.py:361-413).
GATE_SHAPES = ((32, 768), (32, 1024), (16, 2048), (8, 4096))


def reference_paths(torch):
    """Latency of the reference's own call paths on this GPU, with the reference's own methods:
      * publication_optimal: fused_layernorm_cuda.layernorm(x, ln.weight, ln.bias, 1e-5) and
        nn.LayerNorm(x), 500 back-to-back calls each on one tensor between HIP events after 100
        warm-ups (tests/publication_validation.py:181-205), at the published shapes, beside the
        published A100 figures;
      * module_gate: FusedLayerNorm(h) and nn.LayerNorm(h) (weights requiring grad), 100
        back-to-back forwards timed by wall clock after 50 warm-ups
        (tests/test_layernorm.py:376-413; >= 1.2x required there), median of 7 repetitions;
      * c1_binding: the binding call at 32 x 768 fp32 back to back (host-bound: per-call host
        cost) and 32 calls captured in one HIP graph (GPU-side latency per call).
    fp32 throughout, torch.randn inputs, nn.LayerNorm's default affine parameters."""
    import torch.nn as nn
    import fused_layernorm as fl
    import fused_layernorm_cuda as ext
    out = {"publication_optimal": [], "module_gate": []}
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    for name, b, h, pt_a100, ours_a100 in PUBLICATION_OPTIMAL:
        x = torch.randn(b, h, device="cuda")
        ln = nn.LayerNorm(h).cuda()
        for _ in range(100):
            ln(x)
            ext.layernorm(x, ln.weight, ln.bias, 1e-5)
        torch.cuda.synchronize()
        res = {}
        for key, fn in (("pytorch_us", lambda: ln(x)),
                        ("ours_us", lambda: ext.layernorm(x, ln.weight, ln.bias, 1e-5))):
            e0, e1 = ev(), ev()
            e0.record()
            for _ in range(500):
                fn()
            e1.record()
            torch.cuda.synchronize()
            res[key] = round(e0.elapsed_time(e1) / 500 * 1e3, 2)
        out["publication_optimal"].append({
            "config": name, "batch": b, "hidden": h, **res,
            "speedup": round(res["pytorch_us"] / res["ours_us"], 3),
            "reference_a100_ours_us": round(ours_a100 * 1e3, 2),
            "reference_a100_pytorch_us": round(pt_a100 * 1e3, 2)})
    for b, h in GATE_SHAPES:
        x = torch.randn(b, h, device="cuda")
        pt = nn.LayerNorm(h).cuda()
        fu = fl.FusedLayerNorm(h).cuda()
        for _ in range(50):
            pt(x)
            fu(x)
        torch.cuda.synchronize()
        tp, tf = [], []
        for _ in range(7):
            for lst, mod in ((tp, pt), (tf, fu)):
                t0 = time.time()
                for _ in range(100):
                    mod(x)
                torch.cuda.synchronize()
                lst.append((time.time() - t0) / 100 * 1e6)
        sp = [a / c for a, c in zip(tp, tf)]
        out["module_gate"].append({"batch": b, "hidden": h,
                                   "nn_layernorm_us": round(statistics.median(tp), 2),
                                   "fused_layernorm_us": round(statistics.median(tf), 2),
                                   "speedup": round(statistics.median(sp), 3),
                                   "speedup_min": round(min(sp), 3), "required": 1.2})
    x = torch.randn(32, 768, device="cuda")
    ln = nn.LayerNorm(768).cuda()
    w, bb = ln.weight.detach(), ln.bias.detach()
    for _ in range(200):
        ext.layernorm(x, w, bb, 1e-5)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(2000):
        ext.layernorm(x, w, bb, 1e-5)
    torch.cuda.synchronize()
    eager = (time.perf_counter() - t0) / 2000 * 1e6
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            ext.layernorm(x, w, bb, 1e-5)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for _ in range(32):
            ext.layernorm(x, w, bb, 1e-5)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = ev(), ev()
    e0.record()
    for _ in range(20):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    out["c1_binding"] = {"call": "fused_layernorm_cuda.layernorm(x, w, b, 1e-5), 32 x 768 fp32",
                         "eager_us_per_call": round(eager, 2),
                         "graph_us_per_call": round(e0.elapsed_time(e1) / (20 * 32) * 1e3, 2),
                         "target_us": 5.0}
    out["large_rows_fp32"] = large_rows(torch)
    return out


def large_rows(torch, n=200):
    """The reference's large-row forward table (LARGE_ROWS) on this GPU: the binding call
    fused_layernorm_cuda.layernorm and nn.LayerNorm, fp32, each timed over n calls between HIP
    events on rotating inputs of at least 1 GiB (no call reads what an earlier one left in the
    256 MB last-level cache), beside the published A100 figures, the fraction of each GPU's HBM
    peak that the algorithmic bytes (x read, y written) give, and the hand-written 1R1W stream's
    rate at the same tensor size (a 32 MiB stream takes ~12 us, of which ramp and drain are a
    large share)."""
    import torch.nn as nn
    import fused_layernorm_cuda as ext
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    rows_out = []
    ceilings = {}
    for name, rows, cols, pt_ms, ref_ms in LARGE_ROWS:
        nbytes = rows * cols * 4
        k = max(4, -(-(1 << 30) // nbytes))
        xs = [torch.randn(rows, cols, device="cuda") for _ in range(k)]
        ln = nn.LayerNorm(cols).cuda()
        w, b = ln.weight.detach(), ln.bias.detach()
        res = {}
        with torch.no_grad():
            for key, fn in (("pytorch_us", lambda x: ln(x)),
                            ("ours_us", lambda x: ext.layernorm(x, w, b, 1e-5))):
                for i in range(2 * k):
                    fn(xs[i % k])
                torch.cuda.synchronize()
                e0, e1 = ev(), ev()
                e0.record()
                for i in range(n):
                    fn(xs[i % k])
                e1.record()
                torch.cuda.synchronize()
                res[key] = round(e0.elapsed_time(e1) / n * 1e3, 2)
        moved = 2 * nbytes
        if nbytes not in ceilings:  # 1R1W stream of the same tensor size
            ceilings[nbytes] = stream_ceilings(torch, nbytes, patterns=[0])["1r1w_gbs"]
        rows_out.append({
            "config": name, "rows": rows, "hidden": cols, **res,
            "speedup": round(res["pytorch_us"] / res["ours_us"], 3),
            "ours_gbs": round(moved / res["ours_us"] / 1e3, 1),
            "ours_pct_of_hbm_peak": round(100 * moved / res["ours_us"] / 1e3 / HBM_PEAK_GBS, 1),
            "stream_1r1w_gbs": round(ceilings[nbytes], 1),
            "ours_over_stream": round(moved / res["ours_us"] / 1e3 / ceilings[nbytes], 3),
            "reference_a100_pytorch_us": round(pt_ms * 1e3, 1),
            "reference_a100_ours_us": round(ref_ms * 1e3, 1),
            "reference_a100_pct_of_hbm_peak": round(
                100 * moved / (ref_ms * 1e3) / 1e3 / A100_HBM_GBS, 1)})
        del xs
        torch.cuda.empty_cache()
    return rows_out


def torch_gpu_compare(torch, ours, warmup=10, n=50):
    """PyTorch's own GPU ops on the same seeded inputs and shapes, timed like ours (HIP events,
    rotating buffer sets), and our speedup over them: the reference's published headline is a
    speedup over nn.LayerNorm on the same GPU.  `ours` maps case -> our ms per call."""
    from fused_layernorm.testing import WORKLOADS, make_inputs
    F = torch.nn.functional
    aten = torch.ops.aten
    stream = torch.cuda.current_stream()

    def device_sets(w, need=("x",)):
        inp = make_inputs(w)
        base = {k: v.to("cuda") for k, v in inp.items()}
        set_bytes = sum(base[k].numel() * base[k].element_size() for k in need if k in base)
        nsets = min(8, max(2, -(-ROTATE_BYTES // (2 * set_bytes))))
        return [base] + [{k: v.clone() for k, v in base.items()} for _ in range(nsets - 1)]

    def time_ms(fn, sets):
        for i in range(warmup):
            fn(sets[i % len(sets)])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n):
            fn(sets[i % len(sets)])
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    res = {}

    def entry(name, torch_ms, parts=None):
        e = {"torch_us": round(torch_ms * 1e3, 2)}
        if parts:
            e.update({k: round(v * 1e3, 2) for k, v in parts.items()})
        if ours.get(name):
            e["ours_us"] = round(ours[name] * 1e3, 2)
            e["speedup"] = round(torch_ms / ours[name], 2)
        res[name] = e

    # LayerNorm fwd + bwd (aten's own LayerNorm kernels, as nn.LayerNorm runs them).
    w = WORKLOADS[HEADLINE]
    sets = device_sets(w, ("x", "dy"))
    shape = (w.cols,)
    for st in sets:
        st["out"] = aten.native_layer_norm(st["x"], shape, st["gamma"], st["beta"], w.eps)
    f_ms = time_ms(lambda st: aten.native_layer_norm(st["x"], shape, st["gamma"], st["beta"],
                                                      w.eps), sets)
    b_ms = time_ms(lambda st: aten.native_layer_norm_backward(
        st["dy"], st["x"], shape, st["out"][1], st["out"][2], st["gamma"], st["beta"],
        [True, True, True]), sets)
    entry("ln_fwd_bwd_bf16_8192x4096", f_ms + b_ms, {"torch_fwd_us": f_ms, "torch_bwd_us": b_ms})
    del sets
    # RMSNorm fwd + bwd through autograd (backward = fwd+bwd minus fwd).
    for name in ("rms_fwd_bwd_bf16_8192x4096", "c4_rms_fwd_bwd_bf16_16384x8192"):
        w = WORKLOADS[name]
        sets = device_sets(w, ("x", "dy"))
        for st in sets:
            st["x"].requires_grad_(True)
            st["gamma"].requires_grad_(True)

        def fb(st, w=w):
            y = F.rms_norm(st["x"], (w.cols,), st["gamma"], w.eps)
            torch.autograd.grad(y, (st["x"], st["gamma"]), st["dy"])
        f_ms = time_ms(lambda st, w=w: F.rms_norm(st["x"].detach(), (w.cols,),
                                                  st["gamma"].detach(), w.eps), sets)
        fb_ms = time_ms(fb, sets)
        entry(name, fb_ms, {"torch_fwd_us": f_ms, "torch_bwd_us": fb_ms - f_ms})
        del sets
    # LayerNorm + GELU fwd + bwd through autograd (tanh and exact forms).
    for name in ("ln_gelu_fwd_bwd_bf16_8192x4096", "ln_gelu_erf_fwd_bwd_bf16_8192x4096"):
        w = WORKLOADS[name]
        sets = device_sets(w, ("x", "dy"))
        for st in sets:
            for k in ("x", "gamma", "beta"):
                st[k].requires_grad_(True)

        def fwd(st, w=w, grad=True):
            a = [st[k] if grad else st[k].detach() for k in ("x", "gamma", "beta")]
            return F.gelu(F.layer_norm(a[0], (w.cols,), a[1], a[2], w.eps),
                          approximate=w.approximate)

        def fb(st, w=w):
            torch.autograd.grad(fwd(st), (st["x"], st["gamma"], st["beta"]), st["dy"])
        f_ms = time_ms(lambda st: fwd(st, grad=False), sets)
        fb_ms = time_ms(fb, sets)
        entry(name, fb_ms, {"torch_fwd_us": f_ms, "torch_bwd_us": fb_ms - f_ms})
        del sets
    # C1 (back to back, latency-bound).
    w = WORKLOADS["c1_ln_fwd_fp32_32x768"]
    sets = device_sets(w)
    entry(w.name, time_ms(lambda st: F.layer_norm(st["x"], (w.cols,), st["gamma"], st["beta"],
                                                  w.eps), sets))
    # C3: residual add, then LayerNorm of the stored sum.
    w = WORKLOADS["c3_add_ln_fwd_bf16_8192x4096"]
    sets = device_sets(w, ("x", "residual"))

    def c3(st, w=w):
        h = st["x"] + st["residual"]
        return F.layer_norm(h, (w.cols,), st["gamma"], st["beta"], w.eps)
    entry(w.name, time_ms(c3, sets))
    del sets
    # C5: LayerNorm, per-row amax, scale, saturating e4m3fn cast.
    w = WORKLOADS["c5_ln_fp8_bf16_32768x7168"]
    sets = device_sets(w)

    def c5(st, w=w):
        y = F.layer_norm(st["x"], (w.cols,), st["gamma"], st["beta"], w.eps).float()
        scale = y.abs().amax(dim=-1, keepdim=True) / 448.0
        q = (y / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        return q, scale
    entry(w.name, time_ms(c5, sets))
    del sets
    torch.cuda.empty_cache()
    return res


def torch_cpu_configs(seconds=1.5):
    """The reference's CPU path on each config: torch-CPU ops on the same seeded inputs (the
    config's dtype) at full size, the process's host-thread budget; median of >= 3 runs."""
    import torch
    from fused_layernorm.testing import WORKLOADS, algorithmic_bytes, make_inputs
    F = torch.nn.functional
    torch.set_num_threads(cpu_threads())
    res = {}
    cases = (("c1_ln_fwd_fp32_32x768", None), ("c2_ln_gelu_fp32_17x1023", None),
             ("c2_ln_gelu_fp32_64x4096", None), ("c3_add_ln_fwd_bf16_8192x4096", None),
             ("c4_rms_fwd_bwd_bf16_16384x8192", None), ("c5_ln_fp8_bf16_32768x7168", None))
    for name, sample in cases:
        w = WORKLOADS[name]
        rows = w.rows if sample is None else sample
        inp = make_inputs(w, rows)
        x, g, b = inp["x"], inp.get("gamma"), inp.get("beta")
        shape = (w.cols,)
        if w.op == "layer_norm":
            def run():
                F.layer_norm(x, shape, g, b, w.eps)
            what = "F.layer_norm"
        elif w.op == "layer_norm_gelu":
            def run():
                F.gelu(F.layer_norm(x, shape, g, b, w.eps), approximate=w.approximate)
            what = f"F.gelu(F.layer_norm), approximate={w.approximate!r}"
        elif w.op == "add_layer_norm":
            r = inp["residual"]

            def run():
                F.layer_norm(x + r, shape, g, b, w.eps)
            what = "x + r, F.layer_norm"
        elif w.op == "rms_norm_fwd_bwd":
            xg = x.clone().requires_grad_(True)
            gg = g.clone().requires_grad_(True)
            dy = inp["dy"]

            def run():
                torch.autograd.grad(F.rms_norm(xg, shape, gg, w.eps), (xg, gg), dy)
            what = "F.rms_norm + autograd backward"
        else:  # layer_norm_fp8
            def run():
                y = F.layer_norm(x, shape, g, b, w.eps).float()
                scale = y.abs().amax(dim=-1, keepdim=True) / 448.0
                (y / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
            what = "F.layer_norm, row amax, scale, clamp, float8_e4m3fn cast"
        med, n = _median_time(run, seconds, warmup=1 if rows * w.cols > 2 ** 24 else 3)
        res[name] = {"us_per_call": round(med * 1e6, 1),
                     "gbs": round(algorithmic_bytes(w, rows)["total"] / med / 1e9, 2),
                     "sample": f"full {rows} x {w.cols}, {what}, median of {n}"}
    res["threads"] = torch.get_num_threads()
    return res


# ------------------------------------------------------------------------------------------------
def time_graph(runner, n_calls=32, replays=20):
    """GPU-side time (ms) of one forward call: n_calls C-ABI calls captured in one HIP graph
    (hipStreamBeginCapture under torch.cuda.graph; the forward records no memset nodes), the
    graph replayed `replays` times between HIP events.  Without the per-call host cost of an
    eager launch, this is the latency a graph-captured caller sees."""
    import torch
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):  # warm the per-device caches outside the capture
            runner.fwd(runner.sets[i % runner.nsets], runner.capi.stream())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for i in range(n_calls):
            runner.fwd(runner.sets[i % runner.nsets], runner.capi.stream())
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (replays * n_calls)


def measure(lib, capi, torch, w, steps, warmup, stream, stream_obj, graph=False):
    from fused_layernorm.testing import algorithmic_bytes, make_inputs

    r = Runner(lib, capi, torch, w, make_inputs(w))
    r.prime(stream)
    for _ in range(warmup):
        r.step(stream)
    warm_clocks(lambda: r.step(stream))
    ms = r.time_region(lambda: r.step(stream), steps, stream_obj)
    res = dict(ms=ms, bytes=algorithmic_bytes(w), nsets=r.nsets)
    n_group = max(20, steps // 2)
    res["ms_fwd"] = time_launch_group(r, "fwd", n_group, stream, stream_obj)
    if r.has_bwd:
        res["ms_bwd"] = time_launch_group(r, "bwd", n_group, stream, stream_obj)
    if graph:
        res["ms_fwd_graph"] = time_graph(r)
    del r
    torch.cuda.empty_cache()
    return res


def gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9


def traffic_configs(args):
    """--traffic-configs: per bandwidth-bound config (C1 and C2 are latency-bound), the HBM bytes
    of each forward / backward call from the counter passes, the call times, and both the
    algorithmic and the HBM-traffic bandwidth.  One JSON object on stdout."""
    names = [n for n in CONFIGS if not n.startswith(("c1_", "c2_"))]
    traffic = {}
    for n in names:  # counter passes first, in child processes, before this one touches the GPU
        t, note = pmc_traffic(n)
        traffic[n] = t if t else {"note": note}
    import torch
    import capi
    from fused_layernorm.testing import WORKLOADS

    lib = capi.load()
    stream_obj = torch.cuda.current_stream()
    stream = capi.stream()
    out = {}
    for n in names:
        res = measure(lib, capi, torch, WORKLOADS[n], 100, args.warmup, stream, stream_obj)
        entry = {}
        for d in ("fwd", "bwd"):
            ms = res.get(f"ms_{d}")
            if ms is None:
                continue
            ab = res["bytes"][d]
            tb = traffic[n].get(d)
            entry[d] = {"us": round(ms * 1e3, 2), "algorithmic_bytes": ab,
                        "algorithmic_gbs": round(gbs(ab, ms), 1), "traffic_bytes": tb,
                        "hbm_gbs": round(gbs(tb, ms), 1) if tb else None,
                        "traffic_over_algorithmic": round(tb / ab, 4) if tb else None}
        if "note" in traffic[n]:
            entry["traffic_note"] = traffic[n]["note"]
        out[n] = entry
    cal = next((t["calibration"] for t in traffic.values() if "calibration" in t), None)
    print(json.dumps({"traffic_configs": out, "calibration": cal,
                      "passes": "rocprofv3 --pmc FETCH_SIZE | WRITE_SIZE -- bench.py "
                                "--kernel-loop <config> --iters 20"}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "row-sharded multi-GPU layout is not built or measured here.",
              file=sys.stderr)
        sys.exit(2)
    if args.kernel_loop:
        kernel_loop(args)
        return
    if args.stream_loop:
        stream_loop(args)
        return
    if args.traffic_configs:
        traffic_configs(args)
        return
    if args.large_rows_only:
        import torch
        assert torch.cuda.is_available(), "bench.py needs a GPU"
        print(json.dumps({"large_rows_fp32": large_rows(torch)}), flush=True)
        return

    # Counter passes first, in child processes, before this process touches the GPU.
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        traffic, traffic_note = pmc_traffic(HEADLINE)

    import torch
    import capi
    from fused_layernorm.testing import WORKLOADS

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lib = capi.load()
    stream_obj = torch.cuda.current_stream()
    stream = capi.stream()

    head = measure(lib, capi, torch, WORKLOADS[HEADLINE], args.steps, args.warmup, stream,
                   stream_obj)
    rms = None
    if not args.headline_only:
        rms = measure(lib, capi, torch, WORKLOADS["rms_fwd_bwd_bf16_8192x4096"], args.steps,
                      args.warmup, stream, stream_obj)
    value = gbs(head["bytes"]["total"], head["ms"])
    bwd_gbs = gbs(head["bytes"]["bwd"], head["ms_bwd"])
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded torch.randn inputs (x seed 3, gamma 103, beta 203, dy 303)",
        "config": {"workload": HEADLINE, "rows": 8192, "cols": 4096,
                   "step": "LayerNorm fwd (y, mean, rstd) + bwd (dx, dgamma, dbeta fp32); the "
                           "bwd runs on the buffer set half the rotation away from the fwd's",
                   "algorithmic_bytes_per_step": head["bytes"]["total"],
                   "rotating_buffer_sets": head["nsets"]},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "us_per_call": {"fwd": round(head["ms_fwd"] * 1e3, 2),
                        "bwd": round(head["ms_bwd"] * 1e3, 2),
                        "fwd_bwd": round(head["ms"] * 1e3, 2)},
        "roofline": {
            "kernel": "fln_layernorm_backward (bwd_reg_kernel + col_reduce_kernel, one call)",
            "bound": "hbm", "achieved": round(bwd_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic["bwd"] if traffic and traffic.get("bwd") else None,
            "algorithmic_bytes_per_launch": head["bytes"]["bwd"],
            "avg_launch_us": round(head["ms_bwd"] * 1e3, 2),
        },
        "forward_kernel": {
            "kernel": "fwd_reg_kernel", "algorithmic_bytes_per_launch": head["bytes"]["fwd"],
            "avg_launch_us": round(head["ms_fwd"] * 1e3, 2),
            "achieved_gbs": round(gbs(head["bytes"]["fwd"], head["ms_fwd"]), 1),
            "traffic": traffic["fwd"] if traffic and traffic.get("fwd") else None,
        },
    }
    ceil = stream_ceilings(torch, 8192 * 4096 * 2, head["bytes"]["fwd"], head["bytes"]["bwd"])
    ceil["value_over_step_ceiling"] = round(value / ceil["step_ceiling_gbs"], 3)
    ceil["bwd_over_2r1w"] = round(bwd_gbs / ceil["2r1w_gbs"], 3)
    ceil["fwd_over_1r1w"] = round(gbs(head["bytes"]["fwd"], head["ms_fwd"]) / ceil["1r1w_gbs"], 3)
    out["stream_ceilings"] = ceil
    if rms:
        out["rms_fwd_bwd"] = {
            "workload": "rms_fwd_bwd_bf16_8192x4096",
            "value": round(gbs(rms["bytes"]["total"], rms["ms"]), 1), "unit": "GB/s",
            "us_per_call": {"fwd": round(rms["ms_fwd"] * 1e3, 2),
                            "bwd": round(rms["ms_bwd"] * 1e3, 2),
                            "fwd_bwd": round(rms["ms"] * 1e3, 2)},
        }
    if traffic:
        out["roofline"]["traffic_detail"] = {"fetch": traffic["bwd_detail"]["fetch"],
                                             "write": traffic["bwd_detail"]["write"],
                                             "calibration": traffic["calibration"],
                                             "passes": traffic["passes"]}
    else:
        out["roofline"]["traffic_note"] = traffic_note

    if not args.no_configs and not args.headline_only:
        cfg = {}
        ceiling_cache = {(p, 8192 * 4096 * 2): ceil[STREAM_NAMES[p] + "_gbs"]
                         for p in STREAM_NAMES if STREAM_NAMES[p] + "_gbs" in ceil}
        for name in CONFIGS:
            w = WORKLOADS[name]
            small = w.op in ("layer_norm", "layer_norm_gelu")
            res = measure(lib, capi, torch, w, max(50, args.steps // 2), args.warmup, stream,
                          stream_obj, graph=small)
            entry = {"us_per_call": round(res["ms_fwd"] * 1e3, 2)}
            if small:
                entry["us_per_call_graph"] = round(res["ms_fwd_graph"] * 1e3, 2)
            if "ms_bwd" in res:
                entry["us_per_call"] = {"fwd": round(res["ms_fwd"] * 1e3, 2),
                                        "bwd": round(res["ms_bwd"] * 1e3, 2),
                                        "fwd_bwd": round(res["ms"] * 1e3, 2)}
                entry["gbs"] = round(gbs(res["bytes"]["total"], res["ms"]), 1)
            else:
                entry["gbs"] = round(gbs(res["bytes"]["fwd"], res["ms_fwd"]), 1)
            if name in CONFIG_PATTERNS:
                ceil_gbs, pattern, nbytes = config_ceiling(
                    torch, name, res["bytes"]["fwd"], res["bytes"].get("bwd"), ceiling_cache)
                entry["pct_of_hbm_peak"] = round(100 * entry["gbs"] / HBM_PEAK_GBS, 1)
                entry["stream_ceiling"] = {"pattern": pattern, "bytes_per_stream": nbytes,
                                           "gbs": round(ceil_gbs, 1),
                                           "frac": round(entry["gbs"] / ceil_gbs, 3)}
            cfg[name] = entry
        out["configs"] = cfg
        out["reference_paths"] = reference_paths(torch)

    if not args.no_configs and not args.headline_only:
        ours = {HEADLINE: head["ms"], "c1_ln_fwd_fp32_32x768": None,
                "rms_fwd_bwd_bf16_8192x4096": rms["ms"] if rms else None}
        for name in ("c1_ln_fwd_fp32_32x768", "c3_add_ln_fwd_bf16_8192x4096",
                     "c4_rms_fwd_bwd_bf16_16384x8192", "c5_ln_fp8_bf16_32768x7168",
                     "ln_gelu_fwd_bwd_bf16_8192x4096", "ln_gelu_erf_fwd_bwd_bf16_8192x4096"):
            e = out["configs"][name]["us_per_call"]
            ours[name] = (e["fwd_bwd"] if isinstance(e, dict) else e) / 1e3
        out["torch_gpu"] = torch_gpu_compare(torch, ours)

    if not args.no_cpu_baseline:
        w = WORKLOADS[HEADLINE]
        out["cpu_baseline"] = torch_cpu_baseline(w, max(2.0, args.cpu_seconds / 2))
        out["cpu_baseline"]["c_oracle_port"] = cpu_port_baseline(w, args.cpu_seconds / 2)
        if not args.no_configs and not args.headline_only:
            tc = torch_cpu_configs()
            for name, e in tc.items():
                if name in out.get("configs", {}):
                    mine = out["configs"][name]["us_per_call"]
                    mine = mine["fwd_bwd"] if isinstance(mine, dict) else mine
                    e["gpu_speedup"] = round(e["us_per_call"] / mine, 1)
            out["cpu_baseline"]["torch_cpu_configs"] = tc
    out["host"] = platform.node()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
