"""Host-side tests (CPU only): the C-ABI library loads and exports every declared symbol, the
binding validates arguments before anything is launched, the operator schemas trace with fake
tensors, and the host utilities keep the reference's formulas."""
import ctypes

import pytest
import torch

import capi
import fused_layernorm as fl
import fused_layernorm_cuda as ext
from fused_layernorm.testing import WORKLOADS, algorithmic_bytes


def test_c_abi_library_exports_every_declared_symbol():
    lib = capi.load()
    declared = capi.declared_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/fused_layernorm.h but not exported"
    assert set(declared) <= set(capi.SIGNATURES), "tests/capi.py lacks a signature"


def test_stream_library_exports_every_declared_symbol():
    # libfln_stream.so (the streaming reference kernels bench.py measures the HBM ceiling with).
    import os
    import re
    header = open(os.path.join(capi.ROOT, "include", "fln_stream.h")).read()
    declared = sorted(set(re.findall(r"\b(fln_stream_[a-z0-9_]+)\s*\(", header)))
    assert declared == ["fln_stream_blocks_per_cu", "fln_stream_cu_count", "fln_stream_run"]
    lib = ctypes.CDLL(os.path.join(capi.PKG, "libfln_stream.so"))
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/fln_stream.h but not exported"
    lib.fln_stream_run.argtypes = [ctypes.c_int, *[ctypes.c_void_p] * 4, ctypes.c_int64,
                                   *[ctypes.c_int] * 6, ctypes.c_void_p]
    # Invalid arguments are refused before anything is launched (no device needed).
    assert lib.fln_stream_run(0, None, None, None, None, 1 << 20, 256, 1, 1, 1, 0, 0, None) == 1
    assert lib.fln_stream_run(9, 16, 16, 16, 16, 1 << 20, 256, 1, 1, 1, 0, 0, None) == 1
    assert lib.fln_stream_run(0, 16, None, 16, None, 1 << 31, 256, 1, 1, 1, 0, 0, None) == 1


def test_package_without_the_extension_fails_loudly(tmp_path):
    """No fallback path: a copy of the Python package with no built extension beside it must
    refuse to import, naming the missing HIP extension."""
    import os
    import shutil
    import subprocess
    import sys
    src = os.path.dirname(fl.__file__)
    shutil.copytree(src, tmp_path / "fused_layernorm",
                    ignore=shutil.ignore_patterns("__pycache__", "*.so"))
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    code = f"import sys; sys.path.insert(0, {str(tmp_path)!r}); import fused_layernorm"
    r = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "Cannot import fused_layernorm_cuda" in r.stderr, r.stderr[-2000:]


def test_erfc_terms_constants_in_the_device_header():
    """The exact-GELU kernels evaluate Phi(v) through 0.5 erfc(|v| / sqrt 2) = t F(t) exp(-v^2 / 2),
    t = 1 / (1 + p |v| / sqrt 2), F a fitted polynomial.  Parse p and F's coefficients from
    csrc/fln_device.h, evaluate GELU and its derivative under an fp32 emulation of the device
    code, and check them against scipy's erfc in float64 over |v| <= 13 (plus the infinities): a
    mistyped coefficient or a wrong p fails here, on the CPU, and so does a sign slip in either
    formula (the planted cases below)."""
    import os
    import re
    import sys
    import numpy as np
    from scipy.special import erfc
    csrc = os.path.join(os.path.dirname(os.path.dirname(fl.__file__)), "csrc")
    src = open(os.path.join(csrc, "fln_device.h")).read()
    poly = src[src.index("float erfc_poly(float t)"):]
    coef = [np.float32(float(c)) for c in
            re.findall(r"[-+]?\d\.\d+e[-+]\d+", poly[poly.index("kF["):poly.index("};")])]
    body = src[src.index("ErfcTerms erfc_terms(float v)"):]
    body = body[:body.index("return {")]
    p = float(re.search(r"fmaf\(([\d.]+)f \* 0\.7071", body).group(1))
    assert len(coef) >= 6 and 0.2 < p < 0.6
    sys.path.insert(0, csrc)
    try:
        import fit_erfc
    finally:
        sys.path.remove(csrc)
    v = np.linspace(-13, 13, 260001).astype(np.float32)
    vd = v.astype(np.float64)
    phi = np.where(vd < 0, 0.5 * erfc(-vd / np.sqrt(2)), 1 - 0.5 * erfc(vd / np.sqrt(2)))
    g_ref = vd * phi
    d_ref = phi + vd * np.exp(-vd * vd / 2) / np.sqrt(2 * np.pi)
    tail = (vd < -3) & (np.abs(g_ref) > 1e-30)

    def errors(gelu, grad):
        return (np.abs(gelu - g_ref).max(), np.abs(grad - d_ref).max(),
                (np.abs(gelu[tail] - g_ref[tail]) / np.abs(g_ref[tail])).max())

    gelu = fit_erfc.gelu(coef, v, p=p)
    grad = fit_erfc.gelu_grad(coef, v, p=p)
    g_abs, d_abs, g_tail = errors(gelu, grad)
    assert g_abs <= 1e-6 and d_abs <= 2e-6 and g_tail <= 1e-4, (g_abs, d_abs, g_tail)
    special = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0], np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        gs = fit_erfc.gelu(coef, special, p=p)
        ds = fit_erfc.gelu_grad(coef, special, p=p)
    assert gs[0] == np.inf and gs[1] == 0.0 and np.isnan(gs[2]) and gs[3] == 0.0 and gs[4] == 0.0
    assert np.isnan(ds[2]) and abs(ds[3] - 0.5) < 1e-6 and abs(ds[4] - 0.5) < 1e-6
    # The register backward's GELU' tables (fln_gelu_table.h): exactly the fp32 rounding of the
    # float64 quadratics fit_erfc.gelu_table() builds, and their lookup within 1e-6 of GELU'
    # (erf form: d_ref; tanh form: its derivative in float64).
    hdr = open(os.path.join(csrc, "fln_gelu_table.h")).read()
    n_tab = int(re.search(r"kGeluTabN = (\d+);", hdr).group(1))
    v_max = float(re.search(r"kGeluTabMax = ([\d.]+)f;", hdr).group(1))
    assert (n_tab, v_max) == (fit_erfc.TAB_N, fit_erfc.TAB_MAX)
    k0, k1 = np.sqrt(2 / np.pi), 0.044715
    u_t = k0 * (vd + k1 * vd ** 3)
    d_tanh = 0.5 * (1 + np.tanh(u_t)) + 0.5 * vd * k0 * (1 + 3 * k1 * vd * vd) / np.cosh(u_t) ** 2
    tables = {}
    for kind, name, ref in (("erf", "kGeluTabData", d_ref), ("tanh", "kGeluTanhTabData", d_tanh)):
        body_t = hdr[hdr.index(name + "["):]
        body_t = body_t[body_t.index("{"):body_t.index("};")]
        data = np.array([np.float32(float(c)) for c in re.findall(
            r"([-+]?\d+\.\d+(?:e[-+]\d+)?)f", body_t)], np.float32)
        tab = tables[kind] = fit_erfc.gelu_table(kind)
        assert data.shape == (4 * n_tab,) and np.array_equal(data.reshape(n_tab, 4)[:, :3], tab)
        assert not data.reshape(n_tab, 4)[:, 3].any()
        assert np.abs(fit_erfc.gelu_grad_table(tab, v) - ref).max() <= 1e-6, kind
        with np.errstate(invalid="ignore", over="ignore"):
            ts = fit_erfc.gelu_grad_table(tab, special)
        assert np.isnan(ts[2]) and abs(ts[3] - 0.5) < 1e-6 and abs(ts[4] - 0.5) < 1e-6
    tab = tables["erf"]
    # The forward register kernel's GELU table: L = log2(Phi(-|v|)) - log2(16) on intervals of
    # 1 / 16, the last one -inf; its lookup keeps the bounds above, tail included.
    n_log = int(re.search(r"kGeluLogTabN = (\d+);", hdr).group(1))
    inv_h = float(re.search(r"kGeluLogTabInvH = ([\d.]+)f;", hdr).group(1))
    assert (n_log, inv_h) == (fit_erfc.LOG_TAB_N, fit_erfc.LOG_TAB_INV_H)
    body_l = hdr[hdr.index("kGeluLogTabData["):]
    body_l = body_l[body_l.index("{"):body_l.index("};")]
    lits = re.findall(r"(-__builtin_huge_valf\(\)|[-+]?\d+\.\d+(?:e[-+]\d+)?f)", body_l)
    data = np.array([-np.inf if x.startswith("-__") else float(x[:-1]) for x in lits], np.float32)
    log_tab = fit_erfc.gelu_log_table()
    assert data.shape == (4 * n_log,) and np.array_equal(data.reshape(n_log, 4)[:, :3], log_tab)
    gelu_l = fit_erfc.gelu_log_tab(log_tab, v)
    gl_abs = np.abs(gelu_l - g_ref).max()
    gl_tail = (np.abs(gelu_l[tail] - g_ref[tail]) / np.abs(g_ref[tail])).max()
    assert gl_abs <= 1e-6 and gl_tail <= 1e-4, (gl_abs, gl_tail)
    with np.errstate(invalid="ignore", over="ignore"):
        gls = fit_erfc.gelu_log_tab(log_tab, special)
    assert gls[0] == np.inf and gls[1] == 0.0 and np.isnan(gls[2]) and gls[3] == 0 and gls[4] == 0
    # Planted mistakes (in the emulation, on the CPU): each must fail the bounds above.
    bad_coef = list(coef)
    bad_coef[3] = np.float32(bad_coef[3] * (1 + 1e-4))
    planted = [
        errors(fit_erfc.gelu(bad_coef, v, p=p), fit_erfc.gelu_grad(bad_coef, v, p=p)),
        errors(fit_erfc.gelu(coef, v, p=p * 1.001), fit_erfc.gelu_grad(coef, v, p=p * 1.001)),
        errors(gelu, (np.float32(0.5) - (grad - np.float32(0.5))).astype(np.float32)),
        errors(np.maximum(v, 0) - (gelu - np.maximum(v, 0)), grad),
    ]
    for k, (ga, da, gt) in enumerate(planted):
        assert ga > 1e-6 or da > 2e-6 or gt > 1e-4, f"planted mistake {k} passed"
    # ... and the table: a swapped pair of coefficients, an interval off by one, a wrong h, the
    # other form's table.
    swapped = tab.copy()
    swapped[:, [1, 2]] = swapped[:, [2, 1]]
    shifted = np.roll(tab, 1, axis=0)
    bad_log = log_tab.copy()
    bad_log[:, [1, 2]] = bad_log[:, [2, 1]]
    for bad_gelu in (fit_erfc.gelu_log_tab(bad_log, v), fit_erfc.gelu_log_tab(log_tab, v, 15),
                     fit_erfc.gelu_log_tab(np.roll(log_tab, 1, axis=0), v)):
        bad_tail = (np.abs(bad_gelu[tail] - g_ref[tail]) / np.abs(g_ref[tail])).max()
        assert np.abs(bad_gelu - g_ref).max() > 1e-6 or bad_tail > 1e-4
    for bad_grad in (fit_erfc.gelu_grad_table(swapped, v), fit_erfc.gelu_grad_table(shifted, v),
                     fit_erfc.gelu_grad_table(tab, v, vmax=v_max * 1.01),
                     fit_erfc.gelu_grad_table(tables["tanh"], v)):
        assert np.abs(bad_grad - d_ref).max() > 1e-6


def _gfx950_disassembly(lib_path, tmp_path):
    """Disassemble every gfx950 code object bundled in a library built here (its .hip_fatbin
    section holds one clang offload bundle per translation unit)."""
    import os
    import subprocess
    tools = "/opt/rocm/llvm/bin"
    need = [os.path.join(tools, t) for t in ("llvm-objcopy", "clang-offload-bundler",
                                             "llvm-objdump")]
    if not all(os.path.exists(t) for t in need):
        pytest.skip("ROCm LLVM tools not installed")
    fat = tmp_path / "fatbin.bin"
    subprocess.run([need[0], f"--dump-section=.hip_fatbin={fat}", lib_path, os.devnull],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = []
    at = data.find(magic)
    while at >= 0:
        starts.append(at)
        at = data.find(magic, at + 1)
    text = []
    for n, a in enumerate(starts):
        b = starts[n + 1] if n + 1 < len(starts) else len(data)
        bundle, code = tmp_path / f"b{n}.bin", tmp_path / f"b{n}.co"
        bundle.write_bytes(data[a:b])
        r = subprocess.run([need[1], "--unbundle", "--type=o",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={bundle}",
                            f"--output={code}"], capture_output=True)
        if r.returncode != 0 or not code.exists() or code.stat().st_size == 0:
            continue
        text.append(subprocess.run([need[2], "-d", "--mcpu=gfx950", str(code)], check=True,
                                   capture_output=True, text=True).stdout)
    assert text, "no gfx950 code object found"
    return text


def _vgprs(operand):
    """VGPR numbers an operand names (v7, |v7|, -v7, v[4:7]); empty for anything else."""
    import re
    m = re.fullmatch(r"[-|]*v(\d+)\|?", operand) or re.fullmatch(r"[-|]*v\[(\d+):(\d+)\]\|?",
                                                                 operand)
    if not m:
        return set()
    lo = int(m.group(1))
    hi = int(m.group(2)) if m.lastindex == 2 else lo
    return set(range(lo, hi + 1))


def test_no_valu_reads_a_transcendental_result_without_a_wait_state(tmp_path):
    """gfx950 needs one wait state between a transcendental instruction (v_exp, v_rcp, v_rsq,
    ...) and a non-transcendental VALU instruction that reads its result.  The compiler inserts it
    (an s_nop or any other instruction) for code it generates, but not in front of inline
    assembly; the exact-GELU kernels use one inline v_mul_legacy_f32, so a source change that
    hands it a v_rcp / v_exp result would read a stale register on the GPU.  Scan the built
    library's gfx950 code for any such back-to-back pair."""
    import re
    trans = re.compile(r"v_(exp|log|rcp|rsq|sqrt|sin|cos)_")
    bad = []
    for text in _gfx950_disassembly(capi.LIB_PATH, tmp_path):
        prev_dst = None  # VGPRs written by the previous instruction if it was transcendental
        for line in text.splitlines():
            m = re.match(r"\s+([a-z_0-9]+)(?:\s+(.*?))?\s*(//.*)?$", line)
            if not m or line.strip().endswith(">:"):
                continue
            op, args = m.group(1), (m.group(2) or "")
            ops = [a.strip() for a in args.split(",")] if args else []
            if prev_dst and op.startswith("v_") and not trans.match(op):
                if any(prev_dst & _vgprs(a) for a in ops[1:]):
                    bad.append(line.strip())
            prev_dst = _vgprs(ops[0]) if trans.match(op) and ops else None
    assert not bad, f"{len(bad)} reads of a transcendental result with no wait state: {bad[:5]}"


def test_c_abi_rejects_bad_arguments_without_a_device():
    lib = capi.load()
    # Every one of these fails validation before any HIP call is made.
    assert lib.fln_layernorm(None, None, None, None, -1, 8, capi.F32, 1e-5, None) == 1
    assert lib.fln_layernorm(None, None, None, None, 4, 8, capi.F32, 1e-5, None) == 1
    assert lib.fln_layernorm(ctypes.c_void_p(16), None, None, ctypes.c_void_p(16), 4, 8, 77,
                             1e-5, None) == 1
    assert lib.fln_layernorm(ctypes.c_void_p(16), None, None, ctypes.c_void_p(16), 4, 8,
                             capi.F32, -1.0, None) == 1
    assert lib.fln_layernorm_gelu(ctypes.c_void_p(16), None, None, ctypes.c_void_p(16), 4, 8,
                                  capi.F32, 1e-5, 0, None) == 1
    assert lib.fln_layernorm_fp8_forward(ctypes.c_void_p(16), None, None, ctypes.c_void_p(16),
                                         None, None, None, 4, 8, capi.F64, 1e-5, None) == 1
    assert lib.fln_rmsnorm_backward(None, None, None, None, None, None, None, 4, 8, capi.F64,
                                    capi.F32, None, 0, None) == 1
    # empty problems are a successful no-op
    assert lib.fln_layernorm(None, None, None, None, 0, 8, capi.F32, 1e-5, None) == 0
    assert lib.fln_error_string(1).decode().startswith("invalid argument")


def test_version_attributes():
    assert ext.__version__ == "1.0.0" == capi.load().fln_version().decode()
    assert ext.__cuda_version__ == ext.__hip_version__ == capi.load().fln_hip_version()
    assert fl.__version__ == "1.0.0"


def test_get_memory_usage_matches_reference_formula():
    # csrc/layernorm_cuda.cpp:144-164
    for b, h, mp in [(32, 768, False), (8, 4096, True), (1, 1, False)]:
        es = 2 if mp else 4
        expect = 2 * b * h * es + 2 * b * 4 + b * h * es + 2 * h * es + b * 32 * 4
        assert ext.get_memory_usage(b, h, mp) == expect
        assert ext.get_memory_usage(batch_size=b, hidden_size=h, use_mixed_precision=mp) == expect


def test_performance_hints_wording():
    s = ext.get_performance_hints(4, 100)
    assert "hidden_size is not divisible by 32" in s
    assert "Small batch size" in s
    assert "Not enough blocks" in s
    assert "Large hidden dimension" in ext.get_performance_hints(100000, 16384)


def _cpu(*shape, dtype=torch.float32):
    return torch.randn(*shape).to(dtype)


def test_module_eager_path_checks_arguments_on_the_host():
    """FusedLayerNorm's C++ autograd path validates before anything is launched: a last
    dimension other than normalized_shape raises torch's F.layer_norm message, a CPU tensor the
    binding's device error."""
    with pytest.raises(RuntimeError, match="normalized_shape"):
        ext.layer_norm_autograd(_cpu(2, 4), 5, None, None, 1e-5)
    with pytest.raises(RuntimeError, match="GPU"):
        ext.layer_norm_autograd(_cpu(2, 4), 4, None, None, 1e-5)
    with pytest.raises(RuntimeError, match="GPU"):
        fl.FusedLayerNorm(4)(_cpu(2, 4))
    with pytest.raises(RuntimeError, match="normalized_shape"):
        ext.rms_norm_autograd(_cpu(2, 4), 5, None, 1e-6)
    with pytest.raises(RuntimeError, match="GPU"):
        fl.FusedRMSNorm(4)(_cpu(2, 4))


@pytest.mark.parametrize("call", [
    lambda: ext.layernorm(_cpu(4, 8), _cpu(8), _cpu(8), 1e-5),
    lambda: ext.layernorm_gelu(_cpu(4, 8), _cpu(8), _cpu(8)),
    lambda: ext.forward(_cpu(4, 8)),
    lambda: ext.rms_norm_forward(_cpu(4, 8)),
    lambda: ext.layernorm_fp8_forward(_cpu(4, 8)),
    lambda: ext.backward(_cpu(4, 8), _cpu(4, 8), _cpu(4), _cpu(4)),
])
def test_binding_rejects_cpu_tensors(call):
    with pytest.raises(RuntimeError, match="GPU"):
        call()


def test_binding_reports_bad_shapes_and_dtypes_before_launch():
    # The device check comes first on CPU tensors; shape and dtype checks are exercised on
    # fake GPU tensors through the dispatcher-free Python checks of the module API.
    with pytest.raises(ValueError):
        fl.FusedLayerNormFunction.apply(_cpu(2, 3, 4), (4,), None, None, 1e-5)
    with pytest.raises(ValueError):
        fl.FusedLayerNormFunction.apply(_cpu(2, 4), (5,), None, None, 1e-5)
    with pytest.raises(RuntimeError, match="normalized_shape"):
        fl.layer_norm(_cpu(2, 4), (5,))


def test_fake_tensor_shapes_of_every_op():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(3, 5, 64, device="cuda", dtype=torch.bfloat16)
        w = torch.empty(64, device="cuda", dtype=torch.bfloat16)
        y, m, r = torch.ops.fused_layernorm.layer_norm_fwd(x, w, w, 1e-5)
        assert y.shape == x.shape and m.shape == (3, 5) and m.dtype == torch.float32
        dx, dw, db = torch.ops.fused_layernorm.layer_norm_bwd(x, x, m, r, w, w,
                                                              [True, True, False], None)
        assert dx.shape == x.shape and dw.shape == (64,) and db.numel() == 0
        y, r = torch.ops.fused_layernorm.rms_norm_fwd(x, w, 1e-6)
        assert r.shape == (3, 5)
        y, h, m, r = torch.ops.fused_layernorm.add_layer_norm_fwd(x, x, w, None, 1e-5)
        assert h.shape == x.shape
        q, s = torch.ops.fused_layernorm.layer_norm_fp8_fwd(x, None, None, 1e-5)
        assert q.dtype == torch.float8_e4m3fn and s.shape == (3, 5)
        assert fl.layer_norm_gelu(x, 64, w, w, approximate="none").shape == x.shape
        y2, h2 = fl.add_rms_norm(x, x, (64,), w)
        assert y2.shape == x.shape == h2.shape
        q, s = torch.ops.fused_layernorm.rms_norm_fp8_fwd(x, w, 1e-6)
        assert q.dtype == torch.float8_e4m3fn and s.shape == (3, 5)
        for q, s, h in (torch.ops.fused_layernorm.add_rms_norm_fp8_fwd(x, x, w, 1e-6),
                        torch.ops.fused_layernorm.add_layer_norm_fp8_fwd(x, x, w, w, 1e-5)):
            assert q.shape == x.shape and q.dtype == torch.float8_e4m3fn
            assert s.shape == (3, 5) and s.dtype == torch.float32 and h.dtype == x.dtype
        q, s, h = fl.add_rms_norm_fp8(x, x, 64, w)
        assert q.shape == x.shape and s.shape == (3, 5) and h.shape == x.shape
        q, s = torch.ops.fused_layernorm.layer_norm_mxfp8_fwd(x, w, None, 1e-5)
        assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float8_e8m0fnu
        assert s.shape == (3, 5, 2)
        q, s, h = fl.add_rms_norm_mxfp8(x, x, 64, w)
        assert s.shape == (3, 5, 2) and h.shape == x.shape


def test_module_state_dict_keys_match_nn_layernorm():
    a = fl.FusedLayerNorm(768)
    b = torch.nn.LayerNorm(768)
    assert a.state_dict().keys() == b.state_dict().keys()
    assert torch.equal(a.weight, b.weight) and torch.equal(a.bias, b.bias)
    a.load_state_dict(b.state_dict())
    assert repr(a) == "FusedLayerNorm((768,), eps=1e-05, elementwise_affine=True)"
    assert fl.FusedLayerNorm(16, elementwise_affine=False).weight is None
    assert fl.FusedRMSNorm(16).state_dict().keys() == torch.nn.RMSNorm(16).state_dict().keys()


def test_replace_and_restore_torch_layernorm(capsys):
    orig = torch.nn.LayerNorm
    fl.replace_torch_layernorm()
    try:
        assert torch.nn.LayerNorm is fl.FusedLayerNorm
    finally:
        fl.restore_torch_layernorm()
    assert torch.nn.LayerNorm is orig
    out = capsys.readouterr().out
    assert "Successfully replaced torch.nn.LayerNorm with FusedLayerNorm" in out
    assert "Restored original torch.nn.LayerNorm" in out


def test_profiler_utilities():
    p = fl.functional.get_profiler()
    fl.functional.enable_profiling()
    p.record(32, 768, 0.01, 0.02)
    p.record(32, 768, 0.03, 0.04)
    res = fl.functional.disable_profiling()
    assert res["num_calls"] == 2 and res["total"]["max_ms"] == pytest.approx(0.07)
    with pytest.raises(RuntimeError):
        fl.functional.check_input_dtype_and_device(_cpu(2, 4))


def test_optimal_config_reports_dispatch_geometry():
    c = fl.functional.get_optimal_config(8192, 4096, torch.bfloat16)
    assert c["register_resident"] and c["vector_elems"] == 8 and c["exact_tiling"]
    assert c["waves_per_row"] * 64 * c["vectors_per_lane"] * c["vector_elems"] == 4096
    c7 = fl.functional.get_optimal_config(32768, 7168, torch.bfloat16)
    assert (c7["waves_per_row"], c7["vectors_per_lane"], c7["threads_per_block"]) == (7, 2, 448)
    # Exact tilings of 3, 5, 6 or 7 vectors per lane over 1-4 waves for 16-bit LayerNorm /
    # RMSNorm and the fp8 row scale, with rows enough to fill the device (4 waves per CU), where
    # the power-of-two tiles mask more than 1/16 of their slots or use more waves; the residual,
    # MX and GELU flavours and fp32 keep their tilings.
    w7 = lambda *a, **k: (lambda c: (c["waves_per_row"], c["vectors_per_lane"],  # noqa: E731
                                     c["exact_tiling"], c["threads_per_block"]))(
        fl.functional.get_optimal_config(*a, **k))
    plain = {1536: (1, 3, True, 256), 2560: (1, 5, True, 256), 3072: (2, 3, True, 256),
             3584: (1, 7, True, 256), 4608: (3, 3, True, 192), 5120: (2, 5, True, 256),
             6144: (4, 3, True, 256), 7168: (7, 2, True, 448), 7680: (4, 4, False, 256),
             10240: (10, 2, True, 640), 4096: (2, 4, True, 256), 8192: (4, 4, True, 256)}
    fp8 = {1536: (1, 3, True, 256), 2560: (1, 5, True, 256), 3072: (1, 6, True, 256),
           3584: (1, 7, True, 256), 4608: (3, 3, True, 192), 5120: (2, 5, True, 256),
           6144: (2, 6, True, 256), 7168: (2, 7, True, 256), 7680: (4, 4, False, 256),
           10240: (4, 5, True, 256), 4096: (2, 4, True, 256)}
    for cols, want in plain.items():
        assert w7(65536, cols, torch.bfloat16) == want, cols
        assert w7(65536, cols, torch.float16, num_cus=128) == want, cols
    for cols, want in fp8.items():
        assert w7(65536, cols, torch.bfloat16, fp8=1) == want, cols
    assert w7(512, 7168, torch.float16, fp8=1) == (2, 7, True, 256)
    assert w7(511, 7168, torch.bfloat16, fp8=1)[1] != 7
    assert w7(1024, 3584, torch.float16) == (1, 7, True, 256)
    assert w7(1023, 3584, torch.bfloat16)[1] != 7
    assert w7(128, 7168, torch.bfloat16, fp8=1, num_cus=64) == (2, 7, True, 256)
    gelu = {1536: (1, 3), 2560: (1, 5), 3072: (1, 6), 5120: (2, 5), 6144: (4, 3), 7168: (2, 7)}
    for cols, (w, v) in gelu.items():
        for form in ("tanh", "none"):
            assert w7(65536, cols, torch.bfloat16, approximate=form) == (w, v, True, 256), cols
    assert w7(65536, 3584, torch.bfloat16, approximate="tanh") == (1, 7, True, 256)
    assert w7(65536, 4608, torch.bfloat16, approximate="tanh") == (3, 3, True, 192)
    # erf: the 1-wave 7-vector tile measured slower, and its table needs 256-thread blocks
    assert w7(65536, 3584, torch.bfloat16, approximate="none")[1] not in (3, 5, 6, 7)
    assert w7(65536, 4608, torch.bfloat16, approximate="none")[1] not in (3, 5, 6, 7)
    # fp32 rows of 8192 columns with 2-8 rows per CU: 16 waves x 2 vectors per lane.
    for rows in (512, 1024, 2048):
        assert w7(rows, 8192, torch.float32) == (16, 2, True, 1024), rows
    for rows in (511, 2049, 65536):
        assert w7(rows, 8192, torch.float32) != (16, 2, True, 1024), rows
    assert w7(1024, 8192, torch.float32, approximate="tanh") != (16, 2, True, 1024)
    assert w7(1024, 8192, torch.float32, fp8=1) != (16, 2, True, 1024)
    assert w7(1024, 8192, torch.float32, residual=True) != (16, 2, True, 1024)
    assert w7(1024, 8192, torch.bfloat16) != (16, 2, True, 1024)
    # fp32 LayerNorm / RMSNorm 8-vector tiles with rows enough for 32 waves per CU at half the
    # vectors: twice the waves, 4 vectors per lane (8192 columns from 64 rows per CU).
    halved = {(4096, 2048): (2, 4, True, 256), (2048, 4096): (4, 4, True, 256),
              (16384, 4096): (4, 4, True, 256), (2048, 6144): (6, 4, True, 384),
              (16384, 8192): (8, 4, True, 512)}
    for (rows, cols), tile in halved.items():
        assert w7(rows, cols, torch.float32) == tile, (rows, cols)
    kept = {(2048, 2048): (1, 8, True, 256), (1024, 4096): (2, 8, True, 256),
            (1024, 6144): (3, 8, True, 192), (4096, 8192): (4, 8, True, 256),
            (8192, 8192): (4, 8, True, 256)}
    for (rows, cols), tile in kept.items():
        assert w7(rows, cols, torch.float32) == tile, (rows, cols)
    # Residual flavours from 64 waves per CU at half the vectors and up to 6144 columns; LN +
    # GELU like LayerNorm but from 32 rows per CU at 8192 columns; fp8 outputs keep 8 vectors.
    res = {(8192, 4096): (4, 4), (16384, 2048): (2, 4), (2048, 4096): (2, 8),
           (4096, 2048): (1, 8), (16384, 8192): (4, 8)}
    for (rows, cols), wv in res.items():
        assert w7(rows, cols, torch.float32, residual=True)[:2] == wv, (rows, cols)
    for form in ("tanh", "none"):
        assert w7(2048, 4096, torch.float32, approximate=form) == (4, 4, True, 256)
        assert w7(8192, 8192, torch.float32, approximate=form) == (8, 4, True, 512)
        assert w7(4096, 8192, torch.float32, approximate=form)[:2] == (4, 8)
        assert w7(1024, 4096, torch.float32, approximate=form)[:2] == (2, 8)
    assert w7(2048, 4096, torch.float32, fp8=1)[:2] == (2, 8)
    assert w7(16384, 2048, torch.float32, fp8=1)[:2] == (1, 8)
    assert w7(4096, 2048, torch.float32, num_cus=512) == (1, 8, True, 256)
    # Residual flavours: 3 or 5 vectors per lane only, at the shapes each measured faster with.
    odd = lambda c: c[1] in (3, 5, 6, 7)  # noqa: E731
    res = {"": {1536: (1, 3), 2560: (1, 5), 3072: (2, 3), 4608: (3, 3), 6144: (4, 3)},
           "fp8": {1536: (1, 3), 2560: (1, 5), 3072: (2, 3), 4608: (3, 3), 5120: (2, 5)},
           "mx": {1536: (1, 3), 2560: (1, 5), 3072: (2, 3), 4608: (3, 3), 6144: (4, 3)}}
    for name, fp in (("", 0), ("fp8", 1), ("mx", 2)):
        for cols in (1536, 2560, 3072, 3584, 4608, 5120, 6144, 7168):
            got = w7(65536, cols, torch.bfloat16, fp8=fp, residual=True)
            if cols in res[name]:
                w, v = res[name][cols]
                assert got == (w, v, True, 256 if w != 3 else 192), (name, cols, got)
            else:
                assert not odd(got), (name, cols, got)
    for k in (dict(fp8=2), dict(dtype=torch.float32), dict(dtype=torch.float32, approximate="tanh")):
        dt = k.pop("dtype", torch.bfloat16)
        for cols in (1536, 2560, 3584, 5120, 7168):
            assert not odd(w7(65536, cols, dt, **k)), (k, cols)
    # Exact tilings of one vector per lane only for rows too few to fill the device (C1);
    # with many rows a power-of-two tiling with masked slots is taken instead, unless 3-7
    # vectors per lane tile the row exactly (2560: 1 x 5; 6656 = 13 x 512 has none).
    wt = lambda c: (c["waves_per_row"], c["vectors_per_lane"], c["exact_tiling"])  # noqa: E731
    assert wt(fl.functional.get_optimal_config(32, 768, torch.float32)) == (3, 1, True)
    assert wt(fl.functional.get_optimal_config(16384, 2560, torch.bfloat16)) == (1, 5, True)
    assert wt(fl.functional.get_optimal_config(16384, 2560, torch.float32)) == (5, 2, True)
    assert wt(fl.functional.get_optimal_config(16384, 6656, torch.bfloat16)) == (4, 4, False)
    c2 = fl.functional.get_optimal_config(2048, 100000, torch.float32)
    assert not c2["register_resident"] and not c2["lds_staged"] and c2["wide_streamed"]
    # Few rows split over several blocks each: under 4 per CU past the LDS tile, under a
    # quarter of the CUs within it.
    c1 = fl.functional.get_optimal_config(1, 100000, torch.float32)
    assert c1["split_rows"] and not c1["wide_streamed"] and not c1["lds_staged"]
    assert fl.functional.get_optimal_config(1023, 262144, torch.bfloat16)["split_rows"]
    assert not fl.functional.get_optimal_config(1024, 262144, torch.bfloat16)["split_rows"]
    assert fl.functional.get_optimal_config(63, 65536, torch.bfloat16)["split_rows"]
    c3 = fl.functional.get_optimal_config(64, 65536, torch.bfloat16)
    assert not c3["register_resident"] and c3["lds_staged"] and not c3["wide_streamed"]
    c4 = fl.functional.get_optimal_config(64, 40001, torch.bfloat16)  # unaligned: streamed
    assert not c4["register_resident"] and not c4["lds_staged"] and c4["wide_streamed"]
    c5 = fl.functional.get_optimal_config(64, 20480, torch.float32)  # no fp32 RAW tiles
    assert not c5["register_resident"] and c5["lds_staged"]
    # Rows of more than 4 waves: at most 16 elements per lane (1024-thread blocks have 128
    # VGPRs), exact tilings within that cap, the 32-element tiles only past 16 waves.
    geo = lambda c: (c["waves_per_row"], c["vectors_per_lane"], c["exact_tiling"],  # noqa: E731
                     c["threads_per_block"])
    assert geo(fl.functional.get_optimal_config(4096, 12288, torch.bfloat16)) == (12, 2, True, 768)
    assert geo(fl.functional.get_optimal_config(4096, 16384, torch.bfloat16)) == (16, 2, True, 1024)
    assert geo(fl.functional.get_optimal_config(2048, 32768, torch.bfloat16)) == (16, 4, True, 1024)
    assert geo(fl.functional.get_optimal_config(4096, 16384, torch.float32)) == (16, 4, True, 1024)
    assert geo(fl.functional.get_optimal_config(8192, 8192, torch.bfloat16)) == (4, 4, True, 256)
    assert geo(fl.functional.get_optimal_config(4096, 8192, torch.float32)) == (4, 8, True, 256)
    # Rows of 65537..131072 16-bit columns: half of each row in LDS, half in registers, for
    # LayerNorm and the tanh GELU; the exact GELU and the residual / fp8 flavours stream them
    # (split over several blocks each below 4 rows per CU, 1.5 with fp8 outputs).
    route = lambda *a, **k: fl.functional.get_optimal_config(*a, **k)["route"]  # noqa: E731
    assert route(512, 131072, torch.bfloat16) == "lds+registers"
    assert route(512, 131072, torch.bfloat16, approximate="tanh") == "lds+registers"
    assert route(2048, 131072, torch.bfloat16, approximate="none") == "wide"
    assert route(512, 131072, torch.bfloat16, approximate="none") == "split"
    assert route(2048, 131072, torch.bfloat16, residual=True) == "wide"
    assert route(512, 131072, torch.bfloat16, fp8=1) == "wide"
    assert route(256, 131072, torch.bfloat16, fp8=1) == "split"
    assert route(512, 65536, torch.float32, approximate="none") == "lds+registers"
    assert route(512, 65536, torch.bfloat16) == "lds"
    assert route(16, 65536, torch.bfloat16) == "split"
    assert route(4, 8, torch.float64) == "loop"
    assert route(0, 4096, torch.bfloat16) == "none"
    # The plan is the dispatcher's rule for the CU count asked for (the split limits scale).
    assert route(63, 65536, torch.bfloat16, num_cus=256) == "split"
    assert route(63, 65536, torch.bfloat16, num_cus=128) == "lds"


def test_forward_plan_rejects_bad_arguments():
    import capi
    lib = capi.load()
    plan = (ctypes.c_int * 6)()
    assert lib.fln_forward_plan(8, 4096, capi.BF16, 0, 0, 0, 256, plan) == 0
    assert list(plan)[:2] == [0, 8]
    bad = [(-1, 4096, capi.BF16, 0, 0, 0, 256), (8, 4096, 9, 0, 0, 0, 256),
           (8, 4096, capi.BF16, 3, 0, 0, 256), (8, 4096, capi.BF16, 0, 0, 3, 256),
           (8, 4096, capi.BF16, 1, 0, capi.GELU_TANH, 256), (8, 4112, capi.BF16, 2, 0, 0, 256),
           (8, 4096, capi.F64, 1, 0, 0, 256), (8, 4096, capi.F64, 0, 1, 0, 256),
           (8, 4096, capi.BF16, 0, 0, 0, -1)]
    for args in bad:
        assert lib.fln_forward_plan(*args, plan) == capi.ERR_INVALID, args
    assert lib.fln_forward_plan(8, 4096, capi.BF16, 0, 0, 0, 256, None) == capi.ERR_INVALID


def test_byte_model_matches_baseline_figures():
    expect = {
        "c1_ln_fwd_fp32_32x768": 202752,
        "c2_ln_gelu_fp32_17x1023": 147312,
        "c2_ln_gelu_fp32_64x4096": 2129920,
        "c3_add_ln_fwd_bf16_8192x4096": 268451840,
        "c4_rms_fwd_bwd_bf16_16384x8192": 1342373888,
        "c5_ln_fp8_bf16_32768x7168": 704802816,
        "ln_fwd_bwd_bf16_8192x4096": 335732736,
        "rms_fwd_bwd_bf16_8192x4096": 335642624,
    }
    for name, nbytes in expect.items():
        assert algorithmic_bytes(WORKLOADS[name])["total"] == nbytes, name


def test_replace_layernorm_modules_swaps_and_shares_parameters():
    model = torch.nn.Sequential(
        torch.nn.TransformerEncoderLayer(d_model=64, nhead=4, dim_feedforward=128, dropout=0.0),
        torch.nn.LayerNorm(64, elementwise_affine=False), torch.nn.RMSNorm(64, eps=1e-6),
        torch.nn.Linear(64, 10))
    keys = list(model.state_dict().keys())
    w1 = model[0].norm1.weight
    fl.replace_layernorm_modules(model)
    assert isinstance(model[0].norm1, fl.FusedLayerNorm)
    assert isinstance(model[0].norm2, fl.FusedLayerNorm)
    assert isinstance(model[1], fl.FusedLayerNorm) and model[1].weight is None
    assert isinstance(model[2], fl.FusedRMSNorm) and model[2].eps == 1e-6
    assert model[0].norm1.weight is w1  # the same Parameter object
    assert list(model.state_dict().keys()) == keys
