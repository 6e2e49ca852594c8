"""Pins the CPU oracle (oracle/norms.py, oracle/fln_oracle.c) -- CPU only.

The reference ships no golden vectors or known-answer files (its tests compare live against
PyTorch on the GPU), so each oracle function is pinned by checks chosen so that a plausible
mistake (dropped term, wrong sign, wrong reduction axis, biased/unbiased mix-up, transposed
operand, wrong rounding) fails at least one of them:
  * library routines: torch-CPU F.layer_norm / F.rms_norm / F.gelu and autograd in float64;
  * closed forms and invariants (hand-computed rows, mean 0 / variance 1, N = 1, constant rows);
  * finite differences (torch.autograd.gradcheck on the oracle's closed-form backward);
  * a known-answer table and an exhaustive decode/encode round trip for fp8 e4m3fn, plus
    torch's own float8_e4m3fn cast after clamping;
  * the C oracle against the numpy oracle.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle, norms


def t64(a):
    return torch.tensor(np.asarray(a), dtype=torch.float64)


@pytest.fixture(scope="module")
def rng():
    return np.random.RandomState(1234)


# ---------------------------------------------------------------- LayerNorm forward
def test_layer_norm_hand_computed_row():
    # x = [1, 2, 3, 4]: mean 2.5, biased variance 1.25 (reference kernel.cu:69-80 divides by N).
    y, mean, rstd = norms.layer_norm_fwd(np.array([[1.0, 2.0, 3.0, 4.0]]), eps=0.0)
    assert mean[0] == 2.5
    assert rstd[0] == pytest.approx(1 / math.sqrt(1.25), rel=1e-15)
    np.testing.assert_allclose(y[0], (np.array([1, 2, 3, 4]) - 2.5) / math.sqrt(1.25),
                               rtol=1e-15)


@pytest.mark.parametrize("shape", [(3, 5), (7, 768), (2, 3, 1023), (4, 4096)])
def test_layer_norm_matches_torch(rng, shape):
    x = rng.randn(*shape) * 3 + 0.5
    g = 1 + 0.1 * rng.randn(shape[-1])
    b = 0.1 * rng.randn(shape[-1])
    for gg, bb in ((g, b), (None, None), (g, None), (None, b)):
        y, _, _ = norms.layer_norm_fwd(x, gg, bb, 1e-5)
        yt = F.layer_norm(t64(x), (shape[-1],), None if gg is None else t64(gg),
                          None if bb is None else t64(bb), 1e-5)
        np.testing.assert_allclose(y, yt.numpy(), rtol=1e-12, atol=1e-12)


def test_layer_norm_invariants(rng):
    x = rng.randn(16, 513) * 1000 + 7
    y, _, _ = norms.layer_norm_fwd(x, eps=0.0)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(-1), 1, rtol=1e-12)  # biased variance == 1
    # N = 1 and constant rows -> the output is beta exactly
    b = np.array([0.25])
    y1, _, _ = norms.layer_norm_fwd(rng.randn(9, 1), np.array([3.0]), b)
    assert (y1 == 0.25).all()
    yc, _, _ = norms.layer_norm_fwd(np.full((2, 768), 1e8), None, np.full(768, -0.5))
    assert (yc == -0.5).all()


def test_gelu_matches_torch_and_reference_formula(rng):
    v = rng.randn(10000) * 4
    np.testing.assert_allclose(norms.gelu(v, "none"), F.gelu(t64(v)).numpy(), rtol=1e-12,
                               atol=1e-14)
    np.testing.assert_allclose(norms.gelu(v, "tanh"),
                               F.gelu(t64(v), approximate="tanh").numpy(), rtol=1e-12,
                               atol=1e-14)
    # reference formula, csrc/layernorm_cuda_kernel.cu:31-36
    s = math.sqrt(2 / math.pi)
    ref = [0.5 * a * (1 + math.tanh(s * (a + 0.044715 * a ** 3))) for a in v[:50]]
    np.testing.assert_allclose(norms.gelu(v[:50], "tanh"), ref, rtol=1e-13, atol=1e-15)
    assert norms.gelu(np.array([0.0]), "none")[0] == 0.0
    np.testing.assert_allclose(norms.gelu(np.array([40.0, -40.0]), "none"), [40.0, 0.0])


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_gelu_grad_and_layer_norm_gelu_backward_match_autograd(rng, approximate):
    v = t64(rng.randn(5000) * 4).requires_grad_(True)
    F.gelu(v, approximate=approximate).sum().backward()
    np.testing.assert_allclose(norms.gelu_grad(v.detach().numpy(), approximate), v.grad.numpy(),
                               rtol=1e-12, atol=1e-14)
    x = rng.randn(6, 300) * 2 + 0.3
    g, b, dy = 1 + 0.1 * rng.randn(300), 0.2 * rng.randn(300), rng.randn(6, 300)
    xt, gt, bt = (t64(a).requires_grad_(True) for a in (x, g, b))
    F.gelu(F.layer_norm(xt, (300,), gt, bt, 1e-5), approximate=approximate).backward(t64(dy))
    dx, dg, db = norms.layer_norm_gelu_bwd(dy, x, g, b, 1e-5, approximate)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, gt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_layer_norm_gelu_composition(rng):
    x, g, b = rng.randn(5, 64), 1 + 0.1 * rng.randn(64), 0.1 * rng.randn(64)
    y = norms.layer_norm_gelu_fwd(x, g, b, 1e-5, "none")
    yt = F.gelu(F.layer_norm(t64(x), (64,), t64(g), t64(b), 1e-5))
    np.testing.assert_allclose(y, yt.numpy(), rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------- RMSNorm, residual
def test_rms_norm_matches_torch(rng):
    x, w = rng.randn(6, 1000) * 2, 1 + 0.1 * rng.randn(1000)
    y, rstd = norms.rms_norm_fwd(x, w, 1e-6)
    yt = F.rms_norm(t64(x), (1000,), t64(w), 1e-6)
    np.testing.assert_allclose(y, yt.numpy(), rtol=1e-12)
    np.testing.assert_allclose(rstd, 1 / np.sqrt((x ** 2).mean(-1) + 1e-6), rtol=1e-14)


def test_bf16_rounding_matches_torch(rng):
    a = np.concatenate([rng.randn(100000).astype(np.float32) * 10,
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 0.0, -0.0,
                                  np.inf, -np.inf, 3.4e38], np.float32)])
    ours = norms.round_to_bf16(a)
    theirs = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1
    assert norms.round_to_bf16(np.float32(1 + 2 ** -8)) == 1.0


def test_add_layer_norm_rounds_h_before_statistics(rng):
    x = torch.randn(4, 256).to(torch.bfloat16)
    r = torch.randn(4, 256).to(torch.bfloat16)
    y, h, _, _ = norms.add_layer_norm_fwd(x.float().numpy(), r.float().numpy(), eps=1e-5)
    h_t = (x + r).float()
    assert np.array_equal(h, h_t.numpy())
    yt = F.layer_norm(h_t.double(), (256,), eps=1e-5)
    np.testing.assert_allclose(y, yt.numpy(), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- backward
@pytest.mark.parametrize("shape", [(3, 5), (16, 768), (2, 4, 33)])
def test_layer_norm_backward_matches_autograd(rng, shape):
    x, dy = rng.randn(*shape), rng.randn(*shape)
    g, b = 1 + 0.1 * rng.randn(shape[-1]), 0.1 * rng.randn(shape[-1])
    xt, gt, bt = (t64(a).requires_grad_(True) for a in (x, g, b))
    F.layer_norm(xt, (shape[-1],), gt, bt, 1e-5).backward(t64(dy))
    dx, dg, db = norms.layer_norm_bwd(dy, x, g, 1e-5)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, gt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("shape", [(3, 5), (16, 768)])
def test_rms_norm_backward_matches_autograd(rng, shape):
    x, dy, w = rng.randn(*shape), rng.randn(*shape), 1 + 0.1 * rng.randn(shape[-1])
    xt, wt = t64(x).requires_grad_(True), t64(w).requires_grad_(True)
    F.rms_norm(xt, (shape[-1],), wt, 1e-6).backward(t64(dy))
    dx, dw = norms.rms_norm_bwd(dy, x, w, 1e-6)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_closed_forms_against_finite_differences(rng):
    """Brute force: central differences of sum(dy * LN(x)) and sum(dy * RMS(x))."""
    x, dy, g = rng.randn(3, 5), rng.randn(3, 5), 1 + 0.3 * rng.randn(5)
    b = 0.2 * rng.randn(5)
    h = 1e-6

    def loss_ln(xx, gg, bb):
        return float((dy * norms.layer_norm_fwd(xx, gg, bb, 1e-5)[0]).sum())

    def loss_rms(xx, gg):
        return float((dy * norms.rms_norm_fwd(xx, gg, 1e-6)[0]).sum())

    dx, dg, db = norms.layer_norm_bwd(dy, x, g, 1e-5)
    dxr, dgr = norms.rms_norm_bwd(dy, x, g, 1e-6)
    for idx in np.ndindex(x.shape):
        e = np.zeros_like(x)
        e[idx] = h
        fd = (loss_ln(x + e, g, b) - loss_ln(x - e, g, b)) / (2 * h)
        assert fd == pytest.approx(dx[idx], rel=1e-5, abs=1e-7)
        fdr = (loss_rms(x + e, g) - loss_rms(x - e, g)) / (2 * h)
        assert fdr == pytest.approx(dxr[idx], rel=1e-5, abs=1e-7)
    for j in range(5):
        e = np.zeros(5)
        e[j] = h
        assert (loss_ln(x, g + e, b) - loss_ln(x, g - e, b)) / (2 * h) == \
            pytest.approx(dg[j], rel=1e-6, abs=1e-8)
        assert (loss_ln(x, g, b + e) - loss_ln(x, g, b - e)) / (2 * h) == \
            pytest.approx(db[j], rel=1e-6, abs=1e-8)
        assert (loss_rms(x, g + e) - loss_rms(x, g - e)) / (2 * h) == \
            pytest.approx(dgr[j], rel=1e-6, abs=1e-8)


# ---------------------------------------------------------------- fp8 e4m3fn
KNOWN_FP8 = [
    (0.0, 0x00), (-0.0, 0x80), (448.0, 0x7E), (-448.0, 0xFE), (2.0 ** -9, 0x01),
    (2.0 ** -6, 0x08), (0.0625, 0x18), (1.0, 0x38), (-1.0, 0xB8), (1.125, 0x39), (1.75, 0x3E),
    (2.0, 0x40), (240.0, 0x77), (256.0, 0x78), (416.0, 0x7D),
    (1.0625, 0x38),            # tie between 1.0 (even) and 1.125 -> 1.0
    (1.1875, 0x3A),            # tie between 1.125 and 1.25 (even) -> 1.25
    (2.0 ** -10, 0x00),        # tie between 0 and the smallest subnormal -> 0
    (3 * 2.0 ** -10, 0x02),    # tie between 1 and 2 subnormal steps -> 2 (even)
    (464.0, 0x7E), (480.0, 0x7E), (1e6, 0x7E), (-1e6, 0xFE),  # saturation
]


def test_fp8_known_answers():
    vals = np.array([v for v, _ in KNOWN_FP8])
    codes = norms.fp8_e4m3fn_encode(vals)
    assert [int(c) for c in codes] == [c for _, c in KNOWN_FP8]
    assert [c_oracle.fp8_encode_scalar(v) for v in vals] == [c for _, c in KNOWN_FP8]
    assert norms.fp8_e4m3fn_encode(np.array([np.nan]))[0] == 0x7F


def test_fp8_decode_encode_round_trip_all_codes():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    vals = norms.fp8_e4m3fn_decode(codes)
    assert np.array_equal(norms.fp8_e4m3fn_encode(vals), codes)
    # decoded values are strictly increasing over the positive codes (no gaps, no overlaps)
    pos = norms.fp8_e4m3fn_decode(np.arange(0, 0x7F, dtype=np.uint8))
    assert (np.diff(pos) > 0).all() and pos[-1] == 448.0


def test_fp8_matches_torch_cast_after_clamp(rng):
    v = np.concatenate([rng.randn(200000) * 100, rng.randn(50000) * 0.01,
                        np.linspace(-450, 450, 100001)]).astype(np.float32)
    ours = norms.fp8_e4m3fn_encode(v.astype(np.float64))
    t = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(ours, t.numpy())


def test_layer_norm_fp8_row_scale_and_codes(rng):
    x = rng.randn(8, 300).astype(np.float32)
    x[:, 7] *= 20
    q, s = norms.layer_norm_fp8_fwd(x, None, None, 1e-5)
    y, _, _ = norms.layer_norm_fwd(x, None, None, 1e-5)
    np.testing.assert_allclose(s, np.abs(y).max(-1) / 448, rtol=1e-7)
    assert (np.abs(norms.fp8_e4m3fn_decode(q)).max(-1) == 448).all()
    deq = norms.fp8_e4m3fn_decode(q) * s[:, None]
    assert np.abs(deq - y).max() <= np.abs(y).max() * 2 ** -4  # 3 mantissa bits
    qz, sz = norms.layer_norm_fp8_fwd(np.zeros((2, 16), np.float32), None, None)
    assert (qz == 0).all() and (sz == 0).all()


def _torch_fp8_rows(y64):
    """PyTorch's own composition of the fp8 row rule: amax / 448 scale, divide, clamp, cast."""
    amax = y64.abs().amax(-1, keepdim=True)
    scale = amax / 448.0
    q = torch.where(amax > 0, y64 / torch.where(amax > 0, scale, torch.ones_like(scale)),
                    torch.zeros_like(y64))
    return q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy(), \
        scale[..., 0].float().numpy()


def test_rms_and_residual_fp8_variants_match_torch_composition(rng):
    x = rng.randn(12, 768).astype(np.float32)
    x[:, 5] *= 30
    r = rng.randn(12, 768).astype(np.float32)
    w = (1 + 0.1 * rng.randn(768)).astype(np.float32)
    b = (0.1 * rng.randn(768)).astype(np.float32)
    # RMSNorm -> fp8
    q, s = norms.rms_norm_fp8_fwd(x, w, 1e-6)
    qt, st = _torch_fp8_rows(F.rms_norm(t64(x), (768,), t64(w), 1e-6))
    assert np.array_equal(q, qt) and np.array_equal(s, st)
    qc, sc = c_oracle.rmsnorm_fp8(x, w, 1e-6)
    assert np.array_equal(qc, q) and np.array_equal(sc, s)
    # residual add (bf16 rounding of h, as torch's bf16 add) + RMSNorm / LayerNorm -> fp8
    xb = torch.from_numpy(x).to(torch.bfloat16)
    rb = torch.from_numpy(r).to(torch.bfloat16)
    hb = xb + rb
    q, s, h = norms.add_rms_norm_fp8_fwd(xb.float().numpy(), rb.float().numpy(), w, 1e-6)
    assert np.array_equal(h, hb.float().numpy())
    qt, st = _torch_fp8_rows(F.rms_norm(hb.double(), (768,), t64(w), 1e-6))
    assert np.array_equal(q, qt) and np.array_equal(s, st)
    q, s, h = norms.add_layer_norm_fp8_fwd(xb.float().numpy(), rb.float().numpy(), w, b, 1e-5)
    qt, st = _torch_fp8_rows(F.layer_norm(hb.double(), (768,), t64(w), t64(b), 1e-5))
    assert np.array_equal(q, qt) and np.array_equal(s, st)


def test_mx_e4m3_known_answers():
    # block maxima 448 -> e = 0 (byte 127); 1.0 -> e = -8 (119); 2^-130 and 0 -> clamp (0)
    y = np.zeros((1, 128))
    y[0, 0], y[0, 32], y[0, 64] = 448.0, 1.0, 2.0 ** -130
    y[0, 33] = 0.5
    q, sc = norms.mx_e4m3_quantize(y)
    assert list(sc[0]) == [127, 119, 0, 0]
    assert q[0, 0] == 0x7E                       # 448 * 2^0
    assert norms.fp8_e4m3fn_decode(q[0, 32:34]).tolist() == [256, 128]  # 1.0, 0.5 at 2^8
    assert (q[0, 96:] == 0).all()
    # a maximum just below 2^9 * 2^e: 511.9 -> e = 0 and the element saturates to 448
    q2, sc2 = norms.mx_e4m3_quantize(np.full((1, 32), 511.9))
    assert sc2[0, 0] == 127 and (q2 == 0x7E).all()


def test_mx_e4m3_matches_torch_casts(rng):
    y = rng.randn(16, 512) * np.exp(rng.randn(16, 1) * 3)
    y[:, 40] *= 50
    q, sc = norms.mx_e4m3_quantize(y)
    yt = t64(y).reshape(16, 16, 32)
    amax = yt.abs().amax(-1)
    e = (torch.frexp(amax).exponent - 1 - 8).clamp(-127, 127)
    qt = (yt * torch.exp2(-e.double())[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.array_equal(q, qt.view(torch.uint8).reshape(16, 512).numpy())
    e8 = torch.exp2(e.double()).to(torch.float8_e8m0fnu).view(torch.uint8).numpy()
    assert np.array_equal(sc, e8)           # torch's E8M0 encoding of 2^e is the byte e + 127
    # dequantization: within half an e4m3 step (2^-4 relative, or half the subnormal step
    # 2^-10 of the block scale), except block values above 448 2^e, which saturate to it
    x = 2.0 ** (sc.astype(float) - 127)[..., None]
    deq = norms.fp8_e4m3fn_decode(q).reshape(16, 16, 32) * x
    yb = y.reshape(16, 16, 32)
    sat = np.abs(yb) > 448 * x
    assert (np.abs(deq - yb) <= np.abs(yb) * 2.0 ** -4 + x * 2.0 ** -10)[~sat].all()
    assert np.array_equal(deq[sat], np.sign(yb[sat]) * 448 * np.broadcast_to(x, yb.shape)[sat])


def test_mx_e4m3_non_finite_blocks_take_the_e8m0_nan(rng):
    """A block holding a NaN or an infinity: torch's amax propagates the NaN, and its
    float8_e8m0fnu cast of 2^(floor(log2 max) - 8) gives 0xFF (E8M0's NaN) for both; the other
    blocks keep the scales and codes they have without the non-finite values."""
    y = rng.randn(3, 128) * 3
    bad = y.copy()
    bad[0, 5], bad[1, 70], bad[2, 127] = np.nan, np.inf, -np.inf
    q, sc = norms.mx_e4m3_quantize(bad)
    amax = t64(bad).reshape(3, 4, 32).abs().amax(-1)
    e8 = torch.exp2(torch.floor(torch.log2(amax)) - 8).to(torch.float8_e8m0fnu)
    assert np.array_equal(sc, e8.view(torch.uint8).numpy())
    assert sc[0, 0] == sc[1, 2] == sc[2, 3] == 0xFF and (sc == 0xFF).sum() == 3
    q0, sc0 = norms.mx_e4m3_quantize(y)
    keep = sc != 0xFF
    assert np.array_equal(sc[keep], sc0[keep])
    blocks = np.repeat(keep, 32, axis=1)
    assert np.array_equal(q[blocks], q0[blocks])


def test_row_fp8_scale_of_a_non_finite_row_is_nan(rng):
    """torch's amax of a row's LayerNorm / RMSNorm outputs is NaN as soon as one is NaN (a NaN
    input, or an infinity, which makes the mean infinite and every centred value NaN or
    infinite); both oracles give that NaN scale and leave the other rows alone."""
    x = rng.randn(4, 96).astype(np.float32)
    bad = x.copy()
    bad[1, 7], bad[2, 95] = np.nan, np.inf
    with np.errstate(invalid="ignore", over="ignore"):
        for q, s in [norms.layer_norm_fp8_fwd(bad), c_oracle.layernorm_fp8(bad)]:
            yt = F.layer_norm(t64(bad), (96,), eps=1e-5)
            assert np.isnan(s[1:3]).all() and yt.abs().amax(-1)[1:3].isnan().all()
            q0, s0 = norms.layer_norm_fp8_fwd(x)
            assert np.array_equal(q[[0, 3]], q0[[0, 3]])
            np.testing.assert_allclose(s[[0, 3]], s0[[0, 3]], rtol=1e-7)
        for q, s in [norms.rms_norm_fp8_fwd(bad), c_oracle.rmsnorm_fp8(bad)]:
            assert np.isnan(s[1]), s      # a NaN row: NaN
            assert np.isnan(s[2]), s      # rstd = 0: zeros and inf * 0 = NaN


def test_mx_rows_with_unusable_statistics_read_as_nan(rng):
    """MXFP8 of a row whose statistics are not usable: every block scale 0xFF, whatever the
    block holds (LayerNorm: all of y is NaN there, as in torch's composition; RMSNorm with an
    infinity: rstd = 0 leaves zeros beside one NaN, where torch's composition would mark only the
    NaN's block); the other rows are those of the clean input, and eps = 0 on a constant row
    flags that row (rstd infinite)."""
    x = rng.randn(5, 96)
    bad = x.copy()
    bad[1, 7], bad[3, 95] = np.nan, np.inf
    for fn in (norms.layer_norm_mxfp8_fwd, norms.rms_norm_mxfp8_fwd):
        q, sc = fn(bad)
        q0, sc0 = fn(x)
        assert (sc[[1, 3]] == 0xFF).all() and (sc0 != 0xFF).all(), fn
        keep = [0, 2, 4]
        assert np.array_equal(sc[keep], sc0[keep]) and np.array_equal(q[keep], q0[keep]), fn
    with np.errstate(invalid="ignore"):
        y = norms.rms_norm_fwd(bad[3:4])[0]
    assert np.isnan(y[0, 95]) and (y[0, :95] == 0).all()   # what the flag stands in for
    const = np.ones((2, 64))
    const[1] = rng.randn(64)
    _, s = norms.layer_norm_fp8_fwd(const, eps=0.0)
    assert np.isnan(s[0]) and np.isfinite(s[1]) and s[1] > 0
    _, sc = norms.layer_norm_mxfp8_fwd(const, eps=0.0)
    assert (sc[0] == 0xFF).all() and (sc[1] != 0xFF).all()


# ---------------------------------------------------------------- C oracle vs numpy oracle
def test_c_oracle_matches_numpy_oracle(rng):
    x = rng.randn(9, 1023).astype(np.float32)
    dy = rng.randn(9, 1023).astype(np.float32)
    g = (1 + 0.1 * rng.randn(1023)).astype(np.float32)
    b = (0.1 * rng.randn(1023)).astype(np.float32)
    y, m, r = c_oracle.layernorm_fwd(x, g, b, 1e-5)
    yn, mn, rn = norms.layer_norm_fwd(x, g, b, 1e-5)
    np.testing.assert_allclose(y, yn, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(m, mn, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(r, rn, rtol=1e-13)
    dx, dg, db = c_oracle.layernorm_bwd(dy, x, g, 1e-5)
    dxn, dgn, dbn = norms.layer_norm_bwd(dy, x, g, 1e-5)
    np.testing.assert_allclose(dx, dxn, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dg, dgn, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, dbn, rtol=1e-12, atol=1e-12)
    yr, rr = c_oracle.rmsnorm_fwd(x, g, 1e-6)
    yrn, rrn = norms.rms_norm_fwd(x, g, 1e-6)
    np.testing.assert_allclose(yr, yrn, rtol=1e-6, atol=1e-6)
    dxr, dwr = c_oracle.rmsnorm_bwd(dy, x, g, 1e-6)
    dxrn, dwrn = norms.rms_norm_bwd(dy, x, g, 1e-6)
    np.testing.assert_allclose(dxr, dxrn, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dwr, dwrn, rtol=1e-12, atol=1e-12)
    q, s = c_oracle.layernorm_fp8(x, g, b, 1e-5)
    qn, sn = norms.layer_norm_fp8_fwd(x, g, b, 1e-5)
    assert np.array_equal(q, qn)
    np.testing.assert_allclose(s, sn, rtol=1e-7)


def test_c_fp8_encoder_matches_numpy_on_a_sweep(rng):
    v = np.concatenate([rng.randn(3000) * 100, rng.randn(1000) * 1e-3,
                        [(1 + m / 16) * 2.0 ** e for e in range(-11, 10) for m in range(16)]])
    ours = norms.fp8_e4m3fn_encode(v)
    assert [c_oracle.fp8_encode_scalar(a) for a in v] == [int(c) for c in ours]


# ------------------------------------------------------------------------------------------------
# The dx error model (oracle/tolerance.py) used by the GPU parity bar.
# ------------------------------------------------------------------------------------------------
def _fp32_dx(x, dy, gamma, eps, rms, order="pairwise", round_g=False, round_xh=False,
             out="bf16"):
    """An fp32 evaluation of dx = rstd (g - c1 - xhat c2), rounded once to the output type:
    statistics and row sums in fp32 (numpy's pairwise sums, or sequential running sums), with
    optional planted bf16 roundings of g = dy gamma or of xhat."""
    f = np.float32
    x32, dy32, g32 = x.astype(f), dy.astype(f), gamma.astype(f)
    n = x.shape[-1]

    def rowsum(a):
        if order == "pairwise":
            return a.sum(axis=1, keepdims=True, dtype=f)
        if order == "lanes":
            # running sums over 64 elements per lane, then a tree over the lanes (the kernels'
            # shape: per-lane partials, then cross-lane and cross-wave reductions)
            k = min(64, a.shape[1])
            part = np.cumsum(a.reshape(a.shape[0], -1, k), axis=2, dtype=f)[:, :, -1]
            return part.sum(axis=1, keepdims=True, dtype=f)
        return np.cumsum(a, axis=1, dtype=f)[:, -1:]

    if rms:
        mu = np.zeros((x.shape[0], 1), f)
        rs = (f(1) / np.sqrt(rowsum(x32 * x32) / f(n) + f(eps))).astype(f)
    else:
        mu = (rowsum(x32) / f(n)).astype(f)
        rs = (f(1) / np.sqrt(rowsum((x32 - mu) ** 2) / f(n) + f(eps))).astype(f)
    xh = ((x32 - mu) * rs).astype(f)
    gd = (dy32 * g32).astype(f)
    if round_g:
        gd = norms.round_to_bf16(gd).astype(f)
    if round_xh:
        xh = norms.round_to_bf16(xh).astype(f)
    cb = f(0) if rms else (-rs * (rowsum(gd) / f(n))).astype(f)
    cx = (-rs * (rowsum(gd * xh) / f(n))).astype(f)
    dx = (rs * gd + (cx * xh + cb)).astype(f)
    return norms.round_to_bf16(dx) if out == "bf16" else dx.astype(np.float64)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (16, 8192), (4, 65536)])
@pytest.mark.parametrize("rms", [False, True], ids=["ln", "rms"])
def test_dx_allowance_covers_fp32_and_rejects_bf16_intermediates(rows, cols, rms):
    """The dx bar (1 ulp + oracle.tolerance.dx_allowance) holds for an fp32 evaluation of the
    formula, with pairwise or sequential row sums, in bf16 and fp32 outputs, on data with an
    offset mean; and it rejects the same evaluation with g = dy gamma or xhat rounded to bf16
    (what the previous bar, 2^-12 max|dx|, could let through).  Row sums: pairwise, running
    sums of 64 elements per lane then a tree (the kernels' order), and fully sequential running
    sums up to 1024 columns (longer sequential sums grow past a log2 N model; no kernel sums more
    than 64 elements of a row in one running sum)."""
    from oracle import tolerance
    rng = np.random.RandomState(rows + cols + rms)
    to_bf16 = norms.round_to_bf16
    x = to_bf16(rng.standard_normal((rows, cols)) * 1.5 + 0.25)
    dy = to_bf16(rng.standard_normal((rows, cols)))
    g = to_bf16(1 + 0.1 * rng.standard_normal(cols))
    eps = 1e-6 if rms else 1e-5
    if rms:
        ref, _ = norms.rms_norm_bwd(dy, x, g, eps)
    else:
        ref, _, _ = norms.layer_norm_bwd(dy, x, g, eps)
    al = tolerance.dx_allowance(x, dy, g, eps, rms=rms)
    for order in ("pairwise", "lanes") + (("sequential",) if cols <= 1024 else ()):
        for out in ("bf16", "f32"):
            got = _fp32_dx(x, dy, g, eps, rms, order=order, out=out)
            err = np.abs(got - ref)
            assert (err <= tolerance.ulp(ref, out) + al).all(), (order, out)
    for plant in ("round_g", "round_xh"):
        got = _fp32_dx(x, dy, g, eps, rms, **{plant: True})
        assert (np.abs(got - ref) > tolerance.ulp(ref, "bf16") + al).any(), plant
    # For a typical element the bar is one bf16 ulp: the allowance is a small fraction of it.
    assert np.median(al / tolerance.ulp(ref, "bf16")) < 0.125


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_dx_allowance_gelu_covers_an_approximate_derivative(approximate):
    """With the GELU epilogue the allowance also covers GELU' evaluated within 2.1e-7 (the
    tables' bound): an fp32 evaluation that perturbs GELU' by +-2.1e-7 stays inside."""
    from oracle import tolerance
    rng = np.random.RandomState(4096 + len(approximate))
    rows, cols = 32, 4096
    to_bf16 = norms.round_to_bf16
    x = to_bf16(rng.standard_normal((rows, cols)))
    dy = to_bf16(rng.standard_normal((rows, cols)))
    g = to_bf16(1 + 0.1 * rng.standard_normal(cols))
    b = to_bf16(0.2 * rng.standard_normal(cols))
    ref, _, _ = norms.layer_norm_gelu_bwd(dy, x, g, b, 1e-5, approximate)
    a, _, _ = norms.layer_norm_fwd(x, g, b, 1e-5)
    d = norms.gelu_grad(a, approximate) + 2.1e-7 * np.sign(rng.standard_normal(a.shape))
    got = _fp32_dx(x, (dy * d).astype(np.float32), g, 1e-5, False)
    al = tolerance.dx_allowance(x, dy, g, 1e-5, beta=b, approximate=approximate)
    assert (np.abs(got - ref) <= tolerance.ulp(ref, "bf16") + al).all()
    # Rows with ill-conditioned statistics (fp32 pairs with small spreads around large means):
    # GELU' taken at the GELU input of an fp32 forward, whose xhat carries the fp32 mean's
    # centring error, amplified by rstd in dx.  Without the allowance's GELU'' term this fails.
    m = rng.uniform(-3, 3, (512, 1))
    dd = 10.0 ** rng.uniform(-4, -1, (512, 1))
    x2 = np.concatenate([m + dd, m - dd], axis=1).astype(np.float32)
    dy2 = rng.standard_normal((512, 2)).astype(np.float32)
    g2 = (1 + 0.1 * rng.standard_normal(2)).astype(np.float32)
    b2 = (0.2 * rng.standard_normal(2)).astype(np.float32)
    ref2, _, _ = norms.layer_norm_gelu_bwd(dy2, x2, g2, b2, 1e-5, approximate)
    a32 = _fp32_y(x2, g2, b2, 1e-5)
    got2 = _fp32_dx(x2, (dy2 * norms.gelu_grad(a32, approximate)).astype(np.float32), g2, 1e-5,
                    False, out="f32")
    al2 = tolerance.dx_allowance(x2, dy2, g2, 1e-5, beta=b2, approximate=approximate)
    assert (np.abs(got2 - ref2) <= tolerance.ulp(ref2, "f32") + al2).all()


# ------------------------------------------------------------------------------------------------
# The forward error model (oracle.tolerance.y_allowance) used by the GPU parity bar for y.
# ------------------------------------------------------------------------------------------------
def _fp32_y(x, gamma, beta, eps, order="pairwise", round_mean=False, approximate=None):
    """An fp32 two-pass LayerNorm (+ GELU) evaluation, y in fp32: row sums pairwise (numpy) or
    as running sums of 64 elements per lane then a tree (the kernels' shape); optionally the
    mean rounded to bf16 (a planted loss of precision)."""
    f = np.float32
    x32, g32, b32 = x.astype(f), gamma.astype(f), beta.astype(f)
    n = x.shape[-1]

    def rowsum(a):
        if order == "pairwise" or a.shape[1] % 64:
            return a.sum(axis=1, keepdims=True, dtype=f)
        part = np.cumsum(a.reshape(a.shape[0], -1, 64), axis=2, dtype=f)[:, :, -1]
        return part.sum(axis=1, keepdims=True, dtype=f)

    mu = (rowsum(x32) / f(n)).astype(f)
    if round_mean:
        mu = norms.round_to_bf16(mu).astype(f)
    rs = (f(1) / np.sqrt(rowsum((x32 - mu) ** 2) / f(n) + f(eps))).astype(f)
    a = (((x32 - mu) * rs).astype(f) * g32 + b32).astype(f)
    if approximate is None:
        return a.astype(np.float64)
    return torch.nn.functional.gelu(torch.from_numpy(a), approximate=approximate).double().numpy()


def _y_cases():
    """Rows where y cancels or the statistics are ill-conditioned: bf16 h = x + r with an offset
    mean at 416 and 22784 columns (the widths where an extended GPU sweep met the old bar's
    limit), fp32 pairs and f16 triples with small spreads around large means."""
    rng = np.random.RandomState(17)
    to_bf16, to_f16 = norms.round_to_bf16, norms.round_to_f16
    out = []
    for rows, cols in ((512, 416), (8, 22784)):
        h = to_bf16(to_bf16(rng.standard_normal((rows, cols)) * 1.5 + 0.25) +
                    to_bf16(rng.standard_normal((rows, cols))))
        out.append(("bf16 h", h, to_bf16(1 + 0.1 * rng.standard_normal(cols)),
                    to_bf16(0.1 * rng.standard_normal(cols))))
    m = rng.uniform(-3, 3, (512, 1))
    d = 10.0 ** rng.uniform(-4, -1, (512, 1))
    out.append(("f32 pairs", np.concatenate([m + d, m - d], axis=1).astype(np.float32),
                (1 + 0.1 * rng.standard_normal(2)).astype(np.float32),
                (0.1 * rng.standard_normal(2)).astype(np.float32)))
    x3 = to_f16(rng.uniform(-3, 3, (512, 1)) + 1e-3 * rng.standard_normal((512, 3)))
    out.append(("f16 triples", x3, to_f16(1 + 0.1 * rng.standard_normal(3)),
                to_f16(0.1 * rng.standard_normal(3))))
    return out


@pytest.mark.parametrize("approximate", [None, "none", "tanh"], ids=["ln", "gelu-erf", "gelu-tanh"])
def test_y_allowance_covers_fp32_evaluations_and_rejects_a_bf16_mean(approximate):
    """The forward bar (1 ulp + oracle.tolerance.y_allowance) holds for fp32 two-pass
    evaluations -- numpy with pairwise or per-lane-then-tree row sums, and torch's own fp32
    F.layer_norm on the CPU -- on rows where y cancels and rows with ill-conditioned statistics
    (fp32 pairs, f16 triples with small spreads); and it rejects the evaluation whose mean is
    rounded to bf16."""
    from oracle import tolerance
    for what, x, g, b in _y_cases():
        eps = 1e-5
        ref = norms.layer_norm_fwd(x, g, b, eps)[0]
        if approximate is not None:
            ref = norms.gelu(ref, approximate)
        al = tolerance.y_allowance(x, g, b, eps, approximate=approximate)
        bound = tolerance.ulp(ref, "f32") + al
        for order in ("pairwise", "lanes"):
            got = _fp32_y(x, g, b, eps, order=order, approximate=approximate)
            assert (np.abs(got - ref) <= bound).all(), (what, order)
        t = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float32)),
                                           (x.shape[-1],), torch.from_numpy(g.astype(np.float32)),
                                           torch.from_numpy(b.astype(np.float32)), eps)
        if approximate is not None:
            t = torch.nn.functional.gelu(t, approximate=approximate)
        assert (np.abs(t.double().numpy() - ref) <= bound).all(), (what, "torch")
        planted = _fp32_y(x, g, b, eps, round_mean=True, approximate=approximate)
        assert (np.abs(planted - ref) > bound).any(), (what, "bf16 mean")
    # Away from cancellation the allowance is a small fraction of a bf16 ulp.
    x, g, b = _y_cases()[0][1:]
    ref = norms.layer_norm_fwd(x, g, b, 1e-5)[0]
    al = tolerance.y_allowance(x, g, b, 1e-5)
    assert np.median(al / tolerance.ulp(ref, "bf16")) < 0.01
