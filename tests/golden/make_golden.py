"""Writes tests/golden/norm_cases.npz: small input/output vectors of every operator on the path,
computed by PyTorch on the CPU in float64 (F.layer_norm, F.rms_norm, F.gelu, autograd, the
float8_e4m3fn cast) -- an implementation independent of this repository's oracle and kernels.

The reference repository ships no golden vectors (its tests compare live against PyTorch on a
GPU), so PyTorch's CPU path, which the reference's module defers to, is the source here.
Run from the repository root:  python tests/golden/make_golden.py
Arrays only (numpy.load(..., allow_pickle=False) reads them).  Outputs are stored as float32
(their rounding, ~6e-8 relative, is far inside every tolerance that uses them).
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "norm_cases.npz")


def gen(seed):
    return torch.Generator().manual_seed(seed)


def bf16_bits(t):
    """bf16 tensor -> its raw uint16 bit patterns (decode: (bits << 16) viewed as float32)."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def randn(shape, seed, scale=1.0, shift=0.0):
    return torch.randn(shape, generator=gen(seed), dtype=torch.float32) * scale + shift


def main():
    torch.set_num_threads(1)
    out = {}

    # LayerNorm forward (+ mean, rstd), fp32 inputs; affine and identity.
    for i, (rows, cols, shift) in enumerate([(3, 5, 0.0), (7, 768, 2.0), (4, 1023, -30.0),
                                             (2, 4096, 0.5)]):
        x = randn((rows, cols), 10 + i, 3.0, shift)
        g = randn((cols,), 20 + i, 0.1, 1.0)
        b = randn((cols,), 30 + i, 0.1)
        xd = x.double()
        y = F.layer_norm(xd, (cols,), g.double(), b.double(), 1e-5)
        y0 = F.layer_norm(xd, (cols,), None, None, 1e-5)
        var, mean = torch.var_mean(xd, dim=-1, unbiased=False)
        k = f"ln{i}"
        out.update({f"{k}_x": x.numpy(), f"{k}_g": g.numpy(), f"{k}_b": b.numpy(),
                    f"{k}_y": y.numpy(), f"{k}_y_noaffine": y0.numpy(),
                    f"{k}_mean": mean.numpy(), f"{k}_rstd": (1 / torch.sqrt(var + 1e-5)).numpy()})

    # LayerNorm + GELU (erf and tanh), the C2 width.
    x = randn((9, 1023), 40)
    g = randn((1023,), 41, 0.1, 1.0)
    b = randn((1023,), 42, 0.1)
    ln = F.layer_norm(x.double(), (1023,), g.double(), b.double(), 1e-5)
    out.update({"gelu_x": x.numpy(), "gelu_g": g.numpy(), "gelu_b": b.numpy(),
                "gelu_y_erf": F.gelu(ln).numpy(),
                "gelu_y_tanh": F.gelu(ln, approximate="tanh").numpy()})

    # Backward of GELU(LayerNorm) through autograd (float64), both GELU forms.
    x = randn((6, 1024), 45, 1.5, 0.2)
    g = randn((1024,), 46, 0.1, 1.0)
    b = randn((1024,), 47, 0.2)
    dy = randn((6, 1024), 48)
    out.update({"gb_x": x.numpy(), "gb_g": g.numpy(), "gb_b": b.numpy(), "gb_dy": dy.numpy()})
    for mode in ("none", "tanh"):
        xd, gd, bd = (t.double().requires_grad_(True) for t in (x, g, b))
        F.gelu(F.layer_norm(xd, (1024,), gd, bd, 1e-5), approximate=mode).backward(dy.double())
        out.update({f"gb_{mode}_dx": xd.grad.numpy(), f"gb_{mode}_dg": gd.grad.numpy(),
                    f"gb_{mode}_db": bd.grad.numpy()})

    # RMSNorm forward.
    for i, (rows, cols) in enumerate([(5, 96), (3, 4096)]):
        x = randn((rows, cols), 50 + i, 2.0, 0.3)
        w = randn((cols,), 60 + i, 0.1, 1.0)
        y = F.rms_norm(x.double(), (cols,), w.double(), 1e-6)
        ms = x.double().pow(2).mean(-1)
        out.update({f"rms{i}_x": x.numpy(), f"rms{i}_w": w.numpy(), f"rms{i}_y": y.numpy(),
                    f"rms{i}_rstd": (1 / torch.sqrt(ms + 1e-6)).numpy()})

    # Backward through autograd (float64): LayerNorm and RMSNorm.
    for i, (rows, cols) in enumerate([(3, 5), (6, 768), (9, 1024)]):
        x = randn((rows, cols), 70 + i, 1.5, 0.2)
        g = randn((cols,), 80 + i, 0.1, 1.0)
        b = randn((cols,), 90 + i, 0.1)
        dy = randn((rows, cols), 100 + i)
        xd = x.double().requires_grad_(True)
        gd = g.double().requires_grad_(True)
        bd = b.double().requires_grad_(True)
        F.layer_norm(xd, (cols,), gd, bd, 1e-5).backward(dy.double())
        k = f"lnb{i}"
        out.update({f"{k}_x": x.numpy(), f"{k}_g": g.numpy(), f"{k}_b": b.numpy(),
                    f"{k}_dy": dy.numpy(), f"{k}_dx": xd.grad.numpy(),
                    f"{k}_dg": gd.grad.numpy(), f"{k}_db": bd.grad.numpy()})
        xr = x.double().requires_grad_(True)
        wr = g.double().requires_grad_(True)
        F.rms_norm(xr, (cols,), wr, 1e-6).backward(dy.double())
        out.update({f"rmsb{i}_dx": xr.grad.numpy(), f"rmsb{i}_dw": wr.grad.numpy()})

    # Residual add + LayerNorm in bf16: h = bf16(x + r) by torch's bf16 add, y = LN(h) in fp64.
    x = randn((8, 2048), 110).to(torch.bfloat16)
    r = randn((8, 2048), 111).to(torch.bfloat16)
    g = randn((2048,), 112, 0.02, 1.0).to(torch.bfloat16)
    b = randn((2048,), 113, 0.02).to(torch.bfloat16)
    h = x + r
    y = F.layer_norm(h.double(), (2048,), g.double(), b.double(), 1e-5)
    out.update({"res_x_bf16": bf16_bits(x), "res_r_bf16": bf16_bits(r),
                "res_g_bf16": bf16_bits(g), "res_b_bf16": bf16_bits(b),
                "res_h_bf16": bf16_bits(h), "res_y": y.numpy()})

    # LayerNorm -> fp8 e4m3fn with a per-row scale (outlier channels as in C5).
    x = randn((8, 7168), 120)
    idx = torch.randperm(7168, generator=gen(121))[:7]
    x[:, idx] *= 20.0
    xb = x.to(torch.bfloat16)
    g = randn((7168,), 122, 0.05, 1.0).to(torch.bfloat16)
    b = randn((7168,), 123, 0.05).to(torch.bfloat16)
    y = F.layer_norm(xb.double(), (7168,), g.double(), b.double(), 1e-5)
    amax = y.abs().amax(-1, keepdim=True)
    scale = amax / 448.0
    q = (y / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    out.update({"fp8_x_bf16": bf16_bits(xb), "fp8_g_bf16": bf16_bits(g),
                "fp8_b_bf16": bf16_bits(b), "fp8_q": q.numpy(),
                "fp8_scale": scale[:, 0].float().numpy()})

    # Residual add + RMSNorm -> fp8 (bf16 in, per-row scale), the pre-norm of an fp8 GEMM.
    x = randn((8, 4096), 140).to(torch.bfloat16)
    r = randn((8, 4096), 141).to(torch.bfloat16)
    w = randn((4096,), 142, 0.05, 1.0).to(torch.bfloat16)
    h = x + r
    y = F.rms_norm(h.double(), (4096,), w.double(), 1e-6)
    amax = y.abs().amax(-1, keepdim=True)
    q = (y / (amax / 448.0)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    out.update({"arf_x_bf16": bf16_bits(x), "arf_r_bf16": bf16_bits(r),
                "arf_w_bf16": bf16_bits(w), "arf_h_bf16": bf16_bits(h), "arf_q": q.numpy(),
                "arf_scale": (amax[:, 0] / 448.0).float().numpy()})

    # fp8 encoder: torch's cast of a value sweep (clamped to +-448 first: saturation).
    v = torch.cat([torch.tensor([0.0, -0.0, 448.0, -448.0, 449.0, 1e6, 2.0 ** -9, 2.0 ** -10,
                                 3 * 2.0 ** -10, 0.0625, 1.0625, 1.1875, 240.0, 232.0]),
                   randn((4096,), 130, 30.0), randn((1024,), 131, 0.01)]).double()
    codes = v.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    out.update({"enc_v": v.float().numpy(), "enc_q": codes.numpy()})

    out = {k: (v.astype(np.float32) if v.dtype == np.float64 else v) for k, v in out.items()}
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
