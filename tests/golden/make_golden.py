"""Write the golden fixtures of tests/golden (run: python tests/golden/make_golden.py).

Inputs restate the reference's own test vectors where it has them; expected
values come from routines independent of the oracle: torch's CPU casts and
eager bf16 ops (the operations the reference itself executes), and exact
rational arithmetic for the GEMM.  Nothing here imports the reference.

Fixtures:
  e4m3_table.npz     all 256 E4M3 codes -> torch.float8_e4m3fn decode
  quant_kat.npz      tests/test_fp8_linear.py:99-120 rows (1, 16, 17 rows of
                     linspace(-448, 448, 64), a zero row, a bf16-tiny row)
                     with torch's codes/scales (_quantize_activation_torch
                     expression of h3_fp8_linear.py:18-31 on CPU torch)
  weight_only_kat.npz tests/test_fp8_linear.py:13-30 fixture (codes
                     arange(128) -> e4m3 [16, 8], scales linspace(.01, .1, 16))
  lora_kat.npz       tests/test_h3_reference_lora_pika.py:31-44 (rank-128
                     A = 0.30123, B = 0.001234, sample [[1, 2]], strengths)
  gemm_small.npz     a seeded 40x96x48 W8A8 case with bias; expected outputs
                     from exact Fraction sums, rounded once to bf16
"""

from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).float().numpy()


def torch_quantize(matrix: torch.Tensor):
    rows = matrix.shape[0]
    if rows % 16:
        matrix = torch.nn.functional.pad(matrix, (0, 0, 0, 16 - rows % 16))
    floats = matrix.float()
    maxima = floats.abs().amax(dim=1, keepdim=True)
    scale = torch.where(
        maxima > 0, (maxima / 448.0).clamp_min(torch.finfo(torch.float32).tiny), torch.ones_like(maxima)
    )
    codes = (floats / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return codes.view(torch.uint8).numpy(), scale.reshape(-1).numpy()


def e4m3_table():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn)
    np.savez(HERE / "e4m3_table.npz", codes=np.arange(256, dtype=np.uint8), values=codes.float().numpy())


def quant_kat():
    out = {}
    for rows in (1, 16, 17):
        values = torch.empty((rows, 64), dtype=torch.bfloat16)
        values.copy_(torch.linspace(-448, 448, 64))
        values[0].zero_()
        if rows > 1:
            values[1].fill_(torch.finfo(torch.bfloat16).tiny)
        codes, scales = torch_quantize(values)
        out[f"x{rows}"] = values.float().numpy()
        out[f"codes{rows}"] = codes
        out[f"scales{rows}"] = scales
    g = torch.Generator().manual_seed(0)
    x = (torch.randn((37, 200), generator=g) * torch.logspace(-30, 30, 37).unsqueeze(1)).to(torch.bfloat16)
    codes, scales = torch_quantize(x)
    out["xr"], out["codesr"], out["scalesr"] = x.float().numpy(), codes, scales
    np.savez(HERE / "quant_kat.npz", **out)


def weight_only_kat():
    codes = torch.arange(128).reshape(16, 8).to(torch.float8_e4m3fn)
    scales = torch.linspace(0.01, 0.1, 16).unsqueeze(1)
    g = torch.Generator().manual_seed(0)
    values = torch.randn((3, 8), generator=g).to(torch.bfloat16)
    bias = torch.randn(16, generator=g).to(torch.bfloat16)
    restored = (codes.float() * scales).to(torch.bfloat16)
    expected = torch.nn.functional.linear(values, restored, bias)
    np.savez(
        HERE / "weight_only_kat.npz",
        codes=codes.view(torch.uint8).numpy(),
        scales=scales.numpy(),
        values=values.float().numpy(),
        bias=bias.float().numpy(),
        expected=expected.float().numpy(),
    )


def lora_kat():
    sample = torch.tensor([[1, 2]], dtype=torch.bfloat16)
    a = torch.full((128, 2), 0.30123).to(torch.bfloat16)
    b = torch.full((2, 128), 0.001234).to(torch.bfloat16)
    base = sample  # the reference test's target layer is an identity Linear
    delta = torch.nn.functional.linear(torch.nn.functional.linear(sample, a), b)
    strengths = np.array([0.25, 1.0, 1.375], dtype=np.float32)
    expected = []
    for s in strengths:
        d = delta.to(sample.dtype)
        if s != 1.0:
            d = d * float(s)
        expected.append((base + d).float().numpy())
    np.savez(
        HERE / "lora_kat.npz",
        sample=sample.float().numpy(),
        a=a.float().numpy(),
        b=b.float().numpy(),
        strengths=strengths,
        expected=np.stack(expected),
    )


def exact_bf16(q: Fraction) -> float:
    """Round an exact rational to the nearest bf16 (ties to even)."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 7)
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * float(fl * quantum)


def gemm_small():
    g = torch.Generator().manual_seed(0)
    m, n, k = 40, 96, 48
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = torch.randn((n, k), generator=g) * 0.02
    bias = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    a_codes, sa = torch_quantize(x)
    wmax = w.abs().amax(dim=1, keepdim=True)
    sw = (wmax / 448.0).clamp_min(torch.finfo(torch.float32).tiny)
    w_codes = (w / sw).clamp(-448, 448).to(torch.float8_e4m3fn)
    a_val = torch.from_numpy(a_codes[:m]).view(torch.float8_e4m3fn).float().numpy()
    w_val = w_codes.float().numpy()
    sa_f = sa[:m]
    sw_f = sw.reshape(-1).numpy()
    bias_f = bias.float().numpy()
    scaled = np.empty((m, n), np.float32)
    for i in range(m):
        fa = [Fraction(float(v)) for v in a_val[i]]
        for j in range(n):
            acc = sum(fa[t] * Fraction(float(w_val[j, t])) for t in range(k))
            scaled[i, j] = exact_bf16(acc * Fraction(float(sa_f[i])) * Fraction(float(sw_f[j])))
    # Second rounding of the reference: eager bf16 add (binary32 then bf16).
    with_bias = (torch.from_numpy(scaled).to(torch.bfloat16) + bias).float().numpy()
    np.savez(
        HERE / "gemm_small.npz",
        x=x.float().numpy(),
        a_codes=a_codes,
        sa=sa,
        w_codes=w_codes.view(torch.uint8).numpy(),
        sw=sw_f,
        bias=bias_f,
        scaled=scaled,
        expected=with_bias,
    )


if __name__ == "__main__":
    e4m3_table()
    quant_kat()
    weight_only_kat()
    lora_kat()
    gemm_small()
    print("fixtures written to", HERE)
