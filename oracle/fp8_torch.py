"""The FP8 oracle's rounding chains restated in torch, so that outputs of the
full configuration shapes (hundreds of millions of elements) can be checked on
the device.

Test infrastructure: only tests/ imports this module.  Each function restates
the numpy function of oracle/fp8.py (or oracle/formats.py) named in its
docstring, with the same formula, the same rounding points and binary64 where
the numpy oracle uses binary64, and is pinned bit for bit against it on the CPU
by tests/test_oracle_fp8_torch.py.  The activation tables (GELU-tanh, silu) are
the numpy oracle itself, evaluated on every bf16 pattern and indexed here.
"""

from __future__ import annotations

from functools import cache

import numpy as np
import torch

from oracle import fp8 as O
from oracle.formats import bf16_from_bits

BF16_MAX = (2.0 - 2.0**-7) * 2.0**127
RNE_SHIFT = 1.5 * 2.0**52


def pow2(n: torch.Tensor) -> torch.Tensor:
    """2^n in binary64 for integer n in [-1022, 1023], from its bit pattern."""
    return ((n.to(torch.int64) + 1023) << 52).view(torch.float64)


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """formats.bf16_round: round to the nearest bfloat16, ties to even, directly
    from the input (binary64 arithmetic, no intermediate binary32 rounding);
    NaN stays NaN, magnitudes past the bf16 range become +-inf.  Returns float32."""
    x = x.double()
    finite = torch.isfinite(x)
    xf = torch.where(finite, x, torch.zeros_like(x))
    _, e = torch.frexp(xf)  # |x| = m 2^e, 0.5 <= m < 1: the binade of x is 2^(e-1)
    ulp = torch.clamp(e - 1, min=-126) - 7  # log2 of the bf16 spacing at x
    step = pow2(ulp)
    # x in units of the spacing, |q| < 2^9: a product with an exact power of two
    # (torch's binary64 division and ldexp on the GPU are not exact).
    q = xf * pow2(-ulp)
    # Nearest integer, ties to even, from two IEEE binary64 additions (the sum
    # with 1.5 * 2^52 has unit spacing), not torch.round.  copysign keeps the
    # sign of values that round to zero.
    r = torch.copysign(((q + RNE_SHIFT) - RNE_SHIFT) * step, xf)
    r = torch.where(r.abs() > BF16_MAX, torch.copysign(torch.full_like(r, float("inf")), xf), r)
    return torch.where(finite, r, x).float()


def e4m3_values(codes: torch.Tensor) -> torch.Tensor:
    """formats.e4m3_decode: E4M3 codes (uint8 or float8_e4m3fn) as binary64."""
    return codes.view(torch.float8_e4m3fn).to(torch.float64)


def quantize_rows(x: torch.Tensor, pad: int = 16):
    """fp8.quantize_rows (IEEE binary32 division form): binary32 row maximum;
    scale = max(amax / 448, FLT_MIN) if amax > 0 else 1; codes =
    e4m3(clamp(x / scale, -448, 448)) (torch's float8_e4m3fn cast, ties to even,
    the cast the numpy encoder is pinned to); rows padded to a multiple of
    ``pad`` with codes 0 and scale 1.  Returns (uint8 codes [m_pad, k],
    float32 scales [m_pad])."""
    x = x.float()
    m, k = x.shape
    m_pad = -(-m // pad) * pad
    amax = x.abs().amax(dim=1) if k else torch.zeros(m, device=x.device)
    divisor = torch.tensor(448.0, device=x.device)  # a tensor divisor: a true division
    base = torch.clamp(amax / divisor, min=torch.finfo(torch.float32).tiny)
    scale = torch.where(amax > 0, base, torch.ones_like(amax))
    q = torch.clamp(x / scale[:, None], -448.0, 448.0)
    codes = torch.zeros((m_pad, k), dtype=torch.uint8, device=x.device)
    codes[:m] = q.to(torch.float8_e4m3fn).view(torch.uint8)
    scales = torch.ones(m_pad, dtype=torch.float32, device=x.device)
    scales[:m] = scale
    return codes, scales


def scaled_mm(a_codes, sa, w_codes, sw) -> torch.Tensor:
    """fp8.scaled_mm: bf16(acc * sa[m] * sw[n]) with acc the binary64 sum of the
    decoded E4M3 products and the scale products formed in binary64."""
    acc = e4m3_values(a_codes) @ e4m3_values(w_codes).T
    sa = sa.double().reshape(-1, 1)[: acc.shape[0]]
    sw = sw.double().reshape(1, -1)
    return bf16_round(acc * sa * sw)


def add_bias(y: torch.Tensor, bias) -> torch.Tensor:
    """fp8.add_bias: bf16(y + bias) with the sum rounded to binary32 first."""
    if bias is None:
        return y.float()
    return bf16_round(y.float() + bias.float().reshape(1, -1))


def w8a8_linear(x, w_codes, sw, bias=None) -> torch.Tensor:
    """fp8.w8a8_linear for a 2-D input."""
    codes, sa = quantize_rows(x)
    m = x.shape[0]
    return add_bias(scaled_mm(codes[:m], sa[:m], w_codes, sw), bias)


@cache
def _table(name: str) -> np.ndarray:
    values = bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    return (O.gelu_tanh(values) if name == "gelu" else O.silu(values)).astype(np.float32)


def _lookup(name: str, y: torch.Tensor) -> torch.Tensor:
    table = torch.from_numpy(_table(name)).to(y.device)
    idx = y.to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
    return table[idx]


def gelu_tanh(y: torch.Tensor) -> torch.Tensor:
    """fp8.gelu_tanh of bf16 values (the numpy oracle on every bf16 pattern, indexed)."""
    return _lookup("gelu", y)


def silu_mul(packed: torch.Tensor) -> torch.Tensor:
    """fp8.silu_mul: value, gate = packed.chunk(2, -1); bf16(value * bf16(silu(gate)))."""
    f = packed.shape[-1] // 2
    value, gate = packed[..., :f], packed[..., f:]
    return bf16_round(value.double() * _lookup("silu", gate).double())


def gate_residual(residual, gate, y) -> torch.Tensor:
    """fp8.gate_residual: bf16(residual + bf16(gate * y)) in binary32."""
    gated = bf16_round(gate.float() * y.float())
    return bf16_round(residual.float() + gated)


def lora_delta(x, lora_a, lora_b, scaling: float = 1.0, strength: float = 1.0) -> torch.Tensor:
    """fp8.lora_delta: t = bf16(x A^T); d = bf16(t B^T) (binary64 sums);
    bf16(d * scaling) if scaling != 1 and bf16(d * strength) if strength != 1,
    each product formed in binary32."""
    t = bf16_round(x.double() @ lora_a.double().T)
    d = bf16_round(t.double() @ lora_b.double().T)
    for f in (scaling, strength):
        if f != 1.0:
            d = bf16_round(d * torch.tensor(f, dtype=torch.float32, device=d.device))
    return d


def lora_merge(base, delta) -> torch.Tensor:
    """fp8.lora_merge: bf16(base + delta), the sum formed in binary32."""
    return bf16_round(base.float() + delta.float())


def adapted(base, x, adapter, strength: float = 1.0) -> torch.Tensor:
    """fp8.adapted: bf16(base + lora_delta(x, down, up, scaling)); base when
    ``adapter`` (down, up, scaling) is None."""
    if adapter is None:
        return base.float()
    down, up, scaling = adapter
    return lora_merge(base, lora_delta(x, down, up, scaling, strength))
