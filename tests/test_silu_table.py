"""The SwiGLU epilogue's silu rule against the oracle on every bf16 value.

The kernel reads one table entry per gate value g: the window entry of its bf16
pattern for 2^-9 <= |g| <= 126.5, else its sign's below- or above-window entry.
An entry carries T (high half) and a factor M (low half), both bf16, and the
kernel returns bf16(fma(g, M, T)): T inside the window, bf16(g / 2) below it,
g above it for g > 0 and g * 0 for g < 0 (-0, or NaN for -inf).  This restates
that rule in numpy with the table vflash_amd/build.py generates and compares
it, bit for bit, with the oracle's correctly rounded binary32 steps
(oracle/fp8.py silu).
"""

import numpy as np

from oracle import fp8 as O
from oracle.formats import bf16_from_bits
from vflash_amd import build


def kernel_rule(bits: np.ndarray, table: np.ndarray) -> np.ndarray:
    g = bf16_from_bits(bits.astype(np.uint16))
    a = (bits & 0x7FFF).astype(np.int64)
    c = np.clip(a, build.SILU_LO - 1, build.SILU_LO + build.SILU_N)
    idx = (c - (build.SILU_LO - 1)) + np.where(bits & 0x8000, build.SILU_STRIDE, 0)
    e = table[idx]
    t = (e & 0xFFFF0000).astype(np.uint32).view(np.float32).astype(np.float64)
    m = ((e << 16) & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(np.float64)
    # g * m and the sum are exact in binary64 (bf16 operands, m in {0, 1/2, 1}),
    # so one rounding to binary32 is the fma's.
    with np.errstate(invalid="ignore"):
        r = (g.astype(np.float64) * m + t).astype(np.float32)
    return O.bf16_round(r)


def test_window_table_and_rule_equal_the_oracle_on_every_bf16_value():
    bits = np.arange(65536, dtype=np.uint32)
    table = np.array(build.silu_window_table(), dtype=np.uint32)
    got = kernel_rule(bits, table)
    want = O.silu(bf16_from_bits(bits.astype(np.uint16)))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert table.size == 2 * build.SILU_STRIDE
    # Window entries carry no factor; the edges carry no value but a signed zero.
    for s in (0, 1):
        part = table[s * build.SILU_STRIDE:(s + 1) * build.SILU_STRIDE]
        assert np.all((part[1:-1] & 0xFFFF) == 0)
        assert np.all((part[[0, -1]] >> 16) == s * 0x8000)


def test_first_patterns_past_the_window_follow_the_edge_rule():
    # The window stops at 126.5: 127 and -127 (the next patterns) already give
    # g and -0, as the above-window entries compute them.
    hi = build.SILU_LO + build.SILU_N - 1
    assert build.silu_bf16(hi + 1) == hi + 1
    assert build.silu_bf16(0x8000 | (hi + 1)) == 0x8000


def test_generator_spot_values():
    # silu(1) = 1 / (1 + e^-1) = 0.7310585786...; bf16 0.73046875 (0x3F3B).
    assert build.silu_bf16(0x3F80) == 0x3F3B
    # silu(-1) = -0.2689414214 -> bf16 -0.26953125 (0xBE8A).
    assert build.silu_bf16(0xBF80) == 0xBE8A
    assert build.silu_bf16(0x0000) == 0x0000 and build.silu_bf16(0x8000) == 0x8000
    assert build.silu_bf16(0x7F80) == 0x7F80  # +inf
    assert build.silu_bf16(0xFF80) == 0x7FC0  # -inf -> NaN
    assert build.silu_bf16(0xC2C8) == 0x8000  # -100: exp(100) overflows binary32
