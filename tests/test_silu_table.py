"""The SwiGLU epilogue's silu rule against the oracle on every bf16 value.

The kernel looks bf16(silu(g)) up in a window table for 2^-9 <= |g| < 2^7 and
computes it elsewhere: bf16(g / 2) below the window, g above it for g > 0 and
g * 0 for g < 0 (-0, or NaN for -inf).  This restates that rule in numpy with
the table vflash_amd/build.py generates and compares it, bit for bit, with the
oracle's correctly rounded binary32 steps (oracle/fp8.py silu).
"""

import numpy as np

from oracle import fp8 as O
from oracle.formats import bf16_from_bits
from vflash_amd import build


def kernel_rule(bits: np.ndarray, table: np.ndarray) -> np.ndarray:
    g = bf16_from_bits(bits.astype(np.uint16))
    a = bits & 0x7FFF
    i = (a.astype(np.int64) - build.SILU_LO)
    inside = (i >= 0) & (i < build.SILU_N)
    idx = np.clip(i, 0, build.SILU_N - 1) + np.where(bits & 0x8000, build.SILU_N, 0)
    looked_up = table[idx].view(np.float32)
    with np.errstate(invalid="ignore"):
        small = O.bf16_round(g * np.float32(0.5))
        large = np.where(bits & 0x8000, g * np.float32(0.0), g).astype(np.float32)
    outside = np.where(a < build.SILU_LO, small, large)
    return np.where(inside, looked_up, outside).astype(np.float32)


def test_window_table_and_rule_equal_the_oracle_on_every_bf16_value():
    bits = np.arange(65536, dtype=np.uint32)
    table = np.array(build.silu_window_table(), dtype=np.uint32)
    got = kernel_rule(bits, table)
    want = O.silu(bf16_from_bits(bits.astype(np.uint16)))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # The window holds the only values the rule does not compute in closed form.
    assert table.size == 2 * build.SILU_N and np.all((table & 0xFFFF) == 0)


def test_generator_spot_values():
    # silu(1) = 1 / (1 + e^-1) = 0.7310585786...; bf16 0.73046875 (0x3F3B).
    assert build.silu_bf16(0x3F80) == 0x3F3B
    # silu(-1) = -0.2689414214 -> bf16 -0.26953125 (0xBE8A).
    assert build.silu_bf16(0xBF80) == 0xBE8A
    assert build.silu_bf16(0x0000) == 0x0000 and build.silu_bf16(0x8000) == 0x8000
    assert build.silu_bf16(0x7F80) == 0x7F80  # +inf
    assert build.silu_bf16(0xFF80) == 0x7FC0  # -inf -> NaN
    assert build.silu_bf16(0xC2C8) == 0x8000  # -100: exp(100) overflows binary32
