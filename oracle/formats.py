"""Number formats of the path, restated from their specifications (test infrastructure).

* bfloat16: the upper 16 bits of IEEE binary32; round to nearest, ties to even.
* E4M3 ("fn", OCP 8-bit FP spec): bias 7, 3 mantissa bits, subnormal step 2^-9,
  max 448, no infinities, S.1111.111 is NaN.  Used by torch.float8_e4m3fn and by
  the reference's ``.to(torch.float8_e4m3fn)`` / ``tl.float8e4nv`` casts
  (src/vflash/native/h3_fp8_linear.py:30, h3_fp8_activation.py:27).
* E2M1 (OCP MX spec): bias 1, 1 mantissa bit, values 0, .5, 1, 1.5, 2, 3, 4, 6.

Rounding is implemented once, exactly in binary64 (``round_to_grid``), and
pinned in tests/test_oracle_formats.py against torch's casts over every bf16
bit pattern, every tie and every code.
"""

from __future__ import annotations

import numpy as np

FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def round_to_grid(x, mant_bits: int, min_exp: int) -> np.ndarray:
    """Round finite values to a binary format with ``mant_bits`` stored mantissa
    bits and minimum normal exponent ``min_exp`` (no overflow handling):
    nearest representable value, ties to even.  Exact in binary64."""
    x = np.asarray(x, dtype=np.float64)
    _, e = np.frexp(x)  # x = m * 2^e with 0.5 <= |m| < 1, so floor(log2|x|) = e - 1
    exp = np.maximum(e - 1, min_exp)
    quantum = np.ldexp(1.0, exp - mant_bits)
    out = np.rint(x / quantum) * quantum  # np.rint rounds half to even
    return np.where(x == 0, x, out)


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even); returns binary32 values.
    NaN stays NaN; magnitudes beyond the bf16 range become +-inf."""
    x = np.asarray(x, dtype=np.float64)
    finite = np.isfinite(x)
    r = round_to_grid(np.where(finite, x, 0.0), 7, -126)
    bf16_max = (2.0 - 2.0**-7) * 2.0**127
    r = np.where(np.abs(r) > bf16_max, np.copysign(np.inf, x), r)
    return np.where(finite, r, x).astype(np.float32)


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of values that are already bf16-representable."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(x) -> np.ndarray:
    """binary32/64 values with |x| <= 448 (or NaN) -> E4M3 codes, RNE.

    The sign bit follows the input's sign (so -0.0 -> 0x80); NaN -> 0x7f | sign.
    """
    x = np.asarray(x, dtype=np.float64)
    nan = np.isnan(x)
    if np.any(np.abs(x[~nan]) > 448.0):
        raise ValueError("E4M3 encode expects values clamped to [-448, 448]")
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    a = np.abs(np.where(nan, 0.0, x))
    r = round_to_grid(a, 3, -6)
    _, e = np.frexp(r)
    e = e - 1
    sub = r < 2.0**-6
    m_sub = np.rint(r * 512.0)
    e_field = np.where(sub, 0, e + 7)
    m_norm = np.rint((np.where(r > 0, r / np.ldexp(1.0, e), 1.0) - 1.0) * 8.0)
    code = np.where(sub, m_sub, (e_field << 3) + m_norm).astype(np.uint8)
    code = np.where(nan, 0x7F, code).astype(np.uint8)
    return code | sign


def _e4m3_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        if (c & 0x7F) == 0x7F:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0**-9
        else:
            t[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_VALUES = _e4m3_table()


def e4m3_decode(codes) -> np.ndarray:
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


def e2m1_encode(x) -> np.ndarray:
    """Values within [-6, 6] -> E2M1 codes (RNE); the sign bit follows the sign of
    the input, -0 included (E2M1 has a negative zero, and a sign-preserving
    conversion keeps it)."""
    x = np.asarray(x, dtype=np.float64)
    if np.any(np.abs(x) > 6.0):
        raise ValueError("E2M1 encode expects values clamped to [-6, 6]")
    r = round_to_grid(np.abs(x), 1, 0)
    code = np.searchsorted(E2M1_MAGNITUDES.astype(np.float64), r).astype(np.uint8)
    return code | np.where(np.signbit(x), 8, 0).astype(np.uint8)


def e2m1_decode(codes) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8)
    v = E2M1_MAGNITUDES[c & 7]
    return np.where(c & 8, -v, v).astype(np.float32)
