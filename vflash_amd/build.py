"""Build libvflash_amd.so (gfx950) in-tree with hipcc.

Usage: ``python -m vflash_amd.build`` (or ``build()`` from Python).  Each
``csrc/*.hip`` file compiles to an object in parallel, then one shared library
is linked next to this file, where :mod:`vflash_amd._lib` loads it.
"""

from __future__ import annotations

import math
import os
import struct
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from decimal import Decimal, localcontext
from fractions import Fraction
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBRARY = PACKAGE / "libvflash_amd.so"
OBJECTS = PACKAGE / "_objects"
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if not path.exists():
        raise RuntimeError(f"hipcc not found at {path}")
    return str(path)


# Packed binary32 VALU forms stay disabled: the compiler must not emit them.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


GENERATED = CSRC / "_gen"

# Constants of the tanh-approximated GELU as binary32 values, the ones a
# binary32 kernel (torch's gelu(approximate="tanh")) multiplies by.
GELU_BETA = struct.unpack("<f", struct.pack("<f", math.sqrt(2.0 / math.pi)))[0]
GELU_KAPPA = struct.unpack("<f", struct.pack("<f", 0.044715))[0]


def _bf16_bits_of_double(v: float) -> int:
    """A real value rounded to binary32, then to bfloat16 (both to nearest, ties to
    even): what a binary32 evaluation with correctly rounded steps stores."""
    if math.isnan(v):
        return 0x7FC0
    if math.isinf(v):
        return 0x7F80 if v > 0 else 0xFF80
    bits = struct.unpack("<I", struct.pack("<f", v))[0]
    if (bits & 0x7F800000) == 0x7F800000:  # rounded past the binary32 range
        return (bits >> 16) & 0xFF80
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) & 0xFFFF


def gelu_tanh_bf16(bits: int) -> int:
    """GELU-tanh of one bf16 value: x / (1 + exp(-2u)), u = beta (x + kappa x^3),
    in binary64 (the same function as 0.5 x (1 + tanh u), without its
    cancellation for negative x), stored as bf16 through binary32.
    +inf gives +inf; -inf gives NaN (0.5 x (1 + tanh u) is -inf * 0 there); a NaN
    input stays NaN with its sign and payload, quieted."""
    exponent, mantissa = (bits >> 7) & 0xFF, bits & 0x7F
    if exponent == 0xFF and mantissa:
        return bits | 0x0040
    x = struct.unpack("<f", struct.pack("<I", bits << 16))[0]
    if math.isinf(x):
        return 0x7F80 if x > 0 else 0x7FC0
    u = GELU_BETA * (x + GELU_KAPPA * x * x * x)
    t = -2.0 * u
    if t > 709.0:  # exp(t) overflows binary64: the quotient is a signed zero
        return 0x8000 if x < 0 else 0
    return _bf16_bits_of_double(x / (1.0 + math.exp(t)))


F32_MAX = Fraction(struct.unpack("<f", struct.pack("<I", 0x7F7FFFFF))[0])


def _f32_of_fraction(x: Fraction) -> float:
    """A rational rounded to binary32 (nearest, ties to even; past the largest
    finite value it rounds to infinity), as a Python float."""
    if x == 0:
        return 0.0
    sign = -1.0 if x < 0 else 1.0
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    ulp = Fraction(2) ** (max(e, -126) - 23)
    q = x / ulp
    whole = q.numerator // q.denominator
    rest = q - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2):
        whole += 1
    v = whole * ulp
    if v > F32_MAX:
        return sign * math.inf
    return sign * float(v)


def silu_bf16(bits: int) -> int:
    """bf16(silu(g)) of one bf16 value: the binary32 formula g / (1 + exp(-g)) of
    h3_fused_ops.py:205 with each step correctly rounded -- e = RN(exp(-g)),
    d = RN(1 + e), q = RN(g / d) -- then rounded to bf16.  exp(-g) is evaluated
    to 60 digits and rounded once; every other step is exact rational
    arithmetic rounded once.  Where exp(-g) overflows binary32 (g < -88.7) the
    quotient is -0; +inf gives +inf, -inf and NaN give NaN."""
    exponent, mantissa = (bits >> 7) & 0xFF, bits & 0x7F
    if exponent == 0xFF:
        if mantissa or bits & 0x8000:
            return (bits | 0x0040) if mantissa else 0x7FC0
        return bits
    g = struct.unpack("<f", struct.pack("<I", bits << 16))[0]
    if g == 0.0:
        return bits
    if -g > 89.0:
        return 0x8000  # exp(-g) overflows: g / inf
    if -g < -110.0:
        e = 0.0  # exp(-g) < 2^-150 rounds to zero
    else:
        with localcontext() as ctx:
            ctx.prec = 60
            e = _f32_of_fraction(Fraction(Decimal(-g).exp()))
        if math.isinf(e):
            return 0x8000
    d = _f32_of_fraction(1 + Fraction(e))
    return _bf16_bits_of_double(_f32_of_fraction(Fraction(g) / Fraction(d)))


# The silu window: bf16 magnitudes 2^-9 <= |g| <= 126.5 (bit patterns 0x3B00 ..
# 0x42FD without the sign), SILU_N per sign.  Outside it the function is
# bf16(g / 2) below, g above for g > 0 and g * 0 above for g < 0.  Each sign's
# table holds a below-window entry, the window, and an above-window entry
# (SILU_STRIDE entries); an entry is the bf16 pattern of silu(g) in its high
# half (T) and a bf16 factor M in its low half, so that every bf16 g gives
# bf16(fma(g, M, T)): M = 0 inside the window (T = bf16(silu(g))), M = 1/2
# below it, M = 1 (g > 0) or 0 (g < 0) above it, and T = +-0 with the sign of
# g outside it (tests/test_silu_table.py checks the whole rule against the
# oracle on every bf16 value).
SILU_LO = 0x3B00
SILU_N = 2046
SILU_STRIDE = SILU_N + 2


def silu_window_table() -> list[int]:
    """The lookup table, SILU_STRIDE entries per sign (positive g first): entry
    1 + i of a sign is the pattern SILU_LO + i, entry 0 the values below the
    window, entry SILU_STRIDE - 1 those above it."""
    out = []
    for sign in (0, 0x8000):
        below = (sign << 16) | 0x3F00  # T = +-0, M = 0.5
        above = (sign << 16) | (0x0000 if sign else 0x3F80)  # T = +-0, M = 0 or 1
        out.append(below)
        out.extend(silu_bf16(sign | (SILU_LO + i)) << 16 for i in range(SILU_N))
        out.append(above)
    return out


def write_silu_table() -> Path:
    """csrc/_gen/silu_table.h: the lookup table of the SwiGLU epilogue."""
    GENERATED.mkdir(exist_ok=True)
    path = GENERATED / "silu_table.h"
    table = silu_window_table()
    rows = ["    " + ", ".join(f"0x{v:08x}u" for v in table[i:i + 8]) + "," for i in range(0, len(table), 8)]
    text = (
        "// Generated by vflash_amd/build.py (write_silu_table); not edited by hand.\n"
        "// silu lookup entries: bf16(silu(g)) in the high half, a bf16 factor in the low\n"
        f"// half; entry 1 + i of a sign is the pattern 0x{SILU_LO:04X} + i (2^-9 <= |g| <= 126.5),\n"
        f"// entry 0 covers |g| below, entry {SILU_STRIDE - 1} above; the negative table starts at {SILU_STRIDE}.\n"
        "#pragma once\n#include <stdint.h>\n\nnamespace vfa {\n\n"
        f"constexpr uint32_t kSiluLo = 0x{SILU_LO:04X}u, kSiluN = {SILU_N}u, kSiluStride = {SILU_STRIDE}u;\n\n"
        f"__device__ const uint32_t kSiluTable[{2 * SILU_STRIDE}] __attribute__((aligned(16))) = {{\n"
        + "\n".join(rows)
        + "\n};\n\n}  // namespace vfa\n"
    )
    if not path.exists() or path.read_text() != text:
        path.write_text(text)
    return path


def write_activation_tables() -> Path:
    """csrc/_gen/activation_tables.h: the 65536-entry bf16 -> bf16 GELU-tanh table."""
    GENERATED.mkdir(exist_ok=True)
    path = GENERATED / "activation_tables.h"
    rows = []
    for base in range(0, 65536, 16):
        rows.append("    " + ", ".join(f"0x{gelu_tanh_bf16(b):04x}" for b in range(base, base + 16)) + ",")
    text = (
        "// Generated by vflash_amd/build.py (write_activation_tables); not edited by hand.\n"
        "// GELU-tanh of every bf16 bit pattern, as bf16 bit patterns.\n"
        "#pragma once\n#include <stdint.h>\n\nnamespace vfa {\n\n"
        "__device__ const uint16_t kGeluTanhTable[65536] __attribute__((aligned(16))) = {\n"
        + "\n".join(rows)
        + "\n};\n\n}  // namespace vfa\n"
    )
    if not path.exists() or path.read_text() != text:
        path.write_text(text)
    return path


def _compile(source: Path) -> Path:
    obj = OBJECTS / (source.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the C-ABI library."""
    OBJECTS.mkdir(exist_ok=True)
    write_activation_tables()
    write_silu_table()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources found")
    workers = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
