"""Build libvflash_amd.so (gfx950) in-tree with hipcc.

Usage: ``python -m vflash_amd.build`` (or ``build()`` from Python).  Each
``csrc/*.hip`` file compiles to an object in parallel, then one shared library
is linked next to this file, where :mod:`vflash_amd._lib` loads it.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
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
