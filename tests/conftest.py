import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


def golden(name: str):
    return np.load(GOLDEN / name, allow_pickle=False)


@pytest.fixture(scope="session")
def dev():
    """cuda:0 on a gfx950 box; the HIP library must load (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from vflash_amd import _lib

    _lib.library()  # raises if the library is missing
    device = torch.device("cuda:0")
    if not _lib.is_gfx950(device):
        pytest.fail("GPU tests need a gfx950 device")
    return device


def rel_check(actual, expected, rtol=1e-2):
    """Relative parity of bf16 GEMM outputs.

    Elementwise |a - e| <= rtol * |e| + rtol * rms(e): the rms term covers
    outputs that cancel to near zero (a one-ulp bf16 difference of a large
    pre-bias value dominates such an element).  Returns (max_rel, exact_frac).
    """
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape
    assert np.all(np.isfinite(a)), "non-finite kernel output"
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    err = np.abs(a - e)
    bound = rtol * np.abs(e) + rtol * rms
    bad = err > bound
    assert not bad.any(), (
        f"{int(bad.sum())} of {e.size} outside rtol={rtol}: worst "
        f"{a.reshape(-1)[np.argmax(err - bound)]} vs {e.reshape(-1)[np.argmax(err - bound)]}"
    )
    denom = np.maximum(np.abs(e), rms if rms > 0 else 1.0)
    return float(np.max(err / denom)) if e.size else 0.0, float(np.mean(a == e)) if e.size else 1.0


os.environ.setdefault("PYTHONHASHSEED", "0")
