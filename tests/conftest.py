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
    """Parity of bf16 GEMM outputs against the oracle.

    Tolerance, per element with e the oracle value and rms the rms of e:
      * |a - e| <= rtol |e| + rtol rms        for all but 1 in 10^4 elements;
      * |a - e| <= 2^-6 |e| + rtol rms        for every element.
    The rms term covers outputs that cancel to near zero.  A bf16 output
    resolves only 2^-8 .. 2^-7 relative, and the reference's two roundings
    (bf16(acc * scales), then bf16(+ bias)) can turn a one-ulp difference of a
    larger pre-bias value into two ulps of the result (2^-6 relative); those
    rare cases are bounded by the second line.  Returns (max_rel, exact_frac).
    """
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape
    assert np.all(np.isfinite(a)), "non-finite kernel output"
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    err = np.abs(a - e)
    bound = rtol * np.abs(e) + rtol * rms
    bad = err > bound
    hard = err > 2.0**-6 * np.abs(e) + rtol * rms
    assert not hard.any(), (
        f"{int(hard.sum())} of {e.size} beyond two bf16 ulps: worst "
        f"{a.reshape(-1)[np.argmax(err - bound)]} vs {e.reshape(-1)[np.argmax(err - bound)]}"
    )
    assert bad.sum() <= e.size // 10000, (
        f"{int(bad.sum())} of {e.size} outside rtol={rtol}: worst "
        f"{a.reshape(-1)[np.argmax(err - bound)]} vs {e.reshape(-1)[np.argmax(err - bound)]}"
    )
    denom = np.maximum(np.abs(e), rms if rms > 0 else 1.0)
    return float(np.max(err / denom)) if e.size else 0.0, float(np.mean(a == e)) if e.size else 1.0




def rel_check_device(actual, expected, rtol=1e-2):
    """rel_check for device tensors of the full configuration shapes (the same two
    bounds, evaluated with torch in binary64 on the tensors' device).  Returns
    (max_rel, exact_frac)."""
    import torch

    a = actual.double()
    e = expected.double()
    assert a.shape == e.shape
    assert bool(torch.isfinite(a).all()), "non-finite kernel output"
    rms = float(torch.sqrt(torch.mean(e * e))) if e.numel() else 0.0
    err = (a - e).abs()
    bound = rtol * e.abs() + rtol * rms
    hard = int((err > 2.0**-6 * e.abs() + rtol * rms).sum())
    assert hard == 0, f"{hard} of {e.numel()} beyond two bf16 ulps"
    bad = int((err > bound).sum())
    assert bad <= e.numel() // 10000, f"{bad} of {e.numel()} outside rtol={rtol}"
    denom = torch.clamp(e.abs(), min=rms if rms > 0 else 1.0)
    return float((err / denom).max()), float((a == e).double().mean())
