"""NVFP4-weight (W4A8) linear on gfx950 against the oracle."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from oracle import nvfp4 as N
from tests.conftest import rel_check
from vflash_amd import _lib
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
from vflash_amd.prepare import quantize_nvfp4_weight

pytestmark = pytest.mark.gpu


def make(m, n, k, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = torch.randn((n, k), generator=g) * 0.02
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16) if bias else None
    return x, quantize_nvfp4_weight(w), b


def oracle(x, packed, scales, alpha, b, rows=None):
    xs = x.float().numpy() if rows is None else x.float().numpy()[rows]
    codes, sa = O.quantize_rows(xs, pad=1)
    return N.linear(codes, sa, packed.numpy(), scales.numpy(), alpha.item(),
                    None if b is None else b.float().numpy())


@pytest.fixture
def tile():
    yield
    _lib.set_gemm_tile(0)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
@pytest.mark.parametrize("m,n,k", [(1, 128, 64), (37, 256, 192), (300, 384, 512), (513, 640, 1088)])
def test_small_shapes_every_tile(dev, tile, cfg, m, n, k):
    _lib.set_gemm_tile(cfg)
    x, (packed, scales, alpha, ins), b = make(m, n, k, seed=m + n + k)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
    ex = NVFP4Execution()
    out = ex.linear(x.to(dev), weight, b.to(dev))
    rel_check(out.float().cpu().numpy(), oracle(x, packed, scales, alpha, b))
    out = ex.linear(x.to(dev), weight)
    rel_check(out.float().cpu().numpy(), oracle(x, packed, scales, alpha, None))
    assert ex.calls == 2 and ex.rows == 2 * m


def test_fp32_and_3d_inputs(dev):
    x, (packed, scales, alpha, ins), b = make(2 * 3 * 32, 128, 256)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
    out = NVFP4Execution().linear(x.float().reshape(2, 96, 256).to(dev), weight, b.to(dev))
    assert out.shape == (2, 96, 128) and out.dtype == torch.bfloat16
    rel_check(out.reshape(-1, 128).float().cpu().numpy(), oracle(x, packed, scales, alpha, b))


def test_config_shape_sampled_rows(dev):
    # X [32760, 5120] per-token e4m3; W e2m1 [13824, 5120] + e4m3 block-16 scales + fp32 global.
    x, (packed, scales, alpha, ins), _ = make(32760, 13824, 5120, bias=False)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
    out = NVFP4Execution().linear(x.to(dev), weight)
    rows = np.r_[0:8, 12000:12008, 32752:32760]
    rel_check(out.float().cpu().numpy()[rows], oracle(x, packed, scales, alpha, None, rows))
    assert bool(torch.isfinite(out.float()).all())
