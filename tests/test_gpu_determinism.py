"""Repeated calls give bit-identical results.

Every kernel of the path sums in a fixed order: no atomics and no cross-
workgroup reductions, so two calls on the same inputs (with other work in
between) must agree bit for bit at the full shapes.
"""

import pytest
import torch

from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import fp8_ffn
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
from vflash_amd.prepare import quantize_nvfp4_weight, quantize_weight_rows

pytestmark = pytest.mark.gpu


def test_w8a8_linear_and_ffn_repeat_bit_for_bit(dev):
    m, h, f = 32760, 5120, 13824
    g = torch.Generator().manual_seed(9)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16).to(dev)
    cu, su = quantize_weight_rows(torch.randn((f, h), generator=g) * 0.02)
    bu = (torch.randn(f, generator=g) * 0.01).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand(h, generator=g).to(torch.bfloat16)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su, bu, cd, sd, bd, gate, res = (t.to(dev) for t in (cu, su, bu, cd, sd, bd, gate, res))
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    first = ex.linear(x, cu, su, bu)
    ffn_first = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res)
    assert torch.equal(ex.linear(x, cu, su, bu), first)
    assert torch.equal(fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res), ffn_first)


@pytest.mark.parametrize("activations", ["nvfp4", "e4m3"])
def test_nvfp4_linear_repeats_bit_for_bit(dev, activations):
    m, k, n = 32760, 5120, 13824
    g = torch.Generator().manual_seed(10)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    packed, scales, alpha, _ = quantize_nvfp4_weight(torch.randn((n, k), generator=g) * 0.02)
    gsf = torch.tensor(2688.0 / float(x.float().abs().max()), dtype=torch.float32)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), gsf.to(dev))
    ex = NVFP4Execution(activations)
    first = ex.linear(x, weight)
    assert torch.equal(ex.linear(x, weight), first)
