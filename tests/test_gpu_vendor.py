"""The drop-in linear against the reference's own arithmetic call on this GPU.

The reference's W8A8 GEMM is ``torch._scaled_mm(codes, weight.t(), scale_a,
scale_b=scale.t(), out_dtype=bf16)`` followed by ``output[:rows] + bias``
(src/vflash/native/h3_fp8_linear.py:109-121); on ROCm torch runs it on
hipBLASLt with row-wise scales.  The same codes and scales go through both;
the sums differ only in accumulation order, so the results must agree to the
GEMM tolerance, and all but a few ties per hundred thousand must be identical
(measured: 99.999-100 %).
"""

import numpy as np
import pytest
import torch

from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def reference_call(codes, act_scale, weight, scale, bias, rows):
    """h3_fp8_linear.py:109-121, verbatim in its arguments."""
    output = torch._scaled_mm(codes, weight.t(), scale_a=act_scale, scale_b=scale.t(),
                              out_dtype=torch.bfloat16, use_fast_accum=False)
    if isinstance(output, tuple):
        output = output[0]
    output = output[:rows]
    return output if bias is None else output + bias


def inputs(m, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    codes, scale = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    return x, codes, scale, b


@pytest.mark.parametrize("m,k,n", [(4096, 3072, 3072), (1000, 1536, 4608), (256, 1536, 1536)])
def test_linear_matches_the_reference_scaled_mm_call(dev, m, k, n):
    x, codes, scale, b = inputs(m, k, n, seed=m + n)
    xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    ours = ex.linear(xd, cd, sd, bd)
    a, sa = kernels.quantize_rows(xd)  # the padded codes/scales the reference passes
    ref = reference_call(a, sa, cd, sd, bd, m)
    worst, exact = rel_check(ours.float().cpu().numpy(), ref.float().cpu().numpy())
    print(f"[{m}x{k}x{n}] identical {exact:.5f}, worst relative difference {worst:.3g}")
    assert exact > 0.999, f"only {exact:.5f} of the elements are identical"
    # Without bias the comparison is of the scaled sums alone.
    ref_nb = reference_call(a, sa, cd, sd, None, m)
    _, exact = rel_check(ex.linear(xd, cd, sd).float().cpu().numpy(), ref_nb.float().cpu().numpy())
    assert exact > 0.999


def test_metric_shape_matches_the_reference_scaled_mm_call(dev):
    # M=32760, K=5120, N=13824, compared on the device over every element.
    m, k, n = 32760, 5120, 13824
    x, codes, scale, b = inputs(m, k, n, seed=0)
    xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
    del x
    ours = RowFP8Execution("w8a8", activation_quantizer="triton").linear(xd, cd, sd, bd)
    a, sa = kernels.quantize_rows(xd)
    ref = reference_call(a, sa, cd, sd, bd, m)
    o, r = ours.float(), ref.float()
    rms = float(torch.sqrt(torch.mean(r * r)))
    err = (o - r).abs()
    bound = 1e-2 * r.abs() + 1e-2 * rms
    assert int((err > bound).sum()) <= r.numel() // 10000
    assert not bool((err > 2.0**-6 * r.abs() + 1e-2 * rms).any())
    exact = float((o == r).float().mean())
    print(f"[{m}x{k}x{n}] identical {exact:.5f}, max |diff| / (|ref| + rms) "
          f"{float((err / (r.abs() + rms)).max()):.3g}")
    assert exact > 0.999, f"only {exact:.5f} of the elements are identical"
    assert bool(torch.isfinite(o).all())
    np.testing.assert_array_equal(ours.shape, (m, n))
