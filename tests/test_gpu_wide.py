"""GEMM epilogues whose outputs span more than 2^31 bytes.

The reference chooses 64-bit addressing when a buffer's span passes 2^31
(native/h3_fused_ops.py:24-40, pinned by tests/test_wide_index.py:46-57).  Here
every row offset is 64-bit and the GEMMs rebase their buffer resources at each
tile's first row; these cases check the rows on both sides of the 2^31-byte
boundary and at the partial last tile against the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu

M, K, N = 70000, 128, 16384  # bf16 output 70000 x 16384 = 2.29e9 bytes
# Row 65536 starts at byte 65536 * 16384 * 2 = 2^31; 70000 = 273 * 256 + 112.
ROWS = np.r_[0:4, 65528:65544, 69984:70000]


@pytest.fixture(scope="module")
def wide(dev):
    assert 65536 * N * 2 == 2**31 and M * N * 2 > 2**31
    g = torch.Generator().manual_seed(31)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    codes, scale = quantize_weight_rows(torch.randn((N, K), generator=g) * 0.02)
    b = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    a, sa = kernels.quantize_rows(x.to(dev))
    lin = O.w8a8_linear(x.float().numpy()[ROWS], codes.view(torch.uint8).numpy(),
                        scale.reshape(-1).numpy(), b.float().numpy())
    return a, sa, codes.to(dev), scale.to(dev), b.to(dev), lin


def test_linear_output_beyond_two_gib(dev, wide):
    a, sa, c, s, b, lin = wide
    out = kernels.fp8_gemm(a, sa, c, s, M, b)
    rel_check(out[torch.from_numpy(ROWS).to(dev)].float().cpu().numpy(), lin)
    del out


def test_gate_residual_beyond_two_gib(dev, wide):
    a, sa, c, s, b, lin = wide
    g = torch.Generator(device=dev).manual_seed(5)
    res = torch.randn((M, N), generator=g, device=dev, dtype=torch.bfloat16)
    gate = torch.rand(N, generator=g, device=dev).to(torch.bfloat16)
    out = kernels.fp8_gemm_gate_residual(a, sa, c, s, M, gate, res, b)
    idx = torch.from_numpy(ROWS).to(dev)
    ref = O.gate_residual(res[idx].float().cpu().numpy(), gate.float().cpu().numpy(), lin)
    rel_check(out[idx].float().cpu().numpy(), ref)
    del out, res


def test_gelu_quantization_beyond_two_gib(dev, wide):
    # The up-projection output [70000, 16384] (2.29 GB) through the GELU
    # quantizer: g and the codes of rows on both sides of byte 2^31, against the
    # oracle on the kernel's own input rows.
    a, sa, c, s, b, lin = wide
    y = kernels.fp8_gemm(a, sa, c, s, M, b)
    codes, scales, g = kernels.gelu_quantize_rows(y, keep_values=True)
    idx = torch.from_numpy(ROWS).to(dev)
    y_rows = y[idx].float().cpu().numpy()
    g_rows = g[idx].float().cpu().numpy()
    assert np.array_equal(g_rows.view(np.uint32), O.gelu_tanh(y_rows).view(np.uint32))
    ref_codes, ref_scales = O.quantize_rows(g_rows, pad=1)
    assert np.array_equal(codes[idx].view(torch.uint8).cpu().numpy(), ref_codes)
    assert np.array_equal(scales[idx].reshape(-1).cpu().numpy().view(np.uint32),
                          ref_scales.view(np.uint32))
    del y, g, codes, scales


def test_swiglu_output_beyond_two_gib(dev):
    # Packed [2F, K] projection with F = 16384: h is [70000, 16384] bf16.
    g = torch.Generator().manual_seed(37)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(torch.randn((2 * N, K), generator=g) * 0.02)
    bu = (torch.randn(2 * N, generator=g) * 0.01).to(torch.bfloat16)
    a, sa = kernels.quantize_rows(x.to(dev))
    hh, amax = kernels.fp8_gemm_swiglu(a, sa, cu.to(dev), su.to(dev), M, bu.to(dev))
    idx = torch.from_numpy(ROWS).to(dev)
    h_rows = hh[idx].float().cpu().numpy()
    lin = O.w8a8_linear(x.float().numpy()[ROWS], cu.view(torch.uint8).numpy(),
                        su.reshape(-1).numpy(), bu.float().numpy())
    rel_check(h_rows, O.silu_mul(lin))
    assert np.array_equal(amax[idx].cpu().numpy(), np.abs(h_rows).reshape(len(ROWS), -1, 128).max(axis=2))
    del hh, amax


@pytest.mark.parametrize("activations", ["e4m3", "nvfp4"])
def test_nvfp4_output_beyond_two_gib(dev, activations):
    from oracle import nvfp4 as NV
    from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
    from vflash_amd.prepare import quantize_nvfp4_weight

    g = torch.Generator().manual_seed(41)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    packed, scales, alpha, ins = quantize_nvfp4_weight(torch.randn((N, K), generator=g) * 0.02)
    b = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
    out = NVFP4Execution(activations).linear(x.to(dev), weight, b.to(dev))
    got = out[torch.from_numpy(ROWS).to(dev)].float().cpu().numpy()
    xs = x.float().numpy()[ROWS]
    if activations == "e4m3":
        codes, sa = O.quantize_rows(xs, pad=1)
        ref = NV.linear(codes, sa, packed.numpy(), scales.numpy(), alpha.item(), b.float().numpy())
    else:
        a, a_scales = NV.quantize_activation(xs, float(ins))
        out_scale = np.float32(float(alpha)) / np.float32(float(ins))
        ref = NV.linear_w4a4(a, a_scales, packed.numpy(), scales.numpy(), out_scale, b.float().numpy())
    rel_check(got, ref)
    del out
