"""Empty activations (no tokens) through every drop-in entry.

The reference's modules accept a zero-row input: the quantizer pads 0 rows to
0, the GEMM returns ``[.., 0, N]`` and the counters still move
(h3_fp8_linear.py:18-31,67-121).  Here no kernel is launched with an empty
grid, and every output has the consuming layout's shape.
"""

import pytest
import torch

from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import fp8_ffn, fp8_linear_lora, merge_qkv, qkv_linear
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
from vflash_amd.prepare import quantize_nvfp4_weight, quantize_weight_rows

pytestmark = pytest.mark.gpu


def weights(n, k, seed, dev):
    g = torch.Generator().manual_seed(seed)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    return c.to(dev), s.to(dev), b.to(dev)


def test_empty_w8a8_linear(dev):
    c, s, b = weights(64, 128, 1, dev)
    for quantizer in ("triton", "torch"):
        ex = RowFP8Execution("w8a8", activation_quantizer=quantizer)
        out = ex.linear(torch.empty((0, 128), dtype=torch.bfloat16, device=dev), c, s, b)
        assert out.shape == (0, 64) and out.dtype == torch.bfloat16
        out = ex.linear(torch.empty((2, 0, 128), dtype=torch.bfloat16, device=dev), c, s, b)
        assert out.shape == (2, 0, 64)
        assert ex.calls == {"weight_only": 0, "w8a8": 2}
    codes, scales = kernels.quantize_rows(torch.empty((0, 128), dtype=torch.bfloat16, device=dev))
    assert codes.shape == (0, 128) and scales.shape == (0, 1)


def test_empty_merged_qkv(dev):
    parts = [weights(64, 128, i, dev) for i in range(3)]
    w, s = merge_qkv([p[0] for p in parts], [p[1] for p in parts])
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    x = torch.empty((0, 128), dtype=torch.bfloat16, device=dev)
    for planes in (False, True):
        q, k, v = qkv_linear(ex, x, w, s, planes=planes)
        assert q.shape == k.shape == v.shape == (0, 64)


@pytest.mark.parametrize("activation", ["gelu_tanh", "swiglu"])
def test_empty_ffn(dev, activation):
    h, f = 128, 256
    up_rows = 2 * f if activation == "swiglu" else f
    cu, su, bu = weights(up_rows, h, 2, dev)
    cd, sd, bd = weights(h, f, 3, dev)
    gate = torch.rand(h, device=dev).to(torch.bfloat16)
    x = torch.empty((0, h), dtype=torch.bfloat16, device=dev)
    res = torch.empty((0, h), dtype=torch.bfloat16, device=dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    out = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, activation=activation)
    assert out.shape == (0, h)


def test_empty_lora_linear(dev):
    c, s, b = weights(64, 128, 4, dev)
    la = torch.zeros((16, 128), dtype=torch.bfloat16, device=dev)
    lb = torch.zeros((64, 16), dtype=torch.bfloat16, device=dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    out = fp8_linear_lora(ex, torch.empty((0, 128), dtype=torch.bfloat16, device=dev), c, s, b, la, lb)
    assert out.shape == (0, 64)


@pytest.mark.parametrize("activations", ["nvfp4", "e4m3"])
def test_empty_nvfp4_linear_is_refused_as_in_the_reference(dev, activations):
    # h3_nvfp4_linear.py:100-101 refuses zero rows before quantizing.
    g = torch.Generator().manual_seed(5)
    packed, scales, alpha, _ = quantize_nvfp4_weight(torch.randn((128, 128), generator=g) * 0.02)
    weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev),
                         torch.tensor(100.0, device=dev))
    ex = NVFP4Execution(activations)
    with pytest.raises(ValueError, match="NVFP4 input rows must be nonempty"):
        ex.linear(torch.empty((0, 128), dtype=torch.bfloat16, device=dev), weight)


def test_empty_producer(dev):
    from vflash_amd.producers import rmsnorm_modulate_quantize

    h = 128
    x = torch.empty((1, 0, h), dtype=torch.bfloat16, device=dev)
    table = torch.zeros((4, 6, h), dtype=torch.bfloat16, device=dev)
    index = torch.empty((0,), dtype=torch.int64, device=dev)
    rows = rmsnorm_modulate_quantize(x, None, table[:, 1, :], table[:, 0, :], eps=1e-6, index=index,
                                     keep_values=True)
    assert rows.codes.shape[0] == 0 and rows.shape == (1, 0, h) and rows.values.shape == (1, 0, h)
    # The empty rows feed the consuming linear like an empty bf16 activation.
    c, s, b = weights(64, h, 6, dev)
    out = RowFP8Execution("w8a8", activation_quantizer="hip").linear(rows, c, s, b)
    assert out.shape == (1, 0, 64)
