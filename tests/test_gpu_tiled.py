"""Row tiling never changes a result bit (the invariant of the reference's tiled_forward).

The reference runs every linear of a block on row tiles of 1024..65536 rows
(src/vflash/native/h3_tiled_block.py:10-126) and pins tiled == untiled
(tests/test_tiled_block.py:80-95).  Here every drop-in entry is run on the whole
token matrix, on 1024-row tiles plus a 17-row remainder, and on 16384-row tiles,
and the three results must be identical.  The widths are the configuration
widths (hidden 5120, merged QKV 15360, FFN 13824, adapter K 1536 / N 6144), so
the automatic GEMM tiling changes with the tile height: 256x256 on the whole
matrix and on 16384-row tiles, 128x192 for 1024-row tiles of the 5120- and
6144-wide projections, and 64x64 for the 17-row remainder.
"""

import pytest
import torch

from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import fp8_ffn, fp8_linear_lora, qkv_linear
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
from vflash_amd.prepare import quantize_nvfp4_weight, quantize_weight_rows

pytestmark = pytest.mark.gpu

ROWS = 32 * 1024 + 17
TILINGS = [1024, 16384]


def row_tiles(rows, height):
    return [(s, min(s + height, rows)) for s in range(0, rows, height)]


def tiled(fn, height, *row_args):
    """fn applied to row slices [s:e] of every argument, results concatenated."""
    outs = [fn(*(a[s:e] for a in row_args)) for s, e in row_tiles(ROWS, height)]
    if isinstance(outs[0], tuple):
        return tuple(torch.cat(parts) for parts in zip(*outs))
    return torch.cat(outs)


def assert_tiling_invariant(fn, *row_args):
    whole = fn(*row_args)
    for height in TILINGS:
        got = tiled(fn, height, *row_args)
        pairs = zip(whole, got) if isinstance(whole, tuple) else [(whole, got)]
        for w, g in pairs:
            assert torch.equal(w, g), f"{height}-row tiles differ from the whole matrix"


@pytest.fixture(scope="module")
def gen(dev):
    return lambda seed: torch.Generator(device=dev).manual_seed(seed)


def weight(dev, gen, n, k, seed):
    return quantize_weight_rows(torch.randn((n, k), generator=gen(seed), device=dev) * 0.02)


def bias(dev, gen, n, seed):
    return (torch.randn(n, generator=gen(seed), device=dev) * 0.01).to(torch.bfloat16)


def activations(dev, gen, k, seed=0):
    return torch.randn((ROWS, k), generator=gen(seed), device=dev).to(torch.bfloat16)


def test_w8a8_linear(dev, gen):
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    x = activations(dev, gen, 5120)
    for n in (13824, 5120):
        w, s = weight(dev, gen, n, 5120, 1)
        b = bias(dev, gen, n, 2)
        assert_tiling_invariant(lambda v: ex.linear(v, w, s, b), x)


def test_merged_qkv_planes(dev, gen):
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    x = activations(dev, gen, 5120)
    w, s = weight(dev, gen, 15360, 5120, 3)
    b = bias(dev, gen, 15360, 4)
    assert_tiling_invariant(lambda v: qkv_linear(ex, v, w, s, b, planes=True), x)


@pytest.mark.parametrize("activation", ["gelu_tanh", "swiglu"])
def test_ffn(dev, gen, activation):
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    h, f = 5120, 13824
    x = activations(dev, gen, h)
    residual = activations(dev, gen, h, seed=5)
    wu, su = weight(dev, gen, 2 * f if activation == "swiglu" else f, h, 6)
    bu = bias(dev, gen, wu.shape[0], 7)
    wd, sd = weight(dev, gen, h, f, 8)
    bd = bias(dev, gen, h, 9)
    gate = torch.rand(h, generator=gen(10), device=dev).to(torch.bfloat16)
    token_gate = torch.rand((ROWS, h), generator=gen(11), device=dev).to(torch.bfloat16)

    def ffn(v, res, g=gate):
        return fp8_ffn(ex, v, wu, su, bu, wd, sd, bd, g, res, activation=activation)

    assert_tiling_invariant(ffn, x, residual)
    assert_tiling_invariant(lambda v, res, g: ffn(v, res, g), x, residual, token_gate)


@pytest.mark.parametrize("rank", [16, 32, 128])
def test_lora_linear(dev, gen, rank):
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    k, n = 1536, 6144
    x = activations(dev, gen, k)
    w, s = weight(dev, gen, n, k, 12)
    b = bias(dev, gen, n, 13)
    a = (torch.randn((rank, k), generator=gen(14), device=dev) * 0.01).to(torch.bfloat16)
    bb = (torch.randn((n, rank), generator=gen(15), device=dev) * 0.01).to(torch.bfloat16)
    assert_tiling_invariant(
        lambda v: fp8_linear_lora(ex, v, w, s, b, a, bb, scaling=0.5, strength=1.375), x
    )


@pytest.mark.parametrize("activations_kind", ["nvfp4", "e4m3"])
def test_nvfp4(dev, gen, activations_kind):
    packed, scales, alpha, input_scale = quantize_nvfp4_weight(
        torch.randn((13824, 5120), generator=gen(16), device=dev) * 0.02, input_scale=0.5
    )
    wt = NVFP4Weight(packed, scales, alpha, input_scale)
    ex = NVFP4Execution(activations=activations_kind)
    x = activations(dev, gen, 5120)
    b = bias(dev, gen, 13824, 17)
    assert_tiling_invariant(lambda v: ex.linear(v, wt, b), x)
