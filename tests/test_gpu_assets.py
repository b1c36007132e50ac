"""Tensors read from the on-disk formats run through the kernels on gfx950, vs the oracle."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import fp8 as O
from tests.conftest import rel_check
from tests.test_assets_cpu import block_tensors, qad_file
from vflash_amd import assets
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import qkv_linear
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def test_block_artifact_through_the_kernels(dev, tmp_path):
    hidden, inner, ffn = 512, 256, 384
    t = block_tensors(hidden, inner, ffn, seed=4)
    path = tmp_path / "block-003.safetensors"
    save_file(t, str(path))
    block = assets.load_fp8_block(path, device=dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    g = torch.Generator().manual_seed(5)
    m = 200
    x = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
    # Merged QKV: one launch over the stored [3 * inner, hidden] rows, each plane
    # bit-identical to the linear of its .chunk(3) part.
    q, k, v = qkv_linear(ex, x.to(dev), block.qkv, block.qkv_scale, planes=True)
    for got, (w, s) in zip((q, k, v), block.qkv_parts()):
        assert torch.equal(got, ex.linear(x.to(dev), w, s))
    ref = O.w8a8_linear(x.float().numpy(), u8(block.qkv), block.qkv_scale.reshape(-1).cpu().numpy())
    rel_check(torch.cat((q, k, v), 1).float().cpu().numpy(), ref)
    # SwiGLU feed-forward built from the stored packed input and output projections.
    gate = (torch.rand((m, hidden), generator=g) * 0.5).to(torch.bfloat16)
    res = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
    out = assets.block_feed_forward(block, ex)(x.to(dev), gate.to(dev), res.to(dev))
    *_, chain = O.ffn(x.float().numpy(), u8(block.ffn_in), block.ffn_in_scale.reshape(-1).cpu().numpy(),
                      None, u8(block.ffn_out), block.ffn_out_scale.reshape(-1).cpu().numpy(), None,
                      gate.float().numpy(), res.float().numpy(), activation="swiglu")
    # A chain of two GEMMs: ulp-level differences upstream flip single E4M3 codes
    # of the requantized activations, so the chain is compared in the Frobenius norm.
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    assert np.linalg.norm(got - chain) / np.linalg.norm(chain) <= 1e-2


def test_qad_matrix_through_the_kernel(dev, tmp_path):
    prefix = "transformer_blocks.0.ff.net.2"
    path, t = qad_file(tmp_path, [prefix])
    loaded = assets.load_nvfp4_qad(path, prefix, device=dev)
    direct = NVFP4Weight(*(t[prefix + "::" + f].to(dev) for f in
                           ("_nvfp4_weight", "_nvfp4_weight_scale", "_nvfp4_alpha", "_nvfp4_input_global_sf")))
    x = torch.randn((64, loaded.in_features), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    ex = NVFP4Execution()
    assert torch.equal(ex.linear(x.to(dev), loaded), ex.linear(x.to(dev), direct))
