"""On-disk formats (safetensors) of the quantized linears: reading and checks, on the CPU.

The files are written here with the key layouts of the reference's prepared
artifacts (src/vflash/native/h3_fp8_text.py:58-64,
src/vflash/adapters/h3_reference_assets.py:138-139,198-227,
src/vflash/adapters/h3_qad.py:104-129); no reference file is read.
"""

import pytest
import torch
from safetensors.torch import save_file

from vflash_amd import assets
from vflash_amd.fp8_linear import RowFP8Execution, RowFP8Linear
from vflash_amd.prepare import quantize_nvfp4_weight, quantize_weight_rows


def block_tensors(hidden=64, inner=32, ffn=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = {}
    for key, rows, cols in [
        ("attn.qkv.weight", 3 * inner, hidden),
        ("attn.out.weight", hidden, inner),
        ("ffn.in.weight", 2 * ffn, hidden),
        ("ffn.out.weight", hidden, ffn),
    ]:
        codes, scale = quantize_weight_rows(torch.randn((rows, cols), generator=g) * 0.02)
        t[key] = codes
        t[key + ".row_scale"] = scale
    for key in ("norm.attn.weight", "norm.ffn.weight"):
        t[key] = torch.rand(hidden, generator=g).to(torch.bfloat16)
    for key in ("attn.q_norm.weight", "attn.k_norm.weight"):
        t[key] = torch.rand(inner, generator=g).to(torch.bfloat16)
    return t


def test_block_artifact_round_trip(tmp_path):
    t = block_tensors()
    path = tmp_path / "block-000.safetensors"
    save_file(t, str(path))
    block = assets.load_fp8_block(path, device="cpu")
    assert block.hidden == 64 and block.inner == 32 and block.ffn_width == 128
    assert torch.equal(block.qkv.view(torch.uint8), t["attn.qkv.weight"].view(torch.uint8))
    assert torch.equal(block.ffn_out_scale, t["ffn.out.weight.row_scale"])
    # Q, K, V are the .chunk(3) split of the merged rows, scales with them.
    parts = block.qkv_parts()
    assert [p[0].shape for p in parts] == [(32, 64)] * 3
    assert torch.equal(parts[1][0].view(torch.uint8), t["attn.qkv.weight"][32:64].view(torch.uint8))
    assert torch.equal(parts[2][1], t["attn.qkv.weight.row_scale"][64:])
    assert set(block.norms) == {"norm1", "norm2", "norm_q", "norm_k"}
    assert assets.block_path("/r", 7).as_posix() == "/r/artifact/blocks/block-007.safetensors"


@pytest.mark.parametrize(
    "edit,match",
    [
        (lambda t: t.pop("ffn.out.weight.row_scale"), "misses"),
        (lambda t: t.__setitem__("attn.out.weight.row_scale", torch.ones(64, 2)), "fp32"),
        (lambda t: t.__setitem__("attn.qkv.weight", t["attn.qkv.weight"].float()), "E4M3"),
        (lambda t: t.pop("norm.ffn.weight"), "misses"),
        (lambda t: (t.__setitem__("ffn.in.weight", t["ffn.in.weight"][:255]),
                    t.__setitem__("ffn.in.weight.row_scale", t["ffn.in.weight.row_scale"][:255])),
         "packed"),
    ],
)
def test_block_artifact_refusals(tmp_path, edit, match):
    t = block_tensors()
    edit(t)
    path = tmp_path / "block.safetensors"
    save_file({k: v.contiguous() for k, v in t.items()}, str(path))
    with pytest.raises(ValueError, match=match):
        assets.load_fp8_block(path, device="cpu")


def test_row_fp8_state_assigns_into_the_module(tmp_path):
    # h3_fp8_text.py: <name>.weight.row_scale -> <name>.row_scale, then load_state_dict(assign=True).
    codes, scale = quantize_weight_rows(torch.randn(16, 8) * 0.02)
    path = tmp_path / "text.safetensors"
    save_file({"proj.weight": codes, "proj.weight.row_scale": scale}, str(path))
    state = assets.row_fp8_state(path)
    assert set(state) == {"proj.weight", "proj.row_scale"}
    holder = torch.nn.Module()
    holder.proj = RowFP8Linear(torch.nn.Linear(8, 16, bias=False), RowFP8Execution())
    holder.load_state_dict(state, strict=False, assign=True)
    x = torch.randn(3, 8)
    expect = torch.nn.functional.linear(x, codes.float() * scale)
    torch.testing.assert_close(holder.proj(x), expect, rtol=0, atol=0)


def test_row_scale_without_matrix_is_refused(tmp_path):
    path = tmp_path / "bad.safetensors"
    save_file({"proj.weight.row_scale": torch.ones(4, 1)}, str(path))
    with pytest.raises(ValueError, match="without its matrix"):
        assets.row_fp8_state(path)


def test_cached_matrix_contract():
    codes, scale = quantize_weight_rows(torch.randn(16, 8) * 0.02)
    original = torch.nn.Linear(8, 16, bias=False)
    m = assets.CachedMatrix(original, codes, scale, RowFP8Execution(), device="cpu")
    assert m.weight.dtype == torch.float8_e4m3fn and not m.weight.requires_grad and m.bias is None
    x = torch.randn(2, 8)
    torch.testing.assert_close(m(x), torch.nn.functional.linear(x, codes.float() * scale), rtol=0, atol=0)
    with pytest.raises(AssertionError):
        assets.CachedMatrix(torch.nn.Linear(8, 16), codes, scale, RowFP8Execution(), device="cpu")
    with pytest.raises(AssertionError):
        assets.CachedMatrix(original, codes, scale.T.contiguous(), RowFP8Execution(), device="cpu")


def qad_file(tmp_path, prefixes):
    g = torch.Generator().manual_seed(1)
    t = {}
    for prefix in prefixes:
        packed, scales, alpha, input_scale = quantize_nvfp4_weight(torch.randn(128, 64, generator=g) * 0.02)
        t[prefix + "::_nvfp4_weight"] = packed
        t[prefix + "::_nvfp4_weight_scale"] = scales
        t[prefix + "::_nvfp4_alpha"] = alpha
        t[prefix + "::_weight_global_sf"] = (1.0 / alpha).reshape(())
        if ".ff." in prefix:
            t[prefix + "::_nvfp4_input_global_sf"] = input_scale
    path = tmp_path / "qad.safetensors"
    save_file(t, str(path))
    return path, t


def test_nvfp4_qad_keys(tmp_path):
    prefixes = ["transformer_blocks.0.attn.to_q", "transformer_blocks.0.ff.net.0.proj"]
    path, t = qad_file(tmp_path, prefixes)
    assert assets.qad_prefixes(path) == sorted(prefixes)
    w = assets.load_nvfp4_qad(path, prefixes[1], device="cpu")
    assert w.in_features == 64 and w.out_features == 128
    assert torch.equal(w.packed, t[prefixes[1] + "::_nvfp4_weight"])
    assert torch.equal(w.input_scale, t[prefixes[1] + "::_nvfp4_input_global_sf"])
    # Non-feed-forward matrices carry no input scale: one is used.
    q = assets.load_nvfp4_qad(path, prefixes[0], device="cpu")
    assert float(q.input_scale) == 1.0
    with pytest.raises(ValueError, match="misses"):
        assets.load_nvfp4_qad(path, prefixes[0], feed_forward=True, device="cpu")
