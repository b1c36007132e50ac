"""On-disk formats of the quantized linears (safetensors), loaded into this package's modules.

Formats (all written by the reference's preparation tools; this module only
reads them, with the safetensors loader, which executes nothing from a file):

* Row-FP8 matrices: ``<name>.weight`` F8_E4M3 ``[N, K]`` next to
  ``<name>.weight.row_scale`` F32 ``[N, 1]``.  The scale belongs to the
  replacement module as ``<name>.row_scale``
  (src/vflash/native/h3_fp8_text.py:58-64).
* H3 block artifacts ``block-NNN.safetensors``: ``attn.qkv.weight`` (the merged
  Q/K/V rows, ``[3 * inner, hidden]``), ``attn.out.weight``, ``ffn.in.weight``
  (packed value/gate rows ``[2F, hidden]``) and ``ffn.out.weight``, each with
  its ``.row_scale``, plus four bf16 norm weights
  (src/vflash/adapters/h3_reference_assets.py:138-139, 198-227).
* NVFP4 QAD matrices: ``<prefix>::_nvfp4_weight`` (u8 ``[N, K/2]``),
  ``::_nvfp4_weight_scale`` (u8, 128x4 order), ``::_nvfp4_alpha`` and
  ``::_weight_global_sf`` (F32 0-d), and for feed-forward matrices
  ``::_nvfp4_input_global_sf``; other matrices use an input scale of one
  (src/vflash/adapters/h3_qad.py:104-129).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch
from safetensors import safe_open

from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import FP8FeedForward
from vflash_amd.nvfp4_linear import NVFP4Weight

E4M3 = torch.float8_e4m3fn

# Keys of a block artifact: (module name in the loaded block, tensor key).
BLOCK_MATRICES = (
    ("qkv", "attn.qkv.weight"),
    ("attn_out", "attn.out.weight"),
    ("ffn_in", "ffn.in.weight"),
    ("ffn_out", "ffn.out.weight"),
)
BLOCK_NORMS = (
    ("norm1", "norm.attn.weight"),
    ("norm2", "norm.ffn.weight"),
    ("norm_q", "attn.q_norm.weight"),
    ("norm_k", "attn.k_norm.weight"),
)
NVFP4_FIELDS = ("_nvfp4_weight", "_nvfp4_weight_scale", "_nvfp4_alpha", "_weight_global_sf")


class CachedMatrix(torch.nn.Linear):
    """A prepared row-FP8 base matrix in place of a bias-free ``Linear``.

    Mirrors CachedMatrix (src/vflash/adapters/h3_reference_assets.py:17-31):
    same constructor, checks and forward.
    """

    def __init__(self, original, values, scales, execution, *, device="cuda:0"):
        torch.nn.Module.__init__(self)
        self.in_features, self.out_features = original.in_features, original.out_features
        if values.shape != original.weight.shape:
            raise AssertionError("prepared matrix differs from the target Linear")
        if values.dtype != E4M3:
            raise AssertionError("prepared matrix must hold E4M3 codes")
        if scales.dtype != torch.float32 or scales.shape != (self.out_features, 1):
            raise AssertionError("row scales must be fp32 [out_features, 1]")
        if original.bias is not None:
            raise AssertionError("prepared matrices replace bias-free linears only")
        self.weight = torch.nn.Parameter(values.to(device), requires_grad=False)
        self.register_buffer("row_scale", scales.to(device))
        self.bias = None
        self.execution = execution

    def forward(self, values):
        return self.execution.linear(values, self.weight, self.row_scale)


def row_fp8_state(path) -> dict[str, torch.Tensor]:
    """Read a row-FP8 safetensors file into module state names.

    ``<name>.weight.row_scale`` becomes ``<name>.row_scale`` (the buffer of
    RowFP8Linear / CachedMatrix); every other key keeps its name.  Each
    ``.weight`` that has a row scale must be E4M3 with an F32 ``[N, 1]`` scale.
    """
    out: dict[str, torch.Tensor] = {}
    with safe_open(str(path), framework="pt", device="cpu") as source:
        keys = list(source.keys())
        for name in keys:
            destination = (
                name.removesuffix(".weight.row_scale") + ".row_scale"
                if name.endswith(".weight.row_scale")
                else name
            )
            if destination in out:
                raise ValueError("duplicate row-FP8 tensor: " + destination)
            out[destination] = source.get_tensor(name)
    for name, scale in out.items():
        if not name.endswith(".row_scale"):
            continue
        weight = out.get(name.removesuffix(".row_scale") + ".weight")
        if weight is None:
            raise ValueError("row scale without its matrix: " + name)
        if weight.dtype != E4M3 or weight.ndim != 2:
            raise ValueError("row-FP8 matrix must be 2-D E4M3: " + name)
        if scale.dtype != torch.float32 or tuple(scale.shape) != (weight.shape[0], 1):
            raise ValueError("row scale must be fp32 [N, 1]: " + name)
    return out


@dataclass
class FP8BlockWeights:
    """Tensors of one H3 block artifact, checked and moved to one device."""

    qkv: torch.Tensor
    qkv_scale: torch.Tensor
    attn_out: torch.Tensor
    attn_out_scale: torch.Tensor
    ffn_in: torch.Tensor
    ffn_in_scale: torch.Tensor
    ffn_out: torch.Tensor
    ffn_out_scale: torch.Tensor
    norms: dict[str, torch.Tensor]

    @property
    def hidden(self) -> int:
        return int(self.qkv.shape[1])

    @property
    def inner(self) -> int:
        return int(self.qkv.shape[0]) // 3

    @property
    def ffn_width(self) -> int:
        return int(self.ffn_in.shape[0]) // 2

    def qkv_parts(self):
        """(values, scales) of Q, K and V: the .chunk(3) split of
        h3_reference_assets.py:205-209, as views of the merged tensors."""
        return tuple(zip(self.qkv.chunk(3), self.qkv_scale.chunk(3), strict=True))


def load_fp8_block(path, *, device="cuda:0") -> FP8BlockWeights:
    """Read ``block-NNN.safetensors`` (h3_reference_assets.py:198-227) with the
    geometry checks of its validator (:138-139): merged QKV rows divisible by
    three with a matching ``[rows, 1]`` scale, packed FFN input rows even."""
    state = row_fp8_state(path)
    tensors = {}
    for field, key in BLOCK_MATRICES:
        name = key.removesuffix(".weight")
        if key not in state or name + ".row_scale" not in state:
            raise ValueError("block artifact misses " + key)
        tensors[field] = state[key].to(device)
        tensors[field + "_scale"] = state[name + ".row_scale"].to(device)
    norms = {}
    for field, key in BLOCK_NORMS:
        if key not in state:
            raise ValueError("block artifact misses " + key)
        norms[field] = state[key].to(device)
    block = FP8BlockWeights(norms=norms, **tensors)
    hidden = block.hidden
    if block.qkv.shape[0] % 3:
        raise ValueError("merged QKV rows must divide into three projections")
    if block.attn_out.shape != (hidden, block.inner):
        raise ValueError("attention output projection does not match QKV")
    if block.ffn_in.shape[0] % 2 or block.ffn_in.shape[1] != hidden:
        raise ValueError("FFN input must be a packed [2F, hidden] value/gate matrix")
    if block.ffn_out.shape != (hidden, block.ffn_width):
        raise ValueError("FFN output projection does not match its input")
    return block


class _Projection(torch.nn.Module):
    """Holder with the RowFP8Linear layout (weight, row_scale, bias, execution)."""

    def __init__(self, weight, scale, execution):
        super().__init__()
        self.weight = torch.nn.Parameter(weight, requires_grad=False)
        self.register_buffer("row_scale", scale)
        self.bias = None
        self.execution = execution

    def forward(self, value):
        return self.execution.linear(value, self.weight, self.row_scale)


def block_feed_forward(block: FP8BlockWeights, execution: RowFP8Execution) -> FP8FeedForward:
    """The block's SwiGLU feed-forward (packed input, output projection) as one module."""
    return FP8FeedForward(
        _Projection(block.ffn_in, block.ffn_in_scale, execution),
        _Projection(block.ffn_out, block.ffn_out_scale, execution),
        activation="swiglu",
    )


def load_nvfp4_qad(path, prefix: str, *, feed_forward: bool | None = None, device="cuda:0"):
    """NVFP4Weight of one QAD matrix (h3_qad.py:104-129).

    ``feed_forward`` selects whether ``prefix::_nvfp4_input_global_sf`` must be
    present (the reference stores it for feed-forward matrices, whose prefix
    contains ``.ff.``); other matrices use an input scale of one.
    """
    if feed_forward is None:
        feed_forward = ".ff." in prefix
    with safe_open(str(path), framework="pt", device="cpu") as source:
        keys = set(source.keys())
        required = {prefix + "::" + field for field in NVFP4_FIELDS}
        if feed_forward:
            required.add(prefix + "::_nvfp4_input_global_sf")
        missing = required - keys
        if missing:
            raise ValueError("QAD matrix misses " + ", ".join(sorted(missing)))
        get = lambda field: source.get_tensor(prefix + "::" + field).to(device)  # noqa: E731
        input_scale = (
            get("_nvfp4_input_global_sf")
            if feed_forward
            else torch.ones((), dtype=torch.float32, device=device)
        )
        return NVFP4Weight(
            get("_nvfp4_weight"), get("_nvfp4_weight_scale"), get("_nvfp4_alpha"), input_scale
        )


def qad_prefixes(path) -> list[str]:
    """Matrix prefixes present in a QAD file (keys ``<prefix>::<field>``)."""
    with safe_open(str(path), framework="pt", device="cpu") as source:
        return sorted({k.split("::", 1)[0] for k in source.keys() if "::" in k})


def block_path(root, index: int) -> Path:
    """artifact/blocks/block-NNN.safetensors under a prepared root (h3_reference_assets.py:200)."""
    return Path(root) / "artifact" / "blocks" / f"block-{index:03d}.safetensors"
