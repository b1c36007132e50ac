"""Producers of a linear's input fused with that linear's activation quantization.

The reference normalizes and modulates the block input in bf16
(src/vflash/native/h3_native_denoiser.py:535-540 and :565-566: ``_rms_norm``,
then ``_modulate`` or its fused form ``triton_strict_bf16_modulate``,
src/vflash/native/h3_fused_ops.py:52-122, 575-611), writes it to memory, and
the next W8A8 linear reads it back to quantize it per token
(src/vflash/native/h3_fp8_activation.py:12-55).  Here one HIP pass reads the
block input once and writes only the E4M3 codes and row scales the linear
consumes, as ``QuantizedRows``, which ``RowFP8Execution.linear``,
``fused.qkv_linear``, ``fused.fp8_ffn`` and ``fused.fp8_linear_lora`` accept in
place of the bf16 activation.
"""

from __future__ import annotations

import torch

from vflash_amd import kernels


class QuantizedRows:
    """Per-token E4M3 activations standing in for a bf16 ``[.., K]`` tensor.

    ``codes`` is ``[ceil16(M), K]`` E4M3 and ``scales`` ``[ceil16(M), 1]`` fp32
    (the layout of the activation quantizer), ``shape`` the logical shape of the
    bf16 activation.  ``values`` holds that bf16 activation when the producer
    was asked to keep it (a low-rank adapter on the same input needs it).
    ``shape``, ``ndim``, ``dtype`` and ``device`` describe the replaced
    activation, so the layout checks of the consuming linear apply unchanged.
    """

    __slots__ = ("codes", "scales", "shape", "values")

    def __init__(self, codes, scales, shape, values=None):
        self.codes = codes
        self.scales = scales
        self.shape = torch.Size(shape)
        self.values = values

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def dtype(self) -> torch.dtype:
        return torch.bfloat16

    @property
    def device(self) -> torch.device:
        return self.codes.device

    @property
    def rows(self) -> int:
        return self.shape.numel() // self.shape[-1] if self.shape[-1] else 0


def rmsnorm_modulate_quantize(
    value, norm_weight, scale, shift, *, eps: float, index=None, keep_values: bool = False
) -> QuantizedRows:
    """``_modulate(_rms_norm(value, norm_weight, eps), scale, shift)`` as E4M3 rows.

    ``value`` is bf16 ``[B, S, H]`` (contiguous).  Without ``index``, ``scale``
    and ``shift`` are ``[S, H]`` with unit hidden stride (any token stride, as
    the reference's fused modulation accepts).  With ``index`` (int64 ``[S]``,
    the reference's ``adaln_indices``), they are the ungathered rows
    ``table[:, j, :]`` of an adaLN table and token s uses row ``index[s]``; the
    gather ``index_select`` of h3_native_denoiser.py:527-532 is then done in
    place by the kernel.  An index outside the table gives NaN outputs for its
    tokens.  Rounding: bf16(x * rstd * w), then bf16(bf16(n * bf16(1 + scale)) +
    shift), then the per-token E4M3 quantization of the linear.
    """
    if not isinstance(value, torch.Tensor) or value.ndim != 3 or value.dtype != torch.bfloat16:
        raise ValueError("the fused norm/modulation requires a BF16 [B,S,H] activation")
    if not value.is_contiguous():
        raise ValueError("the fused norm/modulation requires a contiguous activation")
    _batch, tokens, hidden = value.shape
    if index is not None:
        if index.ndim != 1 or index.shape[0] != tokens:
            raise ValueError("modulation indices must be [S]")
        index = index.to(dtype=torch.int64).contiguous()
    elif scale.shape != (tokens, hidden) or shift.shape != (tokens, hidden):
        raise ValueError("scale and shift must be [S,H]")
    matrix = value.view(-1, hidden)
    codes, scales, values = kernels.rmsnorm_modulate_quantize(
        matrix, norm_weight, scale, shift, eps=eps, index=index, keep_values=keep_values
    )
    return QuantizedRows(codes, scales, value.shape,
                         values.view(value.shape) if values is not None else None)
