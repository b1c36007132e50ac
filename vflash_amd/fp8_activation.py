"""Bounded per-row E4M3 activation quantization on gfx950.

Drop-in for ``quantize_activation`` of the reference
(src/vflash/native/h3_fp8_activation.py:31-55): same guards (2-D BF16 matrix,
unit column stride, 16 <= K <= 32768, supported device), same 16-row padding
and outputs (codes float8_e4m3fn [ceil16(M), K], scales fp32 [ceil16(M), 1]).
The kernel is ``vflash_quantize_rows_e4m3``: one wave per row, the row held in
VGPRs, wave-wide maximum, IEEE divisions and round-to-nearest-even E4M3.
"""

from __future__ import annotations

import torch

from vflash_amd import _lib, kernels


def quantize_activation(matrix):
    if (
        matrix.dtype != torch.bfloat16
        or matrix.ndim != 2
        or matrix.stride(1) != 1
        or not 16 <= matrix.shape[1] <= 32768
        or not _lib.is_gfx950(matrix.device)
    ):
        raise ValueError("row FP8 activation requires a bounded gfx950 BF16 matrix")
    return kernels.quantize_rows(matrix)
