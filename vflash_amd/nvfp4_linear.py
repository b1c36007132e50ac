"""NVFP4 block-scaled-weight linear on MI355X (drop-in for the reference module).

Mirrors ``NVFP4Weight`` / ``NVFP4Execution`` of the reference
(src/vflash/native/h3_nvfp4_linear.py:15-139): same packed-weight contract
(uint8 ``[N, K/2]`` E2M1 pairs, uint8 E4M3 block-16 scales ``[N, K/16]`` in the
128x4 tiled order, fp32 scalar ``alpha`` and ``input_scale``), same validation
messages, counters (``calls``, ``rows``), inference-only rule and bias rule.

Arithmetic (W4A8): activations are quantized per token to E4M3 by the same
kernel as the FP8 path (``input_scale`` is validated and carried but only the
W4A4 activation quantizer of the reference uses it); the GEMM multiplies E4M3
activations by E2M1 weights times their E4M3 block scale, accumulates in
binary32 and applies ``sa[m] * alpha`` in the epilogue, then the bias with a
second bf16 rounding (h3_nvfp4_linear.py:139).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from vflash_amd import _lib, kernels


@dataclass(frozen=True, eq=False)
class NVFP4Weight:
    packed: torch.Tensor
    scales: torch.Tensor
    alpha: torch.Tensor
    input_scale: torch.Tensor

    def __post_init__(self):
        if (
            self.packed.dtype != torch.uint8
            or self.packed.ndim != 2
            or min(self.packed.shape) < 1
            or self.packed.shape[0] % 128
            or self.packed.shape[1] % 32
            or self.scales.dtype != torch.uint8
            or self.scales.shape != (self.packed.shape[0], self.packed.shape[1] // 8)
            or not self.packed.is_contiguous()
            or not self.scales.is_contiguous()
        ):
            raise ValueError("NVFP4 requires declared packed codes and 128x4 block scales")
        for scalar in (self.alpha, self.input_scale):
            if scalar.dtype != torch.float32 or scalar.shape != torch.Size([]):
                raise ValueError("NVFP4 calibration and output alpha must be FP32 scalars")
            if scalar.device.type != "meta" and not bool(torch.isfinite(scalar) & (scalar > 0)):
                raise ValueError("NVFP4 scales must be positive and finite")
        if (
            len({v.device for v in (self.packed, self.scales, self.alpha, self.input_scale)})
            != 1
        ):
            raise ValueError("NVFP4 tensors must share one explicit device")

    @property
    def in_features(self):
        return self.packed.shape[1] * 2

    @property
    def out_features(self):
        return self.packed.shape[0]


def _require_device(device):
    if not _lib.is_gfx950(device):
        raise ValueError("This NVFP4 execution requires an explicit gfx950 (MI355X) device")


class NVFP4Execution:
    """W4A8 NVFP4-weight execution on gfx950; host counters remain diagnostic."""

    contract = "nvfp4-e2m1-block16-128x4-w4a8-gfx950-v1"

    def __init__(self):
        self.calls = 0
        self.rows = 0

    def linear(self, values, weight: NVFP4Weight, bias=None):
        if (
            values.ndim < 1
            or values.shape[-1] != weight.in_features
            or values.dtype not in (torch.bfloat16, torch.float16, torch.float32)
            or values.device != weight.packed.device
        ):
            raise ValueError("NVFP4 input differs from its frozen matrix")
        if torch.is_grad_enabled() and values.requires_grad:
            raise ValueError("NVFP4 execution is inference-only")
        _require_device(values.device)
        if bias is not None and (
            bias.shape != (weight.out_features,)
            or bias.device != values.device
            or bias.dtype != torch.bfloat16
        ):
            raise ValueError("NVFP4 bias must match its BF16 output")
        if values.dtype == torch.float16:
            raise ValueError("the W4A8 NVFP4 path quantizes BF16 (or FP32) activations")
        shape = values.shape
        matrix = values.to(torch.bfloat16) if values.dtype == torch.float32 else values
        matrix = matrix.reshape(-1, weight.in_features)
        if matrix.shape[0] == 0:
            raise ValueError("NVFP4 input rows must be nonempty")
        if matrix.stride(1) != 1:
            matrix = matrix.contiguous()
        codes, act_scale = kernels.quantize_rows(matrix)
        output = kernels.nvfp4_gemm(
            codes, act_scale, weight.packed, weight.scales, weight.alpha, matrix.shape[0], bias
        )
        self.calls += 1
        self.rows += matrix.shape[0]
        return output.reshape(*shape[:-1], weight.out_features)
