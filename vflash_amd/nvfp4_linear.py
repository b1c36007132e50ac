"""NVFP4 linear on MI355X (drop-in for the reference module).

Mirrors ``NVFP4Weight`` / ``NVFP4Execution`` of the reference
(src/vflash/native/h3_nvfp4_linear.py:15-139): same packed-weight contract
(uint8 ``[N, K/2]`` E2M1 pairs, uint8 E4M3 block-16 scales ``[N, K/16]`` in the
128x4 tiled order, fp32 scalar ``alpha`` and ``input_scale``), same validation
messages, counters (``calls``, ``rows``), inference-only rule and bias rule.

Arithmetic (default, W4A4, the reference's): activations are quantized to
NVFP4 with the weight's ``input_scale`` as the global scale (the contract of
FlashInfer's ``nvfp4_quantize``, h3_nvfp4_linear.py:102), the GEMM multiplies
E2M1 activations and weights, each times its E4M3 block scale (exact in
binary16, binary32 accumulation), scales by ``alpha / input_scale`` and rounds
to bf16, and the bias is added with a second bf16 rounding
(h3_nvfp4_linear.py:114-139).

``NVFP4Execution(activations="e4m3")`` selects W4A8 instead: per-token E4M3
activations (the FP8 path's quantizer) times the same weights, ``sa[m] *
alpha`` in the epilogue; ``input_scale`` is then not used.  It is the more
accurate arithmetic, not the reference's.
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
    """NVFP4 execution on gfx950 (W4A4 by default); host counters remain diagnostic."""

    contract = "nvfp4-e2m1-block16-128x4-w4a4-gfx950-v1"

    def __init__(self, activations: str = "nvfp4"):
        if activations not in ("nvfp4", "e4m3"):
            raise ValueError("NVFP4 activations are 'nvfp4' (W4A4) or 'e4m3' (W4A8)")
        self.activations = activations
        if activations == "e4m3":
            self.contract = "nvfp4-e2m1-block16-128x4-w4a8-gfx950-v1"
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
        if self.activations == "e4m3" and values.dtype == torch.float16:
            raise ValueError("the W4A8 NVFP4 path quantizes BF16 (or FP32) activations")
        shape = values.shape
        matrix = values.to(torch.bfloat16) if values.dtype == torch.float32 else values
        matrix = matrix.reshape(-1, weight.in_features)
        if matrix.shape[0] == 0:
            raise ValueError("NVFP4 input rows must be nonempty")
        if matrix.stride(1) != 1 or matrix.stride(0) % 8:
            matrix = matrix.contiguous()
        if self.activations == "nvfp4":
            if matrix.data_ptr() % 16:
                matrix = matrix.clone()  # the quantizer reads 16-byte vectors
            codes, scales = kernels.nvfp4_quantize_rows(matrix, weight.input_scale)
            # The output scale as the reference forms it (one fp32 division on the device).
            alpha = weight.alpha / weight.input_scale
            output = kernels.nvfp4_w4a4_gemm(
                codes, scales, weight.packed, weight.scales, alpha, matrix.shape[0], bias
            )
        else:
            codes, act_scale = kernels.quantize_rows(matrix)
            output = kernels.nvfp4_gemm(
                codes, act_scale, weight.packed, weight.scales, weight.alpha, matrix.shape[0], bias
            )
        self.calls += 1
        self.rows += matrix.shape[0]
        return output.reshape(*shape[:-1], weight.out_features)
