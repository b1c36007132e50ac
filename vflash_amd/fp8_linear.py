"""Row-scaled E4M3 linear execution on MI355X (drop-in for the reference module).

Mirrors ``RowFP8Execution`` / ``RowFP8Linear`` of the reference
(src/vflash/native/h3_fp8_linear.py:34-149): same constructor arguments,
attributes, counters, observer cadence, ``measure`` scope names, validation
order and error conditions.  The W8A8 mode runs the HIP kernels of this
package on gfx950 and never falls back to another arithmetic:

* activation quantization: ``vflash_quantize_rows_e4m3`` (the fused kernel;
  ``activation_quantizer="triton"`` is accepted as the name of the reference's
  fused quantizer and selects the same HIP kernel), or the portable torch
  expression for ``"torch"``;
* GEMM + scales + bias: ``vflash_fp8_linear`` with binary32 accumulation and
  the reference's two bf16 roundings (``_scaled_mm`` output, then ``+ bias``).

``fast_accum`` is validated and recorded like the reference's; MFMA
accumulation is always binary32, so it does not change the arithmetic.
"""

from __future__ import annotations

from collections.abc import Callable
from contextlib import AbstractContextManager, nullcontext
from typing import Any

import torch

from vflash_amd import _lib, kernels
from vflash_amd.producers import QuantizedRows


def _quantize_activation_torch(matrix):
    """The reference's portable row quantizer (h3_fp8_linear.py:18-31), as torch
    evaluates it on the value's device, with the 16-row GEMM padding.

    Per row: binary32 maximum of |x|, ``scale = max(amax / 448, FLT_MIN)`` (1 for
    a zero row), codes ``e4m3(clamp(x / scale, -448, 448))``.  ``amax / 448`` is a
    tensor divided by a Python number: torch's GPU kernels evaluate that as a
    product with RN(1/448), its CPU kernels as a division, so on a GPU the scale
    can sit one binary32 ulp away from the fused quantizer's IEEE quotient
    (vflash_quantize_rows_e4m3, like the reference's Triton kernel with div_rn).
    This mode keeps torch's own evaluation, so it returns what the reference's
    portable mode returns on the same device.
    """
    rows = matrix.shape[0]
    if rows % 16:
        matrix = torch.nn.functional.pad(matrix, (0, 0, 0, 16 - rows % 16))
    floats = matrix.float()
    maxima = floats.abs().amax(dim=1, keepdim=True)
    act_scale = torch.where(
        maxima > 0,
        (maxima / 448.0).clamp_min(torch.finfo(torch.float32).tiny),
        torch.ones_like(maxima),
    )
    codes = (floats / act_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return codes, act_scale


def w8a8_supported(value: torch.Tensor) -> bool:
    return value.dtype == torch.bfloat16 and _lib.is_gfx950(value.device)


class RowFP8Execution:
    """One precision policy for a set of row-FP8 linears, with its call counters.

    Modes: ``weight-only`` multiplies by the weight restored from its codes and
    row scales (an ordinary torch linear); ``w8a8`` quantizes BF16 activations
    per token to E4M3 and runs the E4M3 GEMM on a gfx950 device, refusing any
    other input.  ``measure(name)`` optionally wraps the activation quantization
    and the GEMM in caller-supplied scopes (for asynchronous profiling).  Calls
    never synchronize the device, select a device or touch process state.
    """

    def __init__(
        self,
        mode: str = "weight-only",
        *,
        activation_quantizer: str = "torch",
        fast_accum: bool = False,
        measure: Callable[[str], AbstractContextManager[Any]] | None = None,
    ) -> None:
        if activation_quantizer not in ("torch", "triton", "hip"):
            raise ValueError("unknown FP8 activation quantizer")
        if type(fast_accum) is not bool:
            raise ValueError("fast_accum must be an explicit boolean")
        self.activation_quantizer = activation_quantizer
        self.fast_accum = fast_accum
        self.measure = measure if measure is not None else lambda _name: nullcontext()
        self.observer: Callable[[], None] | None = None
        self.calls = {"weight_only": 0, "w8a8": 0}
        self.select(mode)

    def select(self, mode: str) -> None:
        if mode not in ("weight-only", "w8a8"):
            raise ValueError("unknown FP8 execution mode")
        self.mode = mode

    def linear(self, value, weight, scale, bias=None):
        if self.observer is not None and sum(self.calls.values()) % 200 == 0:
            self.observer()
        if (
            weight.ndim != 2
            or value.ndim < 1
            or min(weight.shape) <= 0
            or value.shape[-1] != weight.shape[1]
            or weight.dtype != torch.float8_e4m3fn
            or scale.dtype != torch.float32
            or scale.shape != (weight.shape[0], 1)
            or weight.device != value.device
            or scale.device != value.device
        ):
            raise ValueError("FP8 codes/scales differ from the declared layout")
        if bias is not None and (
            bias.shape != (weight.shape[0],)
            or bias.device != value.device
            or bias.dtype != value.dtype
        ):
            raise ValueError("FP8 bias differs from the declared output")
        if self.mode == "weight-only":
            if isinstance(value, QuantizedRows):
                raise ValueError("pre-quantized activations require the w8a8 mode")
            self.calls["weight_only"] += 1
            restored = (weight.float() * scale).to(value.dtype)
            return torch.nn.functional.linear(value, restored, bias)
        if not w8a8_supported(value):
            raise ValueError("W8A8 requires gfx950 (MI355X) BF16 inputs")
        self.calls["w8a8"] += 1
        shape = value.shape
        if isinstance(value, QuantizedRows):
            # Codes and scales from a fused producer (vflash_amd.producers).
            codes, act_scale, rows = value.codes, value.scales, value.rows
        else:
            matrix = value.reshape(-1, shape[-1])
            rows = matrix.shape[0]
            if self.activation_quantizer == "torch":
                codes, act_scale = _quantize_activation_torch(matrix)
            else:
                with self.measure("linear.activation_quantize"):
                    codes, act_scale = kernels.quantize_rows(matrix)
        with self.measure("linear.fp8_gemm"):
            output = kernels.fp8_gemm(codes, act_scale, weight, scale, rows, bias)
        return output.reshape(*shape[:-1], weight.shape[0])


class RowFP8Linear(torch.nn.Module):
    """Stands in for an ``nn.Linear`` whose weight is stored as E4M3 row codes.

    ``weight`` (E4M3 ``[out, in]``) and ``row_scale`` (fp32 ``[out, 1]``) start
    on the meta device and hold no memory until a loader assigns them (for
    example ``load_state_dict(..., assign=True)``); the module's bias is the
    original module's bias object itself.  The forward pass is the execution's
    ``linear`` on those tensors, on whatever device the loader placed them.
    """

    def __init__(self, original: torch.nn.Linear, execution: RowFP8Execution):
        super().__init__()
        self.in_features = original.in_features
        self.out_features = original.out_features
        self.weight = torch.nn.Parameter(
            torch.empty(
                (self.out_features, self.in_features), device="meta", dtype=torch.float8_e4m3fn
            ),
            requires_grad=False,
        )
        self.register_buffer(
            "row_scale",
            torch.empty((self.out_features, 1), device="meta", dtype=torch.float32),
        )
        self.bias = original.bias
        self.execution = execution

    def forward(self, value):
        return self.execution.linear(value, self.weight, self.row_scale, self.bias)
