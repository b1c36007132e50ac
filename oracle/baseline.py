"""The reference's CPU weight-only dequant-matmul path (test infrastructure).

Restates the ``weight-only`` branch of RowFP8Execution.linear
(src/vflash/native/h3_fp8_linear.py:88-91): restore the bf16 weight from its
E4M3 codes and row scales on every call, then ``F.linear`` with the bias.
This is the CPU baseline that bench.py times on host cores, and the exact
expression the reference test tests/test_fp8_linear.py:19-30 pins.
"""

from __future__ import annotations

import torch


def weight_only_linear(value, codes, scale, bias=None):
    restored = (codes.float() * scale).to(value.dtype)
    return torch.nn.functional.linear(value, restored, bias)


def gelu_ffn(value, up, up_scale, up_bias, down, down_scale, down_bias, gate, residual):
    """The FFN chain on the weight-only path (bf16 CPU ops, eager rounding)."""
    h = torch.nn.functional.gelu(weight_only_linear(value, up, up_scale, up_bias), approximate="tanh")
    y = weight_only_linear(h, down, down_scale, down_bias)
    return residual + gate * y
