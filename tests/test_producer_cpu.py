"""Host-side contract of the fused norm/modulation producer (no GPU needed)."""

import pytest
import torch

from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.producers import QuantizedRows, rmsnorm_modulate_quantize

E4M3 = torch.float8_e4m3fn


def rows(b=2, s=5, h=32):
    codes = torch.zeros((16, h), dtype=E4M3)
    return QuantizedRows(codes, torch.ones(16, 1), (b, s, h))


def test_quantized_rows_describe_the_replaced_activation():
    q = rows()
    assert q.shape == (2, 5, 32) and q.ndim == 3 and q.rows == 10
    assert q.dtype == torch.bfloat16 and q.device == torch.device("cpu") and q.values is None


def test_weight_only_mode_refuses_pre_quantized_rows():
    ex = RowFP8Execution()
    w = torch.zeros((8, 32), dtype=E4M3)
    with pytest.raises(ValueError, match="w8a8"):
        ex.linear(rows(), w, torch.ones(8, 1))
    assert ex.calls == {"weight_only": 0, "w8a8": 0}


def test_w8a8_refuses_pre_quantized_rows_off_gfx950():
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    with pytest.raises(ValueError, match="gfx950"):
        ex.linear(rows(), torch.zeros((8, 32), dtype=E4M3), torch.ones(8, 1))


@pytest.mark.parametrize(
    "value,scale,index,match",
    [
        (torch.zeros(10, 32, dtype=torch.bfloat16), torch.zeros(5, 32, dtype=torch.bfloat16), None, r"\[B,S,H\]"),
        (torch.zeros(2, 5, 32), torch.zeros(5, 32, dtype=torch.bfloat16), None, r"\[B,S,H\]"),
        (torch.zeros(2, 32, 5, dtype=torch.bfloat16).transpose(1, 2), torch.zeros(5, 32, dtype=torch.bfloat16), None, "contiguous"),
        (torch.zeros(2, 5, 32, dtype=torch.bfloat16), torch.zeros(4, 32, dtype=torch.bfloat16), None, r"\[S,H\]"),
        (torch.zeros(2, 5, 32, dtype=torch.bfloat16), torch.zeros(3, 32, dtype=torch.bfloat16), torch.zeros(4, dtype=torch.int64), r"\[S\]"),
        (torch.zeros(2, 5, 32, dtype=torch.bfloat16), torch.zeros(3, 32, dtype=torch.bfloat16), torch.zeros(5, dtype=torch.int64), "gfx950"),
    ],
)
def test_producer_validation(value, scale, index, match):
    with pytest.raises(ValueError, match=match):
        rmsnorm_modulate_quantize(value, None, scale, scale, eps=1e-6, index=index)
