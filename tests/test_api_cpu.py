"""Host-side contract of the drop-in API (mirrors the reference's CPU tests).

Covers tests/test_fp8_linear.py and tests/test_h3_nvfp4_linear.py behaviours:
weight-only exact expression, module construction, refusal of w8a8 off the
supported device without counting, layout refusals before any GEMM, observer
cadence, NVFP4 validation.  No GPU.
"""

import numpy as np
import pytest
import torch

from tests.conftest import golden
from vflash_amd import fused, kernels
from vflash_amd.fp8_linear import RowFP8Execution, RowFP8Linear, _quantize_activation_torch
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight


def weights():
    codes = torch.arange(128).reshape(16, 8).to(torch.float8_e4m3fn)
    scales = torch.linspace(0.01, 0.1, 16).unsqueeze(1)
    return codes, scales


@pytest.mark.parametrize("shape", [(8,), (3, 8), (2, 3, 8), (0, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_weight_only_is_exact_restored_weight_expression(shape, dtype):
    codes, scales = weights()
    values = torch.randn(shape, dtype=dtype)
    bias = torch.randn(16, dtype=dtype)
    execution = RowFP8Execution()
    actual = execution.linear(values, codes, scales, bias)
    restored = (codes.float() * scales).to(dtype)
    expected = torch.nn.functional.linear(values, restored, bias)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)
    assert execution.calls == {"weight_only": 1, "w8a8": 0}


def test_weight_only_golden_vector():
    g = golden("weight_only_kat.npz")
    codes = torch.from_numpy(g["codes"]).view(torch.float8_e4m3fn)
    out = RowFP8Execution().linear(
        torch.from_numpy(g["values"]).to(torch.bfloat16),
        codes,
        torch.from_numpy(g["scales"]),
        torch.from_numpy(g["bias"]).to(torch.bfloat16),
    )
    assert np.array_equal(out.float().numpy(), g["expected"])


def test_module_assigns_weight_scales_without_bias_copy():
    codes, scales = weights()
    original = torch.nn.Linear(8, 16)
    execution = RowFP8Execution()
    module = RowFP8Linear(original, execution)
    assert module.bias is original.bias and module.weight.is_meta and module.row_scale.is_meta
    module.load_state_dict({"weight": codes, "row_scale": scales, "bias": original.bias}, assign=True)
    value = torch.randn(2, 8)
    torch.testing.assert_close(module(value), execution.linear(value, codes, scales, module.bias), rtol=0, atol=0)
    assert not module.weight.requires_grad


@pytest.mark.parametrize("backend", ["torch", "triton", "hip"])
def test_w8a8_off_device_fails_without_fallback_or_count(backend):
    codes, scales = weights()
    execution = RowFP8Execution("w8a8", activation_quantizer=backend)
    with pytest.raises(ValueError, match="gfx950"):
        execution.linear(torch.ones(3, 8, dtype=torch.bfloat16), codes, scales)
    assert execution.calls == {"weight_only": 0, "w8a8": 0}


@pytest.mark.parametrize("bad", ["codes", "scale_dtype", "scale_shape", "input_shape", "rank", "bias"])
def test_bad_layout_never_enters_gemm(bad, monkeypatch):
    codes, scales = weights()
    value = torch.ones(3, 8)
    bias = None
    if bad == "codes":
        codes = codes.float()
    elif bad == "scale_dtype":
        scales = scales.bfloat16()
    elif bad == "scale_shape":
        scales = scales.T
    elif bad == "input_shape":
        value = torch.ones(3, 7)
    elif bad == "rank":
        codes = codes.flatten()
    elif bad == "bias":
        bias = torch.ones(15)

    def forbidden(*args, **kwargs):
        pytest.fail("invalid layout reached GEMM")

    monkeypatch.setattr(torch.nn.functional, "linear", forbidden)
    monkeypatch.setattr(kernels, "fp8_gemm", forbidden)
    for mode in ("weight-only", "w8a8"):
        with pytest.raises(ValueError, match="declared"):
            RowFP8Execution(mode).linear(value, codes, scales, bias)


def test_executions_keep_precision_observation_and_counts_independent():
    codes, scales = weights()
    a, b = RowFP8Execution(), RowFP8Execution("w8a8")
    observed = []
    a.observer = lambda: observed.append(dict(a.calls))
    a.linear(torch.ones(8), codes, scales)
    assert observed == [{"weight_only": 0, "w8a8": 0}]
    assert b.mode == "w8a8" and b.calls == {"weight_only": 0, "w8a8": 0}
    with pytest.raises(ValueError):
        a.select("silent-fallback")
    assert a.mode == "weight-only"
    with pytest.raises(ValueError):
        RowFP8Execution(activation_quantizer="cuda")
    with pytest.raises(ValueError):
        RowFP8Execution(fast_accum=1)


def test_observer_runs_every_200_calls_before_the_call():
    codes, scales = weights()
    ex = RowFP8Execution()
    seen = []
    ex.observer = lambda: seen.append(ex.calls["weight_only"])
    for _ in range(401):
        ex.linear(torch.ones(8), codes, scales)
    assert seen == [0, 200, 400]


@pytest.mark.parametrize("rows", [1, 16, 17])
def test_portable_quantizer_pads_and_keeps_strided_input(rows):
    base = torch.full((rows, 128), float("nan"), dtype=torch.bfloat16)
    values = base[:, :64]
    values.copy_(torch.linspace(-448, 448, 64))
    values[0].zero_()
    if rows > 1:
        values[1].fill_(torch.finfo(torch.bfloat16).tiny)
    codes, scales = _quantize_activation_torch(values)
    padded = (rows + 15) // 16 * 16
    assert codes.shape == (padded, 64) and scales.shape == (padded, 1)
    assert (codes[0].float() == 0).all() and scales[0].item() == 1
    assert (codes[rows:].float() == 0).all() and (scales[rows:] == 1).all()
    assert torch.isnan(base[:, 64:].float()).all()
    g = golden("quant_kat.npz")
    assert np.array_equal(codes.view(torch.uint8).numpy(), g[f"codes{rows}"])


def test_fused_compositions_refuse_before_any_kernel():
    codes, scales = weights()
    ex = RowFP8Execution("w8a8")
    x = torch.ones(3, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="gfx950"):
        fused.qkv_linear(ex, x, torch.cat([codes] * 3), torch.cat([scales] * 3))
    with pytest.raises(ValueError, match="w8a8"):
        fused.qkv_linear(RowFP8Execution(), x, codes, scales)
    with pytest.raises(ValueError, match="matching"):
        fused.merge_qkv([codes, codes, codes[:8]], [scales] * 3)
    assert ex.calls == {"weight_only": 0, "w8a8": 0}


def nv_weight(scale=4.0):
    return NVFP4Weight(
        torch.zeros((128, 32), dtype=torch.uint8),
        torch.zeros((128, 4), dtype=torch.uint8),
        torch.tensor(2.0, dtype=torch.float32),
        torch.tensor(scale, dtype=torch.float32),
    )


@pytest.mark.parametrize("scale", [0.0, -1.0, float("nan"), float("inf")])
def test_nvfp4_invalid_calibration_cannot_become_a_valid_model(scale):
    with pytest.raises(ValueError, match="positive and finite"):
        nv_weight(scale)


def test_nvfp4_layout_refusals():
    with pytest.raises(ValueError, match="128x4"):
        NVFP4Weight(torch.zeros((100, 32), dtype=torch.uint8), torch.zeros((100, 4), dtype=torch.uint8),
                    torch.tensor(1.0), torch.tensor(1.0))
    with pytest.raises(ValueError, match="128x4"):
        NVFP4Weight(torch.zeros((128, 32), dtype=torch.uint8), torch.zeros((128, 3), dtype=torch.uint8),
                    torch.tensor(1.0), torch.tensor(1.0))


def test_nvfp4_unsupported_device_refuses_and_counts_nothing():
    ex = NVFP4Execution()
    with pytest.raises(ValueError, match="gfx950"):
        ex.linear(torch.ones((1, 64), dtype=torch.bfloat16), nv_weight())
    with pytest.raises(ValueError, match="frozen"):
        ex.linear(torch.ones((1, 63), dtype=torch.bfloat16), nv_weight())
    with pytest.raises(ValueError, match="inference-only"):
        ex.linear(torch.ones((1, 64), requires_grad=True), nv_weight())
    assert ex.calls == 0 and ex.rows == 0


def test_bench_measures_one_gpu_only():
    # This path is measured on one MI355X; several GPUs are a design note.
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    result = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, timeout=120)
    assert result.returncode != 0
    assert "one GPU" in result.stderr + result.stdout
