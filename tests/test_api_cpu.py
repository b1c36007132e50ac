"""Host-side contract of the drop-in modules, checked on the CPU.

Each test states one clause of the module contract (RowFP8Execution,
RowFP8Linear, the fused compositions, NVFP4Weight / NVFP4Execution) and checks
it on small tensors; no GPU is involved.  The fixture data (E4M3 codes
0..127 as a 16 x 8 matrix, row scales 0.01..0.1) is the one of the reference's
tests/test_fp8_linear.py:13-16, so the expected values there carry over.
"""

import numpy as np
import pytest
import torch

from tests.conftest import golden
from vflash_amd import fused, kernels
from vflash_amd.fp8_linear import RowFP8Execution, RowFP8Linear, _quantize_activation_torch
from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight

OUT, IN = 16, 8


@pytest.fixture
def fp8_matrix():
    """(codes [16, 8] E4M3 holding codes 0..127, row scales [16, 1])."""
    codes = torch.arange(OUT * IN).reshape(OUT, IN).to(torch.float8_e4m3fn)
    return codes, torch.linspace(0.01, 0.1, OUT).unsqueeze(1)


def restored_linear(value, codes, scales, bias):
    """The weight-only arithmetic of the contract: restore the weight in the
    value's dtype from codes * row scale, then an ordinary linear."""
    return torch.nn.functional.linear(value, (codes.float() * scales).to(value.dtype), bias)


# --- weight-only mode: the exact restored-weight expression --------------------

@pytest.mark.parametrize("lead", [(), (3,), (2, 3), (0,)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_weight_only_output_is_bitwise_the_restored_weight_linear(fp8_matrix, lead, dtype):
    codes, scales = fp8_matrix
    gen = torch.Generator().manual_seed(len(lead))
    value = torch.randn(*lead, IN, generator=gen).to(dtype)
    bias = torch.randn(OUT, generator=gen).to(dtype)
    ex = RowFP8Execution()
    got = ex.linear(value, codes, scales, bias)
    want = restored_linear(value, codes, scales, bias)
    assert got.dtype == dtype and got.shape == (*lead, OUT)
    assert torch.equal(got, want)
    assert ex.calls == {"weight_only": 1, "w8a8": 0}


def test_weight_only_matches_the_committed_vector():
    kat = golden("weight_only_kat.npz")
    out = RowFP8Execution().linear(
        torch.from_numpy(kat["values"]).to(torch.bfloat16),
        torch.from_numpy(kat["codes"]).view(torch.float8_e4m3fn),
        torch.from_numpy(kat["scales"]),
        torch.from_numpy(kat["bias"]).to(torch.bfloat16),
    )
    assert np.array_equal(out.float().numpy(), kat["expected"])


# --- RowFP8Linear: a meta-initialized replacement that keeps the bias object ----

def test_module_starts_on_meta_and_runs_once_assigned(fp8_matrix):
    codes, scales = fp8_matrix
    dense = torch.nn.Linear(IN, OUT)
    ex = RowFP8Execution()
    mod = RowFP8Linear(dense, ex)
    # Nothing is materialized before the loader assigns; the bias is the original object.
    assert mod.weight.is_meta and mod.row_scale.is_meta
    assert mod.bias is dense.bias
    assert (mod.in_features, mod.out_features) == (IN, OUT)
    mod.load_state_dict({"weight": codes, "row_scale": scales, "bias": dense.bias}, assign=True)
    assert not mod.weight.requires_grad
    value = torch.randn(2, IN)
    assert torch.equal(mod(value), ex.linear(value, codes, scales, mod.bias))


# --- refusals: each happens before any GEMM and counts nothing ------------------

LAYOUT_BREAKS = {
    "codes not E4M3": lambda c, s, v, b: (c.float(), s, v, b),
    "scale not fp32": lambda c, s, v, b: (c, s.bfloat16(), v, b),
    "scale [1, N] instead of [N, 1]": lambda c, s, v, b: (c, s.T, v, b),
    "value width differs from K": lambda c, s, v, b: (c, s, torch.ones(3, IN - 1), b),
    "codes not 2-D": lambda c, s, v, b: (c.flatten(), s, v, b),
    "bias of the wrong width": lambda c, s, v, b: (c, s, v, torch.ones(OUT - 1)),
}


@pytest.mark.parametrize("mode", ["weight-only", "w8a8"])
@pytest.mark.parametrize("clause", sorted(LAYOUT_BREAKS))
def test_layout_refusal_precedes_every_gemm(fp8_matrix, monkeypatch, mode, clause):
    codes, scales = fp8_matrix
    args = LAYOUT_BREAKS[clause](codes, scales, torch.ones(3, IN), None)

    def gemm_reached(*_a, **_k):
        raise AssertionError(f"{clause}: a GEMM ran on a refused layout")

    monkeypatch.setattr(torch.nn.functional, "linear", gemm_reached)
    monkeypatch.setattr(kernels, "fp8_gemm", gemm_reached)
    ex = RowFP8Execution(mode)
    with pytest.raises(ValueError, match="declared"):
        ex.linear(args[2], args[0], args[1], args[3])
    assert ex.calls == {"weight_only": 0, "w8a8": 0}


@pytest.mark.parametrize("quantizer", ["torch", "triton", "hip"])
def test_w8a8_without_a_gfx950_device_refuses_with_no_fallback(fp8_matrix, quantizer):
    codes, scales = fp8_matrix
    ex = RowFP8Execution("w8a8", activation_quantizer=quantizer)
    with pytest.raises(ValueError, match="gfx950"):
        ex.linear(torch.ones(3, IN, dtype=torch.bfloat16), codes, scales)
    assert ex.calls == {"weight_only": 0, "w8a8": 0}


@pytest.mark.parametrize(
    "build",
    [
        lambda: RowFP8Execution("fp16"),
        lambda: RowFP8Execution(activation_quantizer="cuda"),
        lambda: RowFP8Execution(fast_accum=1),
        lambda: RowFP8Execution(fast_accum="yes"),
    ],
    ids=["unknown mode", "unknown quantizer", "fast_accum int", "fast_accum str"],
)
def test_construction_refuses_undeclared_choices(build):
    with pytest.raises(ValueError):
        build()


def test_select_refuses_an_unknown_mode_and_keeps_the_current_one():
    ex = RowFP8Execution()
    with pytest.raises(ValueError):
        ex.select("silent-fallback")
    assert ex.mode == "weight-only"
    ex.select("w8a8")
    assert ex.mode == "w8a8"


# --- counters and the observer ---------------------------------------------------

def test_each_execution_owns_its_counters_and_observer(fp8_matrix):
    codes, scales = fp8_matrix
    first, second = RowFP8Execution(), RowFP8Execution("w8a8")
    snapshots = []
    first.observer = lambda: snapshots.append(dict(first.calls))
    first.linear(torch.ones(IN), codes, scales)
    # The observer sees the counters before the call it precedes.
    assert snapshots == [{"weight_only": 0, "w8a8": 0}]
    assert first.calls == {"weight_only": 1, "w8a8": 0}
    assert second.mode == "w8a8" and second.calls == {"weight_only": 0, "w8a8": 0}
    assert second.observer is None


def test_observer_fires_on_every_200th_call_ahead_of_it(fp8_matrix):
    codes, scales = fp8_matrix
    ex = RowFP8Execution()
    fired_at = []
    ex.observer = lambda: fired_at.append(ex.calls["weight_only"])
    for _ in range(401):
        ex.linear(torch.ones(IN), codes, scales)
    assert fired_at == [0, 200, 400]


# --- the portable ("torch") activation quantizer ---------------------------------

@pytest.mark.parametrize("rows", [1, 16, 17])
def test_portable_quantizer_layout_and_known_answers(rows):
    # Rows are a strided view (every other 64-wide half of a 128-wide buffer);
    # row 0 is zero (scale 1), row 1 sits at the bf16 minimum normal, the rest
    # span [-448, 448].
    storage = torch.full((rows, 2 * 64), float("nan"), dtype=torch.bfloat16)
    view = storage[:, :64]
    view.copy_(torch.linspace(-448, 448, 64))
    view[0].zero_()
    if rows > 1:
        view[1].fill_(torch.finfo(torch.bfloat16).tiny)
    codes, scales = _quantize_activation_torch(view)
    padded = -(-rows // 16) * 16
    assert codes.shape == (padded, 64) and scales.shape == (padded, 1)
    assert scales[0].item() == 1.0 and not codes[0].view(torch.uint8).any()
    # Padding rows: codes 0, scale 1.
    assert not codes[rows:].view(torch.uint8).any() and bool((scales[rows:] == 1).all())
    # The input's other half is untouched.
    assert bool(torch.isnan(storage[:, 64:].float()).all())
    assert np.array_equal(codes.view(torch.uint8).numpy(), golden("quant_kat.npz")[f"codes{rows}"])


# --- fused compositions refuse exactly like the linear ---------------------------

def test_fused_compositions_refuse_before_any_kernel(fp8_matrix):
    codes, scales = fp8_matrix
    ex = RowFP8Execution("w8a8")
    x = torch.ones(3, IN, dtype=torch.bfloat16)
    merged = torch.cat([codes] * 3), torch.cat([scales] * 3)
    with pytest.raises(ValueError, match="gfx950"):
        fused.qkv_linear(ex, x, *merged)
    with pytest.raises(ValueError, match="w8a8"):
        fused.qkv_linear(RowFP8Execution(), x, codes, scales)
    with pytest.raises(ValueError, match="matching"):
        fused.merge_qkv([codes, codes, codes[: OUT // 2]], [scales] * 3)
    assert ex.calls == {"weight_only": 0, "w8a8": 0}


# --- NVFP4 ----------------------------------------------------------------------

def nvfp4(rows=128, half_k=32, scale_cols=4, alpha=2.0, input_scale=4.0):
    return NVFP4Weight(
        torch.zeros((rows, half_k), dtype=torch.uint8),
        torch.zeros((rows, scale_cols), dtype=torch.uint8),
        torch.tensor(alpha, dtype=torch.float32),
        torch.tensor(input_scale, dtype=torch.float32),
    )


@pytest.mark.parametrize("bad", [0.0, -1.0, float("nan"), float("inf")])
@pytest.mark.parametrize("which", ["alpha", "input_scale"])
def test_nvfp4_calibration_must_be_positive_and_finite(which, bad):
    with pytest.raises(ValueError, match="positive and finite"):
        nvfp4(**{which: bad})


@pytest.mark.parametrize(
    "shape", [dict(rows=100), dict(scale_cols=3), dict(half_k=30, scale_cols=3)],
    ids=["rows not a multiple of 128", "scales not K/16", "K/2 not a multiple of 32"],
)
def test_nvfp4_layout_must_be_the_128x4_contract(shape):
    with pytest.raises(ValueError, match="128x4"):
        nvfp4(**shape)


@pytest.mark.parametrize(
    "value,match",
    [
        (torch.ones((1, 64), dtype=torch.bfloat16), "gfx950"),
        (torch.ones((1, 63), dtype=torch.bfloat16), "frozen"),
        (torch.ones((1, 64), requires_grad=True), "inference-only"),
    ],
    ids=["no gfx950 device", "width differs", "needs grad"],
)
def test_nvfp4_refusals_count_nothing(value, match):
    ex = NVFP4Execution()
    with pytest.raises(ValueError, match=match):
        ex.linear(value, nvfp4())
    assert (ex.calls, ex.rows) == (0, 0)


@pytest.mark.parametrize("fmt", ["w4a8", "w4a4"])
def test_nvfp4_kernel_wrappers_refuse_mismatched_block_scales(fmt):
    # The kernels address the block scales from N and K alone, so a scale matrix
    # of another shape is refused before any launch (and before the device check).
    from vflash_amd import kernels

    n, k, rows = 128, 128, 16
    packed = torch.zeros((n, k // 2), dtype=torch.uint8)
    bad_scales = torch.zeros((n, k // 32), dtype=torch.uint8)
    alpha = torch.tensor([1.0])
    with pytest.raises(ValueError, match="block scales"):
        if fmt == "w4a8":
            codes = torch.zeros((rows, k), dtype=torch.float8_e4m3fn)
            kernels.nvfp4_gemm(codes, torch.ones(rows, 1), packed, bad_scales, alpha, rows)
        else:
            codes = torch.zeros((rows, k // 2), dtype=torch.uint8)
            act = torch.zeros((128, k // 16), dtype=torch.uint8)
            kernels.nvfp4_w4a4_gemm(codes, act, packed, bad_scales, alpha, rows)
    with pytest.raises(ValueError, match="packed weights"):
        if fmt == "w4a8":
            kernels.nvfp4_gemm(codes, torch.ones(rows, 1), packed.t(), bad_scales, alpha, rows)
        else:
            kernels.nvfp4_w4a4_gemm(codes, act, packed.t(), bad_scales, alpha, rows)


# --- measurement ---------------------------------------------------------------

def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    from pathlib import Path

    bench = Path(__file__).resolve().parents[1] / "bench.py"
    done = subprocess.run([sys.executable, str(bench), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert done.returncode != 0 and "one GPU" in done.stderr + done.stdout


def test_bench_operand_variants_keep_the_shapes_and_finite_codes():
    # The power-limit comparison runs the same GEMM on other operand bits:
    # constant codes, or uniformly random finite E4M3 codes whose activation
    # rows quantize with scale 1 to exactly the drawn codes.
    import importlib.util
    from pathlib import Path

    spec = importlib.util.spec_from_file_location(
        "bench_module", Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    from oracle import fp8 as O

    x = torch.randn((48, 64)).to(torch.bfloat16)
    codes = torch.zeros((32, 64), dtype=torch.uint8).view(torch.float8_e4m3fn)
    scale, bias = torch.ones((32, 1)), torch.zeros(32, dtype=torch.bfloat16)
    cx, cw, cs, cb = bench.operand_variant("constant", x, codes, scale, bias)
    assert torch.equal(cx, torch.ones_like(x)) and bool((cw.view(torch.uint8) == 0x30).all())
    assert cs is scale and cb is bias
    rx, rw, _, _ = bench.operand_variant("random", x, codes, scale, bias)
    assert rx.shape == x.shape and rw.shape == codes.shape
    for c in (rw.view(torch.uint8), rx.float().to(torch.float8_e4m3fn).view(torch.uint8)):
        assert not bool(((c & 0x7F) == 0x7F).any())  # no NaN code
    qc, qs = O.quantize_rows(rx.float().numpy())
    assert np.all(qs[:48] == 1.0)
    assert np.array_equal(qc[:48], rx.float().to(torch.float8_e4m3fn).view(torch.uint8).numpy())


def test_stacked_qkv_adapters_layout():
    # stack_adapters lays the Q/K/V pack out for one down-projection and one
    # epilogue: branch b's down rows at b * R (R = ceil16 of the largest rank),
    # its up rows in its third of the columns, zeros elsewhere.
    from vflash_amd.fused import LowRankResidual, stack_adapters

    g = torch.Generator().manual_seed(0)
    k, inner = 64, 32
    ranks = (16, 8, 20)
    res = [LowRankResidual(torch.randn((r, k), generator=g).to(torch.bfloat16),
                           torch.randn((inner, r), generator=g).to(torch.bfloat16), s)
           for r, s in zip(ranks, (0.5, 1.0, 0.0625))]
    st = stack_adapters(res, k, 3 * inner)
    assert st.rank == 20 and st.width == 32 and st.scalings == (0.5, 1.0, 0.0625)
    assert st.down.shape == (96, k) and st.up.shape == (96, 20)
    assert st.up.stride(0) % 8 == 0  # rows padded to whole 8-element groups
    for b, r in enumerate(res):
        rank = r.down.shape[0]
        assert torch.equal(st.down[b * 32 : b * 32 + rank], r.down)
        assert not st.down[b * 32 + rank : (b + 1) * 32].any()
        assert torch.equal(st.up[b * inner : (b + 1) * inner, :rank], r.up)
        assert not st.up[b * inner : (b + 1) * inner, rank:].any()


def test_low_rank_residual_refusals():
    from vflash_amd.fused import LowRankResidual, stack_adapters

    k, inner = 64, 32
    ok = LowRankResidual(torch.zeros((16, k), dtype=torch.bfloat16),
                         torch.zeros((inner, 16), dtype=torch.bfloat16), 1.0)
    with pytest.raises(ValueError, match="three branches"):
        stack_adapters([ok] * 4, k, 3 * inner)
    with pytest.raises(ValueError, match="does not match"):
        stack_adapters([ok] * 3, k + 16, 3 * inner)
    bad_rank = LowRankResidual(torch.zeros((16, k), dtype=torch.bfloat16),
                               torch.zeros((inner, 8), dtype=torch.bfloat16), 1.0)
    with pytest.raises(ValueError, match="compatible"):
        stack_adapters([ok, ok, bad_rank], k, 3 * inner)
    fp32 = LowRankResidual(torch.zeros((16, k)), torch.zeros((inner, 16)), 1.0)
    with pytest.raises(ValueError, match="BF16"):
        stack_adapters([ok, ok, fp32], k, 3 * inner)
    inf = LowRankResidual(ok.down, ok.up, float("inf"))
    with pytest.raises(ValueError, match="finite"):
        stack_adapters([ok, ok, inf], k, 3 * inner)
    big = LowRankResidual(torch.zeros((136, k), dtype=torch.bfloat16),
                          torch.zeros((inner, 136), dtype=torch.bfloat16), 1.0)
    with pytest.raises(ValueError, match="ranks up to 128"):
        stack_adapters([ok, ok, big], k, 3 * inner)
