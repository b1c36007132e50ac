"""The torch restatement of the FP8 oracle (oracle/fp8_torch.py) against the
numpy oracle, bit for bit, on the CPU."""

import numpy as np
import torch

from oracle import fp8 as O
from oracle import fp8_torch as T
from oracle import formats as F


def test_bf16_round_is_the_oracles_rounding():
    rng = np.random.default_rng(0)
    vals = [rng.standard_normal(20000) * np.exp2(rng.integers(-140, 130, 20000))]
    # Exact ties between two bf16 neighbours, both parities, normal and subnormal,
    # and ties displaced by one binary64 ulp either way.
    base = F.bf16_round(rng.standard_normal(4000) * np.exp2(rng.integers(-135, 120, 4000)))
    base = base[np.isfinite(base) & (base != 0)].astype(np.float64)
    half = np.exp2(np.floor(np.log2(np.abs(base))).clip(min=-126) - 8)
    ties = base + np.sign(base) * half
    vals += [ties, np.nextafter(ties, np.inf), np.nextafter(ties, -np.inf)]
    vals.append(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 2.0**-133,
                          2.0**-134, 3 * 2.0**-135, F.bf16_round(3.3e38).astype(np.float64)]))
    x = np.concatenate(vals)
    want = F.bf16_round(x)
    got = T.bf16_round(torch.from_numpy(x)).numpy()
    assert np.array_equal(got.view(np.uint32)[np.isfinite(want)], want.view(np.uint32)[np.isfinite(want)])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])
    assert np.array_equal(np.signbit(got[want == 0]), np.signbit(want[want == 0]))
    # Ties go to even on every device (the GPU test of this restatement compares
    # against the kernels' hardware RNE conversions, which see many exact ties).
    t = torch.tensor([0.2509765625, -0.2509765625, 0.2529296875, 1.00390625, 1.01171875])
    assert T.bf16_round(t).tolist() == [0.25, -0.25, 0.25390625, 1.0, 1.015625]
    # A rounding through binary32 first (double rounding) differs on displaced ties:
    # the restatement is the direct one.
    through_f32 = torch.from_numpy(x).float().to(torch.bfloat16).float().numpy()
    assert not np.array_equal(through_f32[np.isfinite(want)].view(np.uint32),
                              want[np.isfinite(want)].view(np.uint32))


def test_quantize_rows_is_the_oracles_quantizer():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((37, 300)) * np.exp2(rng.integers(-30, 30, (37, 1)))).astype(np.float32)
    x[3] = 0.0
    x[5] = 1e-39
    x[7, :] = np.linspace(-448, 448, 300)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    codes, scales = T.quantize_rows(xb)
    rc, rs = O.quantize_rows(xb.float().numpy())
    assert np.array_equal(codes.numpy(), rc) and np.array_equal(scales.numpy(), rs)


def test_linear_chain_is_the_oracles_chain():
    rng = np.random.default_rng(2)
    m, k, n = 45, 256, 96
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    w_codes = torch.from_numpy(rng.integers(0, 0x7E, (n, k)).astype(np.uint8)
                               | (rng.integers(0, 2, (n, k)) * 0x80).astype(np.uint8))
    sw = torch.from_numpy((rng.random(n) * 0.01).astype(np.float32))
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * 0.01).to(torch.bfloat16)
    got = T.w8a8_linear(x, w_codes, sw, bias).numpy()
    want = O.w8a8_linear(x.float().numpy(), w_codes.numpy(), sw.numpy(), bias.float().numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # The gate-residual epilogue, with a broadcast gate row and with a per-token gate.
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(torch.bfloat16)
    for gate in (torch.rand(n).to(torch.bfloat16), torch.rand((m, n)).to(torch.bfloat16)):
        got = T.gate_residual(res, gate, torch.from_numpy(want)).numpy()
        ref = O.gate_residual(res.float().numpy(), gate.float().numpy(), want)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_activations_are_the_oracles_activations():
    rng = np.random.default_rng(3)
    y = torch.from_numpy(rng.standard_normal((64, 512)).astype(np.float32) * 4).to(torch.bfloat16)
    y[0, :4] = torch.tensor([float("inf"), float("-inf"), float("nan"), -0.0])
    got = T.gelu_tanh(y).numpy()
    want = O.gelu_tanh(y.float().numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got = T.silu_mul(y).numpy()
    want = O.silu_mul(y.float().numpy())
    same = got.view(np.uint32) == want.view(np.uint32)
    assert np.all(same | (np.isnan(got) & np.isnan(want)))


def test_adapter_chain_is_the_oracles_chain():
    rng = np.random.default_rng(4)
    m, k, n, rank = 33, 320, 72, 24
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    down = torch.from_numpy(rng.standard_normal((rank, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    up = torch.from_numpy(rng.standard_normal((n, rank)).astype(np.float32) * 0.05).to(torch.bfloat16)
    base = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(torch.bfloat16)
    for scaling, strength in ((1.0, 1.0), (0.0625, 1.0), (0.3, 1.375)):
        got = T.adapted(base, x, (down, up, scaling), strength).numpy()
        want = O.adapted(base.float().numpy(), x.float().numpy(),
                         (down.float().numpy(), up.float().numpy(), scaling), strength)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert torch.equal(T.adapted(base, x, None), base.float())
