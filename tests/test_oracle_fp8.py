"""Pin the W8A8 oracle against the reference's KATs, torch, and exact arithmetic."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from oracle.baseline import weight_only_linear
from oracle.formats import FLT_MIN, bf16_round, e4m3_decode
from tests.conftest import golden


@pytest.mark.parametrize("rows", [1, 16, 17])
def test_quant_reference_kat_rows(rows):
    # tests/test_fp8_linear.py:99-120: zero row -> scale 1, codes 0; tiny row ->
    # FLT_MIN floor; padding rows zero / 1; codes finite.
    g = golden("quant_kat.npz")
    codes, scales = O.quantize_rows(g[f"x{rows}"])
    padded = (rows + 15) // 16 * 16
    assert codes.shape == (padded, 64) and scales.shape == (padded,)
    assert np.array_equal(codes, g[f"codes{rows}"])
    assert np.array_equal(scales, g[f"scales{rows}"])
    assert np.all(e4m3_decode(codes[0]) == 0) and scales[0] == 1
    assert np.all(codes[rows:] == 0) and np.all(scales[rows:] == 1)
    if rows > 1:
        assert scales[1] == FLT_MIN
    x = g[f"x{rows}"]
    expected = np.maximum(np.abs(x).max(axis=1) / np.float32(448), FLT_MIN)
    expected[0] = 1
    assert np.array_equal(scales[:rows], expected.astype(np.float32))


def test_quant_random_rows_match_torch_expression_over_60_decades():
    g = golden("quant_kat.npz")
    codes, scales = O.quantize_rows(g["xr"])
    assert np.array_equal(codes, g["codesr"]) and np.array_equal(scales, g["scalesr"])


def test_quant_invariants_on_random_rows():
    rng = np.random.default_rng(3)
    x = bf16_round(rng.standard_normal((64, 333)) * 10.0 ** rng.uniform(-20, 20, (64, 1)))
    codes, scales = O.quantize_rows(x)
    dq = e4m3_decode(codes[:64]).astype(np.float64) * scales[:64, None]
    # The row maximum maps to +-448 exactly (code 0x7e / 0xfe).
    arg = np.argmax(np.abs(x), axis=1)
    assert np.all((codes[np.arange(64), arg] & 0x7F) == 0x7E)
    # Dequantized values are within half an E4M3 step of the input.
    q = np.abs(x / scales[:64, None])
    step = np.where(q < 2.0**-6, 2.0**-9, 2.0 ** (np.floor(np.log2(np.maximum(q, 1e-30))) - 3))
    assert np.all(np.abs(dq - x) <= 0.5 * step * scales[:64, None] * (1 + 1e-6))


def test_gemm_oracle_matches_exact_rational_arithmetic():
    g = golden("gemm_small.npz")
    m = g["x"].shape[0]
    codes, sa = O.quantize_rows(g["x"])
    assert np.array_equal(codes, g["a_codes"]) and np.array_equal(sa, g["sa"])
    scaled = O.scaled_mm(codes[:m], sa[:m], g["w_codes"], g["sw"])
    assert np.array_equal(scaled, g["scaled"])
    out = O.add_bias(scaled, g["bias"])
    assert np.array_equal(out, g["expected"])
    assert np.array_equal(O.w8a8_linear(g["x"], g["w_codes"], g["sw"], g["bias"]), g["expected"])


def test_gemm_oracle_detects_a_transposed_or_dropped_scale():
    g = golden("gemm_small.npz")
    m = g["x"].shape[0]
    right = O.scaled_mm(g["a_codes"][:m], g["sa"][:m], g["w_codes"], g["sw"])
    wrong = O.scaled_mm(g["a_codes"][:m], np.ones(m, np.float32), g["w_codes"], g["sw"])
    assert not np.array_equal(right, wrong)


def test_weight_only_baseline_is_the_reference_expression():
    g = golden("weight_only_kat.npz")
    codes = torch.from_numpy(g["codes"]).view(torch.float8_e4m3fn)
    out = weight_only_linear(
        torch.from_numpy(g["values"]).to(torch.bfloat16),
        codes,
        torch.from_numpy(g["scales"]),
        torch.from_numpy(g["bias"]).to(torch.bfloat16),
    )
    assert np.array_equal(out.float().numpy(), g["expected"])


def test_weight_only_loader_kat_ones():
    # tests/test_fp8_loaders.py:39-47: ones codes x ones scales, ones input -> 16.
    codes = torch.ones(4, 16).to(torch.float8_e4m3fn)
    out = weight_only_linear(torch.ones(2, 16), codes, torch.ones(4, 1))
    assert torch.equal(out, torch.full((2, 4), 16.0))


def test_lora_oracle_matches_reference_kat():
    g = golden("lora_kat.npz")
    for strength, expected in zip(g["strengths"], g["expected"]):
        d = O.lora_delta(g["sample"], g["a"], g["b"], 1.0, float(strength))
        assert np.array_equal(O.lora_merge(g["sample"], d), expected)


def _every_bf16():
    from oracle.formats import bf16_from_bits

    return bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))


def _decimal_to_f32(v):
    """Exact decimal value -> nearest binary32 value (ties to even), as a float."""
    import decimal
    import struct

    if v == 0:
        return -0.0 if v.is_signed() else 0.0
    b = struct.unpack("<I", struct.pack("<f", float(v)))[0]
    cands = [c & 0xFFFFFFFF for c in (b - 1, b, b + 1)]
    cands = [c for c in cands if (c & 0x7F800000) != 0x7F800000]
    val = lambda c: decimal.Decimal(struct.unpack("<f", struct.pack("<I", c))[0])
    b = min(cands, key=lambda c: (abs(val(c) - v), c & 1))
    return struct.unpack("<f", struct.pack("<I", b))[0]


def _decimal_to_bf16_through_f32(v):
    """Exact decimal value -> binary32 (nearest, ties to even) -> bf16 value."""
    import decimal
    import struct

    if v == 0:
        return -0.0 if v.is_signed() else 0.0
    b = struct.unpack("<I", struct.pack("<f", float(v)))[0]
    cands = [c & 0xFFFFFFFF for c in (b - 1, b, b + 1)]
    cands = [c for c in cands if (c & 0x7F800000) != 0x7F800000]
    val = lambda c: decimal.Decimal(struct.unpack("<f", struct.pack("<I", c))[0])
    b = min(cands, key=lambda c: (abs(val(c) - v), c & 1))  # binary32 RNE from the exact value
    return float(bf16_round(np.float32([struct.unpack("<f", struct.pack("<I", b))[0]]))[0])


def test_gelu_oracle_equals_a_60_digit_evaluation_on_every_bf16_value():
    # GELU-tanh as a real function, evaluated with 60 decimal digits and rounded
    # to binary32 and then bf16, for every finite bf16 input.
    import decimal

    ctx = decimal.Context(prec=60)
    beta, kappa = decimal.Decimal(O.GELU_BETA), decimal.Decimal(O.GELU_KAPPA)
    x = _every_bf16()
    x = x[np.isfinite(x)]
    ours = O.gelu_tanh(x)
    ref = np.empty_like(ours)
    for i, xv in enumerate(x.tolist()):
        d = decimal.Decimal(xv)
        t = ctx.multiply(-2 * beta, ctx.add(d, ctx.multiply(kappa, d * d * d)))
        if t > 2000:  # below the smallest bf16 magnitude: a signed zero
            ref[i] = -0.0 if xv < 0 else 0.0
        else:
            ref[i] = _decimal_to_bf16_through_f32(ctx.divide(d, ctx.add(1, ctx.exp(t))))
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_gelu_oracle_equals_torch_binary64_gelu_and_tracks_the_binary32_kernel():
    x = _every_bf16()
    x = x[np.isfinite(x)]
    ours = O.gelu_tanh(x)
    # torch's gelu(approximate="tanh") in binary64 with the same binary32 constants
    # is the same function; its 1 + tanh(u) keeps enough digits above x = -5.
    ok = x > -5
    ref64 = torch.nn.functional.gelu(torch.from_numpy(x[ok]).double(), approximate="tanh")
    assert np.array_equal(ours[ok], bf16_round(ref64.float().numpy()))
    # torch's bf16 kernel (binary32 arithmetic, its own tanh): at most one bf16
    # step apart where 1 + tanh does not cancel; below, its binary32 1 + tanh(u)
    # loses digits and reaches 0 near x = -4.9 (where ours keeps the tiny value).
    ref = torch.nn.functional.gelu(torch.from_numpy(x).to(torch.bfloat16), approximate="tanh")
    ref = ref.float().numpy()
    upper = x > -2.0
    assert np.all(np.abs(ours - ref)[upper] <= np.abs(ref[upper]) * 2.0**-7 + 2.0**-133)
    assert (ours != ref)[upper].mean() < 1e-3
    # Closed forms: gelu(0) = 0, gelu(x) -> x for large x, -> -0 for large -x.
    assert O.gelu_tanh(np.float32([0.0]))[0] == 0
    assert O.gelu_tanh(np.float32([30.0]))[0] == 30.0
    assert O.gelu_tanh(np.float32([-30.0]))[0] == 0
    special = O.gelu_tanh(np.float32([np.inf, -np.inf, np.nan]))
    assert special[0] == np.inf and np.isnan(special[1]) and np.isnan(special[2])


def test_silu_oracle_steps_are_correctly_rounded_on_every_bf16_value():
    # The one step that is not a binary32 operation, RN(exp(-g)), against a
    # 60-digit evaluation; the quotient then follows binary32 arithmetic.
    import decimal
    import struct

    ctx = decimal.Context(prec=60)
    g = _every_bf16()
    g = g[np.isfinite(g)]
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    flt_max = decimal.Decimal(struct.unpack("<f", struct.pack("<I", 0x7F7FFFFF))[0])
    overflow = flt_max * (1 + decimal.Decimal(2) ** -25)  # values past it round to inf
    for gv, ev in zip(g.tolist(), e.tolist()):
        if abs(gv) > 200:  # far past the binary32 range: inf, or 0 below the subnormals
            assert ev == (np.inf if gv < 0 else 0.0)
            continue
        exact = ctx.exp(decimal.Decimal(-gv))
        if exact >= overflow:
            assert ev == np.inf
            continue
        assert ev == np.float32(_decimal_to_f32(exact)), gv
    with np.errstate(over="ignore", invalid="ignore"):
        q = g / (np.float32(1.0) + e)
    assert np.array_equal(O.silu(g).view(np.uint32), bf16_round(q).view(np.uint32))
    # torch's binary64 silu rounded once: the same result except where the three
    # binary32 roundings land differently or exp(-g) overflows binary32.
    ref = bf16_round(torch.nn.functional.silu(torch.from_numpy(g).double()).float().numpy())
    differ = O.silu(g) != ref
    assert differ[g > -88.5].mean() < 1e-3 and np.all(O.silu(g)[g < -88.75] == 0)
    special = O.silu(np.float32([np.inf, -np.inf, np.nan]))
    assert special[0] == np.inf and np.isnan(special[1]) and np.isnan(special[2])


def test_silu_mul_oracle_tracks_torch_eager_bf16_on_every_gate_value():
    # H3's _silu_mul on bf16 tensors: value * F.silu(gate), each op rounding to bf16.
    from oracle.formats import bf16_from_bits

    g = bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    g = g[np.isfinite(g)]
    rng = np.random.default_rng(11)
    v = bf16_round(rng.standard_normal(g.size) * 4)
    ours = O.silu_mul(np.stack([v, g], -1).reshape(-1, 2))
    tv = torch.from_numpy(v).to(torch.bfloat16).reshape(-1, 1)
    tg = torch.from_numpy(g).to(torch.bfloat16).reshape(-1, 1)
    ref = (tv * torch.nn.functional.silu(tg)).float().numpy()
    # Different binary32 exp implementations may flip the rounding of silu by one
    # bf16 step, which the product then carries.
    with np.errstate(invalid="ignore"):
        close = (ours == ref) | (np.abs(ours - ref) <= np.abs(ref) * 2.0**-6 + 2.0**-133)
    assert np.all(close)
    assert (ours != ref).mean() < 2e-3
    # Closed forms: silu(0) = 0; silu(g) -> g for large g and -> -0 for large -g.
    assert O.silu_mul(np.float32([[3.0, 0.0]]))[0, 0] == 0
    assert O.silu_mul(np.float32([[1.0, 100.0]]))[0, 0] == 100.0
    assert O.silu_mul(np.float32([[1.0, -200.0]]))[0, 0] == 0
    # chunk(2, -1): values are the first half of the packed row.
    packed = np.float32([[1.0, 2.0, 0.0, 50.0]])
    assert np.array_equal(O.silu_mul(packed), np.float32([[0.0, 100.0]]))


def test_gate_residual_matches_torch_eager_bf16():
    rng = np.random.default_rng(5)
    res = bf16_round(rng.standard_normal((33, 70)))
    gate = bf16_round(rng.uniform(0, 1, 70))
    y = bf16_round(rng.standard_normal((33, 70)) * 3)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)
    ref = (t(res) + t(gate) * t(y)).float().numpy()
    assert np.array_equal(O.gate_residual(res, gate, y), ref)


def test_merged_qkv_equals_concatenated_projections():
    rng = np.random.default_rng(6)
    x = bf16_round(rng.standard_normal((20, 64)))
    ws = [rng.integers(0, 256, (32, 64)).astype(np.uint8) & 0xF7 for _ in range(3)]
    ss = [rng.uniform(0.001, 0.01, 32).astype(np.float32) for _ in range(3)]
    merged = O.w8a8_linear(x, np.concatenate(ws), np.concatenate(ss))
    parts = [O.w8a8_linear(x, w, s) for w, s in zip(ws, ss)]
    assert np.array_equal(merged, np.concatenate(parts, axis=1))


@pytest.mark.parametrize("hidden", [64, 5120, 5376])
@pytest.mark.parametrize("eps", [0.0, 1e-6, 1e-5, 0.25])
def test_rms_norm_oracle_is_torch_where_the_sum_is_exact(hidden, eps):
    # x = k/16 with |k| <= 16: every square is a multiple of 2^-8 and every
    # partial sum is exact in binary32, so any summation order gives one rstd
    # and torch's rms_norm must agree bit for bit (with and without weight).
    g = torch.Generator().manual_seed(hidden)
    x = (torch.randint(-16, 17, (32, hidden), generator=g).float() / 16).to(torch.bfloat16)
    w = (torch.rand(hidden, generator=g) * 2).to(torch.bfloat16)
    ref = torch.nn.functional.rms_norm(x, (hidden,), w, eps).float().numpy()
    assert np.array_equal(O.rms_norm(x.float().numpy(), w.float().numpy(), eps), ref)
    ref0 = torch.nn.functional.rms_norm(x, (hidden,), None, eps).float().numpy()
    assert np.array_equal(O.rms_norm(x.float().numpy(), None, eps), ref0)


def test_rms_norm_oracle_keeps_eps_in_binary32_and_rounds_once():
    # Mean squares near eps: a bf16-rounded eps, or a bf16 rounding before the
    # weight, changes thousands of outputs; the oracle changes none.
    g = torch.Generator().manual_seed(1)
    x = (torch.randint(-16, 17, (64, 512), generator=g).float() * 2.0**-12).to(torch.bfloat16)
    w = (torch.rand(512, generator=g) * 2).to(torch.bfloat16)
    ref = torch.nn.functional.rms_norm(x, (512,), w, 1e-5).float().numpy()
    xs, ws = x.float().numpy(), w.float().numpy()
    assert np.array_equal(O.rms_norm(xs, ws, 1e-5), ref)
    bf16_eps = float(torch.tensor(1e-5).to(torch.bfloat16))
    assert (O.rms_norm(xs, ws, bf16_eps) != ref).sum() > 1000
    assert (bf16_round(O.rms_norm(xs, None, 1e-5) * ws) != ref).sum() > 1000


def test_rms_norm_oracle_tracks_torch_on_random_rows():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(128, 5120, generator=g) * 3).to(torch.bfloat16)
    w = (torch.rand(5120, generator=g) * 2).to(torch.bfloat16)
    ref = torch.nn.functional.rms_norm(x, (5120,), w, 1e-6).float().numpy().astype(np.float64)
    got = O.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6).astype(np.float64)
    # Summation order only: at most one bf16 step, on a few elements.
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7)
    assert (got != ref).mean() < 1e-4


def test_modulate_oracle_is_torch_eager_bf16():
    g = torch.Generator().manual_seed(3)
    n = (torch.randn(64, 512, generator=g) * 4).to(torch.bfloat16)
    scale = (torch.randn(64, 512, generator=g) * 0.7).to(torch.bfloat16)
    shift = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    ref = (n * (1.0 + scale) + shift).float().numpy()
    got = O.modulate(n.float().numpy(), scale.float().numpy(), shift.float().numpy())
    assert np.array_equal(got, ref)
    # Leaving out the bf16 rounding of 1 + scale is visible.
    fused = bf16_round(bf16_round(n.float().numpy() * (1.0 + scale.float().numpy())) + shift.float().numpy())
    assert (fused != ref).sum() > 0


def _exact_adapter_case(rng, m, k, n, rank):
    """Integer-valued operands whose sums are exact in binary32, so torch's CPU
    bf16 matmuls (binary32 accumulation, one rounding) round the exact sums, as
    the oracle does: t takes values up to k * 9, beyond bf16's 8-bit significand,
    so its rounding is exercised; base values are random bf16."""
    x = rng.integers(-3, 4, (m, k)).astype(np.float32)
    down = rng.integers(-3, 4, (rank, k)).astype(np.float32)
    up = rng.integers(-3, 4, (n, rank)).astype(np.float32)
    base = bf16_round(rng.standard_normal((m, n)).astype(np.float32) * 300)
    return x, down, up, base


def _bf(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def test_adapted_chains_are_the_reference_eager_expressions():
    # The native block's adapter paths written as the reference writes them
    # (h3_native_denoiser.py:280-338: F.linear(F.linear(x, down), up) * scaling,
    # base + that, residual + gate * projected) and evaluated by torch in bf16
    # on the CPU, against the oracle's adapted / adapted_gate_residual chains.
    import torch.nn.functional as F

    rng = np.random.default_rng(11)
    m, k, n, rank = 48, 64, 96, 16
    x, down, up, base = _exact_adapter_case(rng, m, k, n, rank)
    residual = bf16_round(rng.standard_normal((m, n)).astype(np.float32) * 100)
    gate = bf16_round(rng.random(n).astype(np.float32))
    for scaling in (1.0, 0.0625, 0.3, 1.375):
        ref = _bf(base) + F.linear(F.linear(_bf(x), _bf(down)), _bf(up)) * scaling
        got = O.adapted(base, x, (down, up, scaling))
        assert np.array_equal(got.view(np.uint32), ref.float().numpy().view(np.uint32))
        ref_g = _bf(residual) + _bf(gate) * ref
        got_g = O.adapted_gate_residual(residual, gate, base, x, (down, up, scaling))
        assert np.array_equal(got_g.view(np.uint32), ref_g.float().numpy().view(np.uint32))
    # A chain that skips the rounding of the scaled delta differs.
    d = O.lora_delta(x, down, up)
    wrong = bf16_round(base + d * np.float32(0.3))
    assert not np.array_equal(wrong, O.adapted(base, x, (down, up, 0.3)))


def test_qkv_and_ffn_input_adapters_are_the_reference_eager_expressions():
    # _qkv_linear: torch.cat(chunk_b + _residual_linear(x, residual_b)) with three
    # branches of their own rank and scaling (h3_native_denoiser.py:301-316), and
    # _ffn_input: _silu_mul(_adapted_linear(...)) (:375-382).
    import torch.nn.functional as F

    rng = np.random.default_rng(12)
    m, k, inner = 40, 64, 32
    x = rng.integers(-3, 4, (m, k)).astype(np.float32)
    base = bf16_round(rng.standard_normal((m, 3 * inner)).astype(np.float32) * 300)
    adapters = []
    for rank, scaling in ((16, 0.0625), (8, 0.3), (24, 1.0)):
        adapters.append((rng.integers(-3, 4, (rank, k)).astype(np.float32),
                         rng.integers(-3, 4, (inner, rank)).astype(np.float32), scaling))
    chunks = _bf(base).chunk(3, dim=-1)
    ref = torch.cat([c + F.linear(F.linear(_bf(x), _bf(a)), _bf(b)) * s
                     for c, (a, b, s) in zip(chunks, adapters)], dim=-1)
    got = O.qkv_adapted(base, x, adapters)
    assert np.array_equal(got.view(np.uint32), ref.float().numpy().view(np.uint32))
    # The branches are not interchangeable: swapping two changes the result.
    swapped = O.qkv_adapted(base, x, [adapters[1], adapters[0], adapters[2]])
    assert not np.array_equal(swapped, got)

    down = rng.integers(-3, 4, (16, k)).astype(np.float32)
    up = rng.integers(-3, 4, (2 * inner, 16)).astype(np.float32)
    packed = _bf(base[:, : 2 * inner] / 64) + F.linear(F.linear(_bf(x), _bf(down)), _bf(up)) * 0.0625
    value, g = packed.chunk(2, dim=-1)
    ref = value * F.silu(g)
    got = O.silu_mul(O.adapted(bf16_round(base[:, : 2 * inner] / 64), x, (down, up, 0.0625)))
    assert np.array_equal(got.view(np.uint32), ref.float().numpy().view(np.uint32))
