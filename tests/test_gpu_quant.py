"""Per-token E4M3 quantization on gfx950: bit-exact against the oracle."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from oracle.formats import bf16_from_bits, bf16_round
from tests.conftest import golden
from vflash_amd import kernels
from vflash_amd.fp8_activation import quantize_activation
from vflash_amd.fp8_linear import _quantize_activation_torch

pytestmark = pytest.mark.gpu


def gpu_quant(x_np, dev, ldx=None):
    x = torch.from_numpy(np.ascontiguousarray(x_np, np.float32)).to(torch.bfloat16)
    if ldx is not None:
        big = torch.full((x.shape[0], ldx), float("nan"), dtype=torch.bfloat16)
        big[:, : x.shape[1]] = x
        x = big.to(dev)[:, : x_np.shape[1]]
    else:
        x = x.to(dev)
    codes, scales = kernels.quantize_rows(x)
    torch.cuda.synchronize()
    return codes.view(torch.uint8).cpu().numpy(), scales.reshape(-1).cpu().numpy(), x


def assert_exact(x_np, dev, **kw):
    x_np = bf16_round(x_np)  # the device sees the bf16 tensor
    codes, scales, _ = gpu_quant(x_np, dev, **kw)
    ref_codes, ref_scales = O.quantize_rows(x_np)
    assert np.array_equal(scales.view(np.uint32), ref_scales.view(np.uint32)), "scales differ"
    bad = codes != ref_codes
    assert not bad.any(), f"{bad.sum()} codes differ, first at {np.argwhere(bad)[:3]}"


@pytest.mark.parametrize("rows", [1, 16, 17])
def test_reference_kat_rows(dev, rows):
    g = golden("quant_kat.npz")
    codes, scales, _ = gpu_quant(g[f"x{rows}"], dev)
    assert np.array_equal(codes, g[f"codes{rows}"]) and np.array_equal(scales, g[f"scales{rows}"])


def test_random_rows_over_60_decades(dev):
    g = golden("quant_kat.npz")
    codes, scales, _ = gpu_quant(g["xr"], dev)
    assert np.array_equal(codes, g["codesr"]) and np.array_equal(scales, g["scalesr"])


def test_every_bf16_bit_pattern_under_many_scales(dev):
    v = bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    v = v[np.isfinite(v)]
    rng = np.random.default_rng(0)
    v = v[rng.permutation(v.size)]
    k = 256
    n = v.size // k * k
    x = v[:n].reshape(-1, k)  # each row gets its own amax (and so its own scale)
    assert_exact(x, dev)
    # Rows whose maximum is tiny: scale hits the FLT_MIN floor, subnormal inputs.
    tiny = bf16_from_bits(np.arange(1, 0x0100, dtype=np.uint16))
    assert_exact(np.stack([tiny[:128], -tiny[:128], tiny[-128:]]), dev)


@pytest.mark.parametrize("k", [16, 64, 3072, 5120, 13824, 16384])
def test_aligned_widths_exact(dev, k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((67, k)).astype(np.float32) * rng.uniform(0.01, 100, (67, 1))
    x[5] = 0.0
    assert_exact(x, dev)


@pytest.mark.parametrize("k", [17, 100, 1000, 20000, 32768])
def test_generic_widths_exact(dev, k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((9, k)).astype(np.float32) * 3
    assert_exact(x, dev)


def test_strided_input_is_read_not_written(dev):
    # The FFN value half of [M, 2F] has a doubled row stride (test_fp8_linear.py:99-115).
    rng = np.random.default_rng(2)
    x = bf16_round(rng.standard_normal((33, 512)))
    codes, scales, view = gpu_quant(x, dev, ldx=1024)
    ref_codes, ref_scales = O.quantize_rows(x)
    assert np.array_equal(codes, ref_codes) and np.array_equal(scales, ref_scales)
    base = view.as_strided((33, 1024), (1024, 1))
    assert torch.isnan(base[:, 512:].float()).all()


def test_matches_the_portable_expression_where_torch_divides(dev):
    # torch's CPU kernels evaluate amax / 448.0 as a division, the fused
    # quantizer's arithmetic: same codes and scales, bit for bit.
    g = torch.Generator().manual_seed(0)
    x = torch.randn((4096, 3072), generator=g).to(torch.bfloat16)
    c1, s1 = quantize_activation(x.to(dev))
    c2, s2 = _quantize_activation_torch(x)
    assert torch.equal(c1.view(torch.uint8).cpu(), c2.view(torch.uint8)) and torch.equal(s1.cpu(), s2)


def test_metric_shape_sampled_rows_and_full_properties(dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn((32760, 5120), generator=g).to(torch.bfloat16)
    codes, scales = kernels.quantize_rows(x.to(dev))
    assert codes.shape == (32768, 5120)
    # Every element: dequantized value within half an E4M3 step of the input.
    xd = x.to(dev).float()
    dq = codes[:32760].float() * scales[:32760]
    # Half an E4M3 step of |q| = |x / scale|: 2^(e - 4) for q in [2^e, 2^(e+1)),
    # 2^-10 below 2^-6; exponents from frexp (exact).  At an exact tie the
    # binary32 quotient and product roundings add up to ~(q / half) * 2^-23.
    q = (xd / scales[:32760]).abs()
    _, e = torch.frexp(q)
    half = torch.where(q < 2.0**-6, torch.full_like(q, 2.0**-10), torch.ldexp(torch.ones_like(q), e - 5))
    assert bool(((dq - xd).abs() <= half * scales[:32760] * (1 + 2.0**-12)).all())
    assert bool((codes[32760:].view(torch.uint8) == 0).all()) and bool((scales[32760:] == 1).all())
    rows = np.r_[0:64, 16000:16064, 32696:32760]
    c = codes.view(torch.uint8).cpu().numpy()[rows]
    s = scales.reshape(-1).cpu().numpy()[rows]
    rc, rs = O.quantize_rows(x.float().numpy()[rows], pad=1)
    assert np.array_equal(c, rc) and np.array_equal(s, rs)


def test_row_offsets_beyond_2_pow_31_elements(dev):
    # Strided rows whose byte offset crosses 2^31 (test_fp8_compile.py:16-40 shape).
    k = 14336
    stride = 2 * k
    m = (2**31 + stride - 1) // stride + 17
    assert (m - 1) * stride > 2**31
    base = torch.zeros((m, stride), dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(1)
    tail = torch.randn((40, k), generator=g).to(torch.bfloat16)
    base[m - 40 :, :k] = tail.to(dev)
    codes, scales = kernels.quantize_rows(base[:, :k])
    c = codes[m - 40 : m].view(torch.uint8).cpu().numpy()
    s = scales[m - 40 : m].reshape(-1).cpu().numpy()
    rc, rs = O.quantize_rows(tail.float().numpy(), pad=1)
    assert np.array_equal(c, rc) and np.array_equal(s, rs)
    assert bool((scales[: m - 40] == 1).all())


def test_hardware_e4m3_conversion_is_rne_on_every_clamped_binary32(dev):
    # The quantizers convert with v_cvt_pk_fp8_f32 after clamping to +-448; this
    # probe compares it with the software RNE encoder (pinned to torch's
    # float8_e4m3fn cast by the oracle tests) on every binary32 of that range.
    import subprocess
    from pathlib import Path

    probe = Path(__file__).resolve().parent / "probes" / "bin" / "e4m3_convert"
    if not probe.exists():
        pytest.fail("probe not built: run __graft_entry__.build()")
    result = subprocess.run([str(probe)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    fields = result.stdout.split()
    assert fields[0] == "values" and int(fields[1]) == 2 * (0x43E00000 + 1)
    assert fields[2] == "mismatches" and int(fields[3]) == 0, result.stdout


def fast_division_pairs():
    """Number of (amax, x) bf16 pairs the row-division probe covers: every
    positive finite bf16 amax whose scale takes the fast path, with every bf16
    x (both zeros included) of |x| <= amax."""
    a = np.arange(1, 0x7F80, dtype=np.uint32)
    amax = (a << 16).view(np.float32)
    s = np.maximum(amax / np.float32(448.0), np.float32(1.1754943508222875e-38))
    fast = (s >= np.float32(2.0**-72)) & (s <= np.finfo(np.float32).max)
    return int((2 * (a[fast].astype(np.int64) + 1)).sum())


def test_fast_row_division_gives_the_ieee_codes_on_every_bf16_pair(dev):
    # The quantizers divide a row by its scale with Markstein's correction on the
    # correctly rounded reciprocal; the probe converts both that quotient and the
    # IEEE one with the hardware E4M3 conversion for every bf16 pair of the fast path.
    import subprocess
    from pathlib import Path

    probe = Path(__file__).resolve().parent / "probes" / "bin" / "row_division"
    if not probe.exists():
        pytest.fail("probe not built: run __graft_entry__.build()")
    result = subprocess.run([str(probe)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    fields = result.stdout.split()
    assert fields[0] == "pairs" and int(fields[1]) == fast_division_pairs(), result.stdout
    assert fields[2] == "code_mismatches" and int(fields[3]) == 0, result.stdout


def non_finite_rows(k, seed=0):
    """Rows holding NaN, -NaN, +-inf, an all-NaN row, and finite rows around them."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((8, k), generator=g).to(torch.bfloat16)
    x[0, 3], x[0, 10] = float("nan"), 1000.0
    x[1, 5], x[1, 6] = float("inf"), -0.0
    x[2, 7], x[2, 9] = -float("inf"), float("inf")
    x[3, :] = float("nan")
    x[4, 0] = -float("nan")
    x[5, 1], x[5, 2] = float("nan"), float("inf")
    return x


def assert_codes_like_torch(codes, scales, x):
    """Bit-exact against the oracle (torch's arithmetic), except that every NaN
    code may carry either sign: the host computes inf/inf as a negative NaN,
    the GPU (like the reference's) as a positive one."""
    rc, rs = O.quantize_rows(x.float().numpy())
    c = codes.view(torch.uint8).cpu().numpy()
    s = scales.reshape(-1).cpu().numpy()
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    nan_ref = (rc & 0x7F) == 0x7F
    assert np.array_equal((c & 0x7F) == 0x7F, nan_ref)
    assert np.array_equal(c[~nan_ref], rc[~nan_ref])


@pytest.mark.parametrize("k", [512, 5120, 200])
def test_non_finite_rows_follow_torch(dev, k):
    # torch's amax propagates NaN (scale 1), an infinite row gets scale inf
    # (finite values -> signed zeros, inf/inf -> NaN), and clamp keeps NaN:
    # _quantize_activation_torch (h3_fp8_linear.py:18-31) on such rows.
    x = non_finite_rows(k)
    codes, scales = kernels.quantize_rows(x.to(dev))  # k = 200: the generic kernel
    assert_codes_like_torch(codes, scales, x)
    if k % 16 == 0:
        ref_c, ref_s = _quantize_activation_torch(x)  # torch's CPU kernels divide, as the kernel does
        assert torch.equal(scales.cpu(), ref_s)


def test_non_finite_rows_in_the_fused_quantizers(dev):
    from vflash_amd.producers import rmsnorm_modulate_quantize

    x = non_finite_rows(512, seed=1)
    la = (torch.randn((32, 512)) * 0.05).to(torch.bfloat16)
    codes, scales, _ = kernels.quantize_rows_lora(x.to(dev), la.to(dev))
    assert_codes_like_torch(codes, scales, x)
    # A NaN or inf anywhere in a row makes its RMSNorm all NaN (or NaN/zeros),
    # which the producer quantizes with the same rules.
    s = torch.zeros((8, 512), dtype=torch.bfloat16)
    q = rmsnorm_modulate_quantize(x.reshape(1, 8, 512).to(dev), None, s.to(dev), s.to(dev), eps=1e-6,
                                  keep_values=True)
    assert_codes_like_torch(q.codes, q.scales, q.values.reshape(8, 512).cpu())
    n = O.rms_norm(x.float().numpy(), None, 1e-6)
    got = q.values.reshape(8, 512).float().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(n))


def test_requantization_after_a_nan_row(dev):
    # A NaN input row makes the whole up-projection row NaN, and its GELU; the
    # requantization must give NaN codes with scale 1 (torch's amax), not
    # finite codes.
    from vflash_amd.prepare import quantize_weight_rows

    m, h, f = 32, 256, 512
    g = torch.Generator().manual_seed(2)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    x[5, 7] = float("nan")
    cu, su = quantize_weight_rows(torch.randn((f, h), generator=g) * 0.02)
    a, sa = kernels.quantize_rows(x.to(dev))
    y = kernels.fp8_gemm(a, sa, cu.to(dev), su.to(dev), m)
    hc, hs, gg = kernels.gelu_quantize_rows(y, keep_values=True)
    assert torch.isnan(gg[5].float()).all() and not torch.isnan(gg[torch.arange(m) != 5].float()).any()
    assert_codes_like_torch(hc, hs, gg.cpu())
    assert hs[5].item() == 1.0


def test_gelu_table_on_every_bf16_value(dev):
    # Every bf16 pattern (inf, NaN and subnormals included) through the GELU
    # quantizer: g is the oracle's correctly rounded GELU-tanh, bit for bit.
    from oracle import fp8 as O
    from oracle.formats import bf16_from_bits

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    y = bits.reshape(64, 1024).to(dev)
    _, _, g = kernels.gelu_quantize_rows(y, keep_values=True)
    got = g.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    want = O.gelu_tanh(bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16)))
    want_bits = (want.view(np.uint32) >> 16).astype(np.uint16)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan], want_bits[~nan])
    # NaN inputs stay NaN with their sign; -inf gives NaN.
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all(got[nan] & 0x7F)
    src = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    nan_in = ((src & 0x7F80) == 0x7F80) & ((src & 0x7F) != 0)
    assert np.array_equal(got[nan_in] & 0x8000, src[nan_in] & 0x8000)


def test_silu_epilogue_on_every_bf16_gate_value(dev):
    # The SwiGLU epilogue's silu (a window table generated from the correctly
    # rounded binary32 steps, closed forms outside it) against the oracle's
    # correctly rounded steps over every finite bf16 gate value: bit for bit.  Zero activations and weights make the
    # GEMM's output its bias exactly: the value columns carry 1.0 and the gate
    # columns every gate value, so h = bf16(1 * bf16(silu(g))) = bf16(silu(g)).
    from oracle import fp8 as O
    from oracle.formats import bf16_from_bits

    gates = bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    gates = gates[np.isfinite(gates) & ~((gates == 0) & np.signbit(gates))]  # +0 + -0 is +0
    f = -(-gates.size // 128) * 128
    gate_cols = np.zeros(f, np.float32)
    gate_cols[: gates.size] = gates
    bias = torch.from_numpy(np.concatenate([np.ones(f, np.float32), gate_cols])).to(torch.bfloat16)
    m, k = 16, 64
    a = torch.zeros((m, k), dtype=torch.float8_e4m3fn, device=dev)
    sa = torch.ones((m, 1), dtype=torch.float32, device=dev)
    w = torch.zeros((2 * f, k), dtype=torch.float8_e4m3fn, device=dev)
    sw = torch.ones((2 * f, 1), dtype=torch.float32, device=dev)
    h, _ = kernels.fp8_gemm_swiglu(a, sa, w, sw, m, bias.to(dev))
    got = h.float().cpu().numpy()
    assert np.array_equal(got[0], got[m - 1])
    got = got[0, : gates.size]
    want = O.silu(gates)
    differ = got.view(np.uint32) != want.view(np.uint32)
    print(f"silu epilogue: {int(differ.sum())} of {gates.size} gate values differ from the oracle")
    assert int(differ.sum()) == 0


def test_silu_epilogue_on_non_finite_and_extreme_gates(dev):
    # The closed forms outside the silu table's window: +inf stays +inf, -inf
    # and NaN give NaN, the largest negative bf16 gives -0, bf16 subnormals give
    # bf16(g / 2); the window's edges on both sides.  Same construction as above:
    # zero operands make each gate column its bias.
    gates = np.array([np.inf, -np.inf, np.nan, 3.3895314e38, -3.3895314e38, 128.0, -128.0,
                      127.5, -127.5, 2.0**-9, -(2.0**-9), 2.0**-10, -(2.0**-10), 1e-40, -1e-40,
                      -88.0, -89.0, -100.0], np.float32)
    gates = bf16_round(gates)
    f = 128
    gate_cols = np.zeros(f, np.float32)
    gate_cols[: gates.size] = gates
    bias = torch.from_numpy(np.concatenate([np.ones(f, np.float32), gate_cols])).to(torch.bfloat16)
    m, k = 16, 64
    a = torch.zeros((m, k), dtype=torch.float8_e4m3fn, device=dev)
    sa = torch.ones((m, 1), dtype=torch.float32, device=dev)
    w = torch.zeros((2 * f, k), dtype=torch.float8_e4m3fn, device=dev)
    sw = torch.ones((2 * f, 1), dtype=torch.float32, device=dev)
    h, _ = kernels.fp8_gemm_swiglu(a, sa, w, sw, m, bias.to(dev))
    got = h.float().cpu().numpy()[0, : gates.size]
    want = O.silu(gates)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert got[0] == np.inf and np.isnan(got[1]) and np.isnan(got[2])
    assert got[4] == 0.0 and np.signbit(got[4])



def test_portable_mode_keeps_torchs_scalar_division_on_the_gpu(dev):
    # One row per positive finite bf16 maximum.  The portable ("torch") mode is
    # the reference's expression amax / 448.0, which torch's GPU kernels
    # evaluate as amax * RN(1/448); the fused quantizer divides (IEEE), as the
    # reference's Triton kernel does with div_rn.  The two scales differ by one
    # ulp in 17410 of the 32639 maxima, and nowhere else.
    maxima = bf16_from_bits(np.arange(0x0001, 0x7F80, dtype=np.uint32).astype(np.uint16))
    x = np.zeros((maxima.size, 16), np.float32)
    x[:, 3] = maxima
    xd = torch.from_numpy(x).to(torch.bfloat16).to(dev)
    _, portable = _quantize_activation_torch(xd)
    _, fused = kernels.quantize_rows(xd)
    tiny = np.float32(np.finfo(np.float32).tiny)
    product = np.maximum((maxima * (np.float32(1.0) / np.float32(448.0))).astype(np.float32), tiny)
    quotient = np.maximum((maxima / np.float32(448.0)).astype(np.float32), tiny)
    rows = maxima.size
    assert np.array_equal(portable.reshape(-1)[:rows].cpu().numpy().view(np.uint32), product.view(np.uint32))
    assert np.array_equal(fused.reshape(-1)[:rows].cpu().numpy().view(np.uint32), quotient.view(np.uint32))
    assert int((product != quotient).sum()) == 17410


def test_oracle_restatement_rounds_like_the_oracle_on_the_device(dev):
    # oracle/fp8_torch.py checks full-size outputs on the device: its bf16
    # rounding must be the numpy oracle's there too, exact ties included.
    from oracle import formats as F
    from oracle import fp8_torch as T

    rng = np.random.default_rng(5)
    base = F.bf16_round(rng.standard_normal(50000) * np.exp2(rng.integers(-135, 120, 50000)))
    base = base[np.isfinite(base) & (base != 0)].astype(np.float64)
    half = np.exp2(np.floor(np.log2(np.abs(base))).clip(min=-126) - 8)
    x = np.concatenate([base + np.sign(base) * half, rng.standard_normal(50000), [0.0, -0.0]])
    got = T.bf16_round(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), F.bf16_round(x).view(np.uint32))
