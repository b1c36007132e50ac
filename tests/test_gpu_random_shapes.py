"""Seeded random shapes through every GEMM epilogue and the NVFP4 GEMMs: each
FP8 output within the tolerance of the oracle's rounding chain (its torch
restatement, binary64 sums on the device), and every call split at a row
bit-identical to the whole call.  The shapes sweep M from 1 to several thousand rows and N and K
over multiples of 16, so every tiling the shape rule picks, partial tiles in
both directions and the multi-round grids all run."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from oracle import fp8_torch as T
from oracle import nvfp4 as N
from tests.conftest import rel_check, rel_check_device
from vflash_amd import kernels
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def shapes(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        m = int(rng.choice([1, 7, 16, 63, 200, 777, 1500, 4100, 9000]))
        n = 16 * int(rng.integers(1, 400))
        k = 16 * int(rng.integers(1, 200))
        out.append((m, n, k))
    return out


def operands(dev, m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    cw, sw = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.05)
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    return x, cw.to(dev), sw.to(dev), bias


def split_equal(run, m, split):
    """run(lo, hi) computes rows [lo, hi); the two parts must equal the whole."""
    whole = run(0, m)
    if 0 < split < m:
        parts = torch.cat([run(0, split), run(split, m)])
        assert torch.equal(parts, whole)
    return whole


@pytest.mark.parametrize("m,n,k", shapes(5, 12))
def test_linear_bias_random_shape(dev, m, n, k):
    x, cw, sw, bias = operands(dev, m, n, k, m + n + k)
    codes, sa = kernels.quantize_rows(x)
    ref_codes, ref_sa = T.quantize_rows(x)
    assert torch.equal(codes.view(torch.uint8), ref_codes) and torch.equal(sa.reshape(-1), ref_sa)

    def run(lo, hi):
        c, s = kernels.quantize_rows(x[lo:hi])
        return kernels.fp8_gemm(c, s, cw, sw, hi - lo, bias)

    out = split_equal(run, m, max(1, m // 3))
    want = T.add_bias(T.scaled_mm(ref_codes[:m], ref_sa[:m], cw.view(torch.uint8), sw), bias)
    rel_check_device(out, want)


@pytest.mark.parametrize("m,n,k", shapes(6, 8))
@pytest.mark.parametrize("gate_form", ["per_row", "broadcast", "one_row"])
def test_gate_residual_random_shape(dev, m, n, k, gate_form):
    # Per-row gates [m, n], and the one-row forms [n] and [1, n] (loaded once
    # per thread in whole tiles).
    x, cw, sw, bias = operands(dev, m, n, k, 3 * m + n + k)
    g = torch.Generator().manual_seed(m + 2 * n)
    res = torch.randn((m, n), generator=g).to(torch.bfloat16).to(dev)
    rows = {"per_row": m, "broadcast": 1, "one_row": 1}[gate_form]
    gate = torch.rand((rows, n), generator=g).to(torch.bfloat16).to(dev)
    if gate_form == "broadcast":
        gate = gate[0]

    def run(lo, hi):
        c, s = kernels.quantize_rows(x[lo:hi])
        gt = gate[lo:hi] if gate_form == "per_row" else gate
        return kernels.fp8_gemm_gate_residual(c, s, cw, sw, hi - lo, gt, res[lo:hi], bias)

    out = split_equal(run, m, max(1, m // 2))
    codes, sa = T.quantize_rows(x)
    y = T.add_bias(T.scaled_mm(codes[:m], sa[:m], cw.view(torch.uint8), sw), bias)
    # The projection is within the GEMM tolerance; the epilogue on the kernel's
    # own projection is bit-exact.
    c, s = kernels.quantize_rows(x)
    y_k = kernels.fp8_gemm(c, s, cw, sw, m, bias)
    rel_check_device(y_k, y)
    full_gate = gate.reshape(-1, n).expand(m, n)
    assert torch.equal(out, T.gate_residual(res, full_gate, y_k).to(torch.bfloat16))


@pytest.mark.parametrize("m,n,k", shapes(7, 8))
@pytest.mark.parametrize("rank", [16, 48])
def test_lora_random_shape(dev, m, n, k, rank):
    x, cw, sw, bias = operands(dev, m, n, k, 5 * m + n + k + rank)
    g = torch.Generator().manual_seed(m + 7 * n + rank)
    la = (torch.randn((rank, k), generator=g) * 0.05).to(torch.bfloat16).to(dev)
    lb = (torch.randn((n, rank), generator=g) * 0.05).to(torch.bfloat16).to(dev)

    def run(lo, hi):
        c, s = kernels.quantize_rows(x[lo:hi])
        t = kernels.lora_down(x[lo:hi], la)
        return kernels.fp8_gemm_lora(c, s, cw, sw, hi - lo, t, lb, scale=0.5, strength=1.25,
                                     bias=bias)

    out = split_equal(run, m, max(1, (2 * m) // 3))
    # The fused quantization + down-projection gives the separate kernels' bits.
    if kernels.quantize_lora_supported(k, rank):
        c2, s2, t2 = kernels.quantize_rows_lora(x, la)
        c1, s1 = kernels.quantize_rows(x)
        assert torch.equal(c2.view(torch.uint8), c1.view(torch.uint8)) and torch.equal(s2, s1)
        assert torch.equal(t2, kernels.lora_down(x, la))
    # Within tolerance of the whole chain in binary64: base + bf16 rounded delta.
    codes, sa = T.quantize_rows(x)
    base = T.add_bias(T.scaled_mm(codes[:m], sa[:m], cw.view(torch.uint8), sw), bias)
    t = T.bf16_round(x.double() @ la.double().T)
    delta = T.bf16_round(T.bf16_round(T.bf16_round(t.double() @ lb.double().T).double() * 0.5)
                         .double() * 1.25)
    want = T.bf16_round(base.double() + delta.double())
    rel_check_device(out, want)


def shapes_multiple(seed, count, n_unit, k_unit, n_max, k_max):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        m = int(rng.choice([1, 7, 63, 200, 777, 1500, 4100, 9000]))
        out.append((m, n_unit * int(rng.integers(1, n_max // n_unit + 1)),
                    k_unit * int(rng.integers(1, k_max // k_unit + 1))))
    return out


@pytest.mark.parametrize("m,n,k", shapes_multiple(8, 8, 256, 16, 8192, 3072))
def test_swiglu_random_shape(dev, m, n, k):
    x, cw, sw, bias = operands(dev, m, n, k, 7 * m + n + k)

    def run(lo, hi):
        c, s = kernels.quantize_rows(x[lo:hi])
        h, amax = kernels.fp8_gemm_swiglu(c, s, cw, sw, hi - lo, bias)
        return torch.cat([h.float(), amax], dim=1)

    out = split_equal(run, m, max(1, m // 4))
    f = n // 2
    h, amax = out[:, :f], out[:, f:]
    # The row maxima per 128 columns are those of the kernel's own h.
    assert torch.equal(amax, h.abs().reshape(m, -1, 128).amax(dim=2))
    # The SwiGLU tile's packed projection is the plain GEMM's on the same codes
    # (same K order, same epilogue rounding), within the GEMM tolerance of the
    # oracle; h is the oracle's SwiGLU of that projection bit for bit.
    c, s = kernels.quantize_rows(x)
    packed = kernels.fp8_gemm(c, s, cw, sw, m, bias)
    codes, sa = T.quantize_rows(x)
    rel_check_device(packed, T.add_bias(T.scaled_mm(codes[:m], sa[:m], cw.view(torch.uint8), sw),
                                        bias))
    assert torch.equal(h, T.silu_mul(packed))


@pytest.mark.parametrize("m,n,k", shapes_multiple(9, 6, 48, 16, 6144, 2048))
def test_planes_random_shape(dev, m, n, k):
    x, cw, sw, bias = operands(dev, m, n, k, 11 * m + n + k)
    c, s = kernels.quantize_rows(x)
    whole = kernels.fp8_gemm(c, s, cw, sw, m, bias)

    def run(lo, hi):
        cc, ss = kernels.quantize_rows(x[lo:hi])
        return kernels.fp8_gemm_planes(cc, ss, cw, sw, hi - lo, 3, bias).permute(1, 0, 2)

    planes = split_equal(run, m, max(1, m // 3))
    assert torch.equal(planes.reshape(m, n), whole)


@pytest.mark.parametrize("m,n,k", shapes_multiple(10, 6, 128, 64, 4096, 4096))
def test_nvfp4_random_shape(dev, m, n, k):
    from vflash_amd.prepare import quantize_nvfp4_weight

    g = torch.Generator().manual_seed(13 * m + n + k)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    packed, scales, alpha, _ = quantize_nvfp4_weight((torch.randn((n, k), generator=g) * 0.05).to(dev))
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    gsf = torch.tensor(2688.0 / float(x.float().abs().amax()), device=dev)

    def w4a8(lo, hi):
        c, s = kernels.quantize_rows(x[lo:hi])
        return kernels.nvfp4_gemm(c, s, packed, scales, alpha, hi - lo, bias)

    def w4a4(lo, hi):
        c, s = kernels.nvfp4_quantize_rows(x[lo:hi], gsf)
        return kernels.nvfp4_w4a4_gemm(c, s, packed, scales, alpha / gsf, hi - lo, bias)

    o8 = split_equal(w4a8, m, max(1, m // 2))
    o4 = split_equal(w4a4, m, max(1, m // 3))
    # Sampled rows against the oracle (exact sums of the dequantized operands).
    rows = np.unique(np.r_[0:16, m // 2 : m // 2 + 16, max(m - 16, 0) : m].clip(0, m - 1))
    xs = x.float().cpu().numpy()[rows]
    pk, sc, b = packed.cpu().numpy(), scales.cpu().numpy(), bias.float().cpu().numpy()
    codes, sa = O.quantize_rows(xs, pad=1)
    rel_check(o8.float().cpu().numpy()[rows], N.linear(codes, sa, pk, sc, float(alpha), b))
    a4, s4 = N.quantize_activation(xs, float(gsf))
    out_scale = np.float32(float(alpha)) / np.float32(float(gsf))  # one fp32 division, as on the device
    rel_check(o4.float().cpu().numpy()[rows], N.linear_w4a4(a4, s4, pk, sc, out_scale, b))
