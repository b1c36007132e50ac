"""The drop-in linear against the reference's own arithmetic call on this GPU.

The reference's W8A8 GEMM is ``torch._scaled_mm(codes, weight.t(), scale_a,
scale_b=scale.t(), out_dtype=bf16)`` followed by ``output[:rows] + bias``
(src/vflash/native/h3_fp8_linear.py:109-121); on ROCm torch runs it on
hipBLASLt with row-wise scales.  The same codes and scales go through both;
the sums differ only in accumulation order, so the results must agree to the
GEMM tolerance, and all but a few ties per hundred thousand must be identical
(measured: 99.999-100 %).
"""

import numpy as np
import pytest
import torch

from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def reference_call(codes, act_scale, weight, scale, bias, rows):
    """h3_fp8_linear.py:109-121, verbatim in its arguments."""
    output = torch._scaled_mm(codes, weight.t(), scale_a=act_scale, scale_b=scale.t(),
                              out_dtype=torch.bfloat16, use_fast_accum=False)
    if isinstance(output, tuple):
        output = output[0]
    output = output[:rows]
    return output if bias is None else output + bias


def inputs(m, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    codes, scale = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    return x, codes, scale, b


@pytest.mark.parametrize("m,k,n", [(4096, 3072, 3072), (1000, 1536, 4608), (256, 1536, 1536)])
def test_linear_matches_the_reference_scaled_mm_call(dev, m, k, n):
    x, codes, scale, b = inputs(m, k, n, seed=m + n)
    xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    ours = ex.linear(xd, cd, sd, bd)
    a, sa = kernels.quantize_rows(xd)  # the padded codes/scales the reference passes
    ref = reference_call(a, sa, cd, sd, bd, m)
    worst, exact = rel_check(ours.float().cpu().numpy(), ref.float().cpu().numpy())
    print(f"[{m}x{k}x{n}] identical {exact:.5f}, worst relative difference {worst:.3g}")
    assert exact > 0.999, f"only {exact:.5f} of the elements are identical"
    # Without bias the comparison is of the scaled sums alone.
    ref_nb = reference_call(a, sa, cd, sd, None, m)
    _, exact = rel_check(ex.linear(xd, cd, sd).float().cpu().numpy(), ref_nb.float().cpu().numpy())
    assert exact > 0.999


def test_metric_shape_matches_the_reference_scaled_mm_call(dev):
    # M=32760, K=5120, N=13824, compared on the device over every element.
    m, k, n = 32760, 5120, 13824
    x, codes, scale, b = inputs(m, k, n, seed=0)
    xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
    del x
    ours = RowFP8Execution("w8a8", activation_quantizer="triton").linear(xd, cd, sd, bd)
    a, sa = kernels.quantize_rows(xd)
    ref = reference_call(a, sa, cd, sd, bd, m)
    o, r = ours.float(), ref.float()
    rms = float(torch.sqrt(torch.mean(r * r)))
    err = (o - r).abs()
    bound = 1e-2 * r.abs() + 1e-2 * rms
    assert int((err > bound).sum()) <= r.numel() // 10000
    assert not bool((err > 2.0**-6 * r.abs() + 1e-2 * rms).any())
    exact = float((o == r).float().mean())
    print(f"[{m}x{k}x{n}] identical {exact:.5f}, max |diff| / (|ref| + rms) "
          f"{float((err / (r.abs() + rms)).max()):.3g}")
    assert exact > 0.999, f"only {exact:.5f} of the elements are identical"
    assert bool(torch.isfinite(o).all())
    np.testing.assert_array_equal(ours.shape, (m, n))


def reference_ffn(x, cu, su, bu, cd, sd, bd, gate, res, activation):
    """The reference FFN composition from torch operations on the same GPU:
    linear (h3_fp8_linear.py:109-121), the activation in eager bf16
    (GELU-tanh, or h3_native_denoiser.py:369-373 value * silu(gate)), the down
    linear's own per-token quantization, and the eager bf16 gate-residual
    (h3_fused_ops.py:153-170).  Returns the output, the down linear's input
    codes and row scales, and |residual| + |gate * z| (the magnitude of the
    final sum's addends)."""
    m = x.shape[0]
    a, sa = kernels.quantize_rows(x)  # the fused quantizer, the arithmetic of the reference's Triton kernel
    y = reference_call(a, sa, cu, su, bu, m)
    if activation == "swiglu":
        value, g = y.chunk(2, dim=-1)
        h = value * torch.nn.functional.silu(g)
    else:
        h = torch.nn.functional.gelu(y, approximate="tanh")
    hc, hs = kernels.quantize_rows(h.contiguous())
    z = reference_call(hc, hs, cd, sd, bd, m)
    gz = gate * z
    return res + gz, hc[:m], hs[:m], res.float().abs() + gz.float().abs()


@pytest.mark.parametrize("activation", ["gelu_tanh", "swiglu"])
@pytest.mark.parametrize("m,h,f", [(2048, 1024, 4096), (32760, 5120, 13824)])
def test_ffn_matches_the_reference_composition(dev, activation, m, h, f):
    from vflash_amd.fused import fp8_ffn

    up_rows = 2 * f if activation == "swiglu" else f
    g = torch.Generator().manual_seed(m + f)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(torch.randn((up_rows, h), generator=g) * 0.02)
    bu = (torch.randn(up_rows, generator=g) * 0.01).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand(h, generator=g).to(torch.bfloat16)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16)
    t = [v.to(dev) for v in (x, cu, su, bu, cd, sd, bd, gate, res)]
    xd, cud, sud, bud, cdd, sdd, bdd, gated, resd = t
    del x, res
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    ours = fp8_ffn(ex, *t, activation=activation)
    # The same launches staged, to read the down linear's input codes and scales.
    a, sa = kernels.quantize_rows(xd)
    if activation == "swiglu":
        hh, amax = kernels.fp8_gemm_swiglu(a, sa, cud, sud, m, bud)
        hc, hs = kernels.requant_rows(hh, amax)
        del amax
    else:
        hh = kernels.fp8_gemm(a, sa, cud, sud, m, bud)
        hc, hs, _ = kernels.gelu_quantize_rows(hh)
    assert torch.equal(kernels.fp8_gemm_gate_residual(hc, hs, cdd, sdd, m, gated, resd, bdd), ours)
    ref, ref_hc, ref_hs, addends = reference_ffn(*t, activation)
    del hh, a, sa
    # Error model.  The hidden activations differ from torch's where the two
    # up-projection sums round apart (about 1e-5 of the outputs) and where
    # torch's binary32 activation is not correctly rounded: its GELU loses
    # digits where 1 + tanh(u) cancels (y below about -2), and its exp and
    # quotient round within an ulp or so.  Requantization turns such a bf16 step
    # into a re-rounded E4M3 code, or, at a row's maximum, a new row scale.  Those input
    # differences reach z through the down weights exactly:
    #   |dz| <= (|dequant(ours) - dequant(ref)| . |W_down|^T) * s_down,
    # and z enters the output as gate * z.  Beyond that propagated bound, the
    # output must meet the GEMM tolerance relative to the magnitude of the final
    # sum's addends |residual| + |gate * z| (the result itself may cancel).
    dq = (hc[:m].float() * hs[:m] - ref_hc.float() * ref_hs).abs_()
    wd = cdd.float().abs_()
    propagated = torch.matmul(dq, wd.t().contiguous()) * sdd.reshape(1, -1)
    propagated *= gated.float().reshape(1, -1)
    del dq, wd
    o, r = ours.float(), ref.float()
    rms = float(torch.sqrt(torch.mean(r * r)))
    err = (o - r).abs_()
    slack = err - propagated
    assert int((slack > 1e-2 * addends + 1e-2 * rms).sum()) <= r.numel() // 10000
    assert not bool((slack > 2.0**-6 * addends + 1e-2 * rms).any())
    rows_moved = float((hc[:m] != ref_hc).any(dim=1).float().mean())
    codes_moved = float((hc[:m] != ref_hc).float().mean())
    exact = float((o == r).float().mean())
    print(f"[{activation} {m}x{h}x{f}] identical {exact:.5f}; requantization codes differing "
          f"{codes_moved:.2e} (in {rows_moved:.3f} of the rows); max (|diff| - propagated) / "
          f"(addends + rms) {float((slack / (addends + rms)).max()):.3g}")
    # Measured at the full shape: 1.69e-5 (GELU: torch's binary32 1 + tanh(u)
    # cancels at negative inputs, where the kernel's correctly rounded GELU
    # differs from it) and 6.4e-7 (SwiGLU).
    assert exact > 0.9 and codes_moved < (2e-5 if activation == "gelu_tanh" else 1e-6)


def test_merged_qkv_planes_match_the_reference_call(dev):
    # X [32760, 5120] against cat(Wq, Wk, Wv) [15360, 5120]: the reference makes
    # one linear call and chunks it (h3_reference_execution.py:161-192); the
    # planes here are written by the epilogue.
    from vflash_amd.fused import merge_qkv, qkv_linear

    m, hidden, inner = 32760, 5120, 5120
    g = torch.Generator().manual_seed(3)
    x = torch.randn((m, hidden), generator=g).to(torch.bfloat16).to(dev)
    parts = [quantize_weight_rows(torch.randn((inner, hidden), generator=g) * 0.02) for _ in range(3)]
    b = (torch.randn(3 * inner, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    w, s = merge_qkv([p[0].to(dev) for p in parts], [p[1].to(dev) for p in parts])
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    planes = qkv_linear(ex, x, w, s, b, planes=True)
    a, sa = kernels.quantize_rows(x)
    ref = reference_call(a, sa, w, s, b, m).chunk(3, dim=-1)
    for name, got, want in zip("qkv", planes, ref):
        o, r = got.float(), want.float()
        rms = float(torch.sqrt(torch.mean(r * r)))
        err = (o - r).abs()
        assert int((err > 1e-2 * r.abs() + 1e-2 * rms).sum()) <= r.numel() // 10000
        assert not bool((err > 2.0**-6 * r.abs() + 1e-2 * rms).any())
        exact = float((o == r).float().mean())
        print(f"[qkv {name} 32760x5120x5120] identical {exact:.5f}")
        assert exact > 0.999


@pytest.mark.parametrize("m", [256, 512, 1024])
@pytest.mark.parametrize("n", [1536, 4608, 6144])
def test_lora_linear_matches_the_reference_hook(dev, m, n):
    # The adapter hook of h3_reference_lora.py:75-90 on the reference linear:
    # delta = F.linear(F.linear(x, A), B) in bf16, * scaling, * strength (each
    # rounded), result + delta.
    from vflash_amd.fused import fp8_linear_lora

    k, rank, scaling, strength = 1536, 32, 0.5, 1.375
    x, codes, scale, b = inputs(m, k, n, seed=m * n)
    g = torch.Generator().manual_seed(m + n + 1)
    la = (torch.randn((rank, k), generator=g) * 0.01).to(torch.bfloat16).to(dev)
    lb = (torch.randn((n, rank), generator=g) * 0.01).to(torch.bfloat16).to(dev)
    xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    ours = fp8_linear_lora(ex, xd, cd, sd, bd, la, lb, scaling=scaling, strength=strength)
    a, sa = kernels.quantize_rows(xd)
    result = reference_call(a, sa, cd, sd, bd, m)
    delta = torch.nn.functional.linear(torch.nn.functional.linear(xd, la), lb).to(result.dtype)
    delta = delta * scaling
    delta = delta * strength
    ref = result + delta
    worst, exact = rel_check(ours.float().cpu().numpy(), ref.float().cpu().numpy())
    print(f"[lora {m}x{k}x{n}] identical {exact:.5f}, worst relative difference {worst:.3g}")
    assert exact > 0.999
