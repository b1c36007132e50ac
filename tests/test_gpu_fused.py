"""Merged QKV, the GELU-tanh and SwiGLU FFN chains and the LoRA linear on gfx950 vs the oracle."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from tests.conftest import rel_check, rel_check_device
from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution, RowFP8Linear
from vflash_amd.fused import FusedQKV, fp8_ffn, fp8_linear_lora, merge_qkv, qkv_linear
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def qkv_inputs(m, hidden, inner, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
    parts = [quantize_weight_rows(torch.randn((inner, hidden), generator=g) * 0.02) for _ in range(3)]
    return x, parts


def test_merged_qkv_is_bit_identical_to_three_separate_linears(dev):
    x, parts = qkv_inputs(300, 512, 256)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    xd = x.to(dev)
    w, s = merge_qkv([p[0].to(dev) for p in parts], [p[1].to(dev) for p in parts])
    q, k, v = qkv_linear(ex, xd, w, s)
    sep = [ex.linear(xd, c.to(dev), sc.to(dev)) for c, sc in parts]
    for got, ref in zip((q, k, v), sep):
        assert torch.equal(got, ref)
    # Plane layout: same values, three contiguous [rows, inner] planes.
    qp, kp, vp = qkv_linear(ex, xd, w, s, planes=True)
    for got, ref in zip((qp, kp, vp), sep):
        assert got.is_contiguous() and torch.equal(got, ref)
    assert qp.data_ptr() + qp.numel() * 2 == kp.data_ptr()


def test_merged_qkv_config_shape_sampled(dev):
    # X [32760, 5120]; W [3*5120, 5120]; output planes Q/K/V [32760, 40, 128].
    x, parts = qkv_inputs(32760, 5120, 5120)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    w, s = merge_qkv([p[0] for p in parts], [p[1] for p in parts])
    b = (torch.randn(15360, generator=torch.Generator().manual_seed(7)) * 0.01).to(torch.bfloat16)
    q, k, v = qkv_linear(ex, x.to(dev), w.to(dev), s.to(dev), b.to(dev), planes=True)
    heads = [t.view(32760, 40, 128) for t in (q, k, v)]
    rows = np.r_[0:16, 20000:20016, 32744:32760]
    ref = O.w8a8_linear(x.float().numpy()[rows], u8(w), s.reshape(-1).numpy(), b.float().numpy())
    got = np.concatenate([h.reshape(32760, 5120).float().cpu().numpy()[rows] for h in heads], axis=1)
    rel_check(got, ref)


def test_merged_qkv_config_shape_every_element(dev):
    # All 503 million outputs of the three planes against the oracle's chain
    # restated in torch on the device (oracle/fp8_torch.py).
    from oracle import fp8_torch as T

    x, parts = qkv_inputs(32760, 5120, 5120)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    w, s = merge_qkv([p[0] for p in parts], [p[1] for p in parts])
    b = (torch.randn(15360, generator=torch.Generator().manual_seed(7)) * 0.01).to(torch.bfloat16)
    xd, wd, sd, bd = x.to(dev), w.to(dev), s.to(dev), b.to(dev)
    q, k, v = qkv_linear(ex, xd, wd, sd, bd, planes=True)
    ref = T.w8a8_linear(xd, wd, sd, bd)
    for i, plane in enumerate((q, k, v)):
        worst, exact = rel_check_device(plane, ref[:, 5120 * i:5120 * (i + 1)])
        print(f"[qkv plane {i}] identical {exact:.6f}, worst {worst:.3g}")
        assert exact > 0.95, (i, exact, worst)


def test_fused_qkv_module_checks_its_parts(dev):
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    mods = []
    x, parts = qkv_inputs(64, 128, 64)
    for c, s in parts:
        mod = RowFP8Linear(torch.nn.Linear(128, 64, bias=False), ex)
        mod.load_state_dict({"weight": c.to(dev), "row_scale": s.to(dev)}, assign=True)
        mods.append(mod)
    fused = FusedQKV(*mods)
    out = fused(x.to(dev))
    for got, mod in zip(out, mods):
        assert torch.equal(got, mod(x.to(dev)))
    other = RowFP8Linear(torch.nn.Linear(128, 64, bias=False), RowFP8Execution("w8a8"))
    other.load_state_dict({"weight": parts[0][0].to(dev), "row_scale": parts[0][1].to(dev)}, assign=True)
    with pytest.raises(ValueError, match="matching"):
        FusedQKV(mods[0], mods[1], other)


def ffn_inputs(m, h, f, seed=0, token_gate=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    wu, bu = torch.randn((f, h), generator=g) * 0.02, (torch.randn(f, generator=g) * 0.01).to(torch.bfloat16)
    wd, bd = torch.randn((h, f), generator=g) * 0.02, (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand((m, h) if token_gate else (h,), generator=g).to(torch.bfloat16)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(wu)
    cd, sd = quantize_weight_rows(wd)
    return x, cu, su, bu, cd, sd, bd, gate, res


@pytest.mark.parametrize("m,h,f,token_gate", [(300, 512, 1024, False), (77, 256, 768, True)])
def test_ffn_chain_stages_against_the_oracle(dev, m, h, f, token_gate):
    x, cu, su, bu, cd, sd, bd, gate, res = ffn_inputs(m, h, f, token_gate=token_gate)
    d = lambda t: t.to(dev)
    a, sa = kernels.quantize_rows(d(x))
    # Stage 1: the up linear, against the oracle within the GEMM tolerance.
    y = kernels.fp8_gemm(a, sa, d(cu), d(su), m, d(bu))
    y_np = y.float().cpu().numpy()
    rel_check(y_np, O.w8a8_linear(x.float().numpy(), u8(cu), su.reshape(-1).numpy(), bu.float().numpy()))
    # Stage 2: GELU-tanh and the requantization, bit-exact against the oracle on
    # the kernel's own y.
    hc, hs, g = kernels.gelu_quantize_rows(y, keep_values=True)
    g_np = g.float().cpu().numpy()
    assert np.array_equal(g_np.view(np.uint32), O.gelu_tanh(y_np).view(np.uint32))
    rc, rs = O.quantize_rows(g_np)
    assert np.array_equal(u8(hc), rc) and np.array_equal(hs.reshape(-1).cpu().numpy(), rs)
    assert torch.equal(kernels.gelu_quantize_rows(y)[0], hc)  # the values are optional
    # Stage 3: down projection with gate-residual epilogue, against the oracle on the same codes.
    out = kernels.fp8_gemm_gate_residual(hc, hs, d(cd), d(sd), m, d(gate), d(res), d(bd))
    y = O.add_bias(O.scaled_mm(rc[:m], rs[:m], u8(cd), sd.reshape(-1).numpy()), bd.float().numpy())
    ref = O.gate_residual(res.float().numpy(), gate.float().numpy(), y)
    rel_check(out.float().cpu().numpy(), ref)
    # Whole chain through the module-level composition vs the oracle chain.
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    full = fp8_ffn(ex, d(x), d(cu), d(su), d(bu), d(cd), d(sd), d(bd), d(gate), d(res))
    assert torch.equal(full, out)
    *_, chain = O.ffn(x.float().numpy(), u8(cu), su.reshape(-1).numpy(), bu.float().numpy(),
                      u8(cd), sd.reshape(-1).numpy(), bd.float().numpy(), gate.float().numpy(),
                      res.float().numpy())
    assert chain_error(full.float().cpu().numpy(), chain) <= 1e-2
    assert ex.calls["w8a8"] == 2


def chain_error(got, ref):
    """Norm-wise relative error of a two-GEMM chain.

    Elementwise parity is asserted per stage (the requantization is bit-exact
    on the kernel's own GELU output); against an independently computed chain
    an ulp-level difference upstream flips individual E4M3 codes, so the chain
    as a whole is compared in the Frobenius norm.
    """
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def test_ffn_config_shape_sampled(dev):
    # X [32760, 5120]; up [13824, 5120]; down [5120, 13824]; gate [5120] ~U(0,1).
    m, h, f = 32760, 5120, 13824
    x, cu, su, bu, cd, sd, bd, gate, res = ffn_inputs(m, h, f)
    d = lambda t: t.to(dev)
    a, sa = kernels.quantize_rows(d(x))
    y = kernels.fp8_gemm(a, sa, d(cu), d(su), m, d(bu))
    hc, hs, g = kernels.gelu_quantize_rows(y, keep_values=True)
    out = kernels.fp8_gemm_gate_residual(hc, hs, d(cd), d(sd), m, d(gate), d(res), d(bd))
    rows = np.r_[0:8, 16380:16388, 32752:32760]
    xs = x.float().numpy()[rows]
    # Stage 1 within tolerance; stage 2 (GELU and requantization) bit-exact on
    # every row of the kernel's own y.
    y_np = y.float().cpu().numpy()
    rel_check(y_np[rows], O.w8a8_linear(xs, u8(cu), su.reshape(-1).numpy(), bu.float().numpy()))
    g_all = O.gelu_tanh(y_np)
    assert np.array_equal(g.float().cpu().numpy().view(np.uint32), g_all.view(np.uint32))
    del y_np
    rc_all, rs_all = O.quantize_rows(g_all)
    assert np.array_equal(u8(hc), rc_all) and np.array_equal(hs.reshape(-1).cpu().numpy(), rs_all)
    rc, rs = rc_all[rows], rs_all[rows]
    del g_all, rc_all
    # Stage 3 within tolerance on the same codes.
    y = O.add_bias(O.scaled_mm(rc, rs, u8(cd), sd.reshape(-1).numpy()), bd.float().numpy())
    got = out.float().cpu().numpy()[rows]
    rel_check(got, O.gate_residual(res.float().numpy()[rows], gate.float().numpy(), y))
    # The whole chain against an independent oracle chain.
    *_, chain = O.ffn(xs, u8(cu), su.reshape(-1).numpy(), bu.float().numpy(), u8(cd),
                      sd.reshape(-1).numpy(), bd.float().numpy(), gate.float().numpy(),
                      res.float().numpy()[rows])
    assert chain_error(got, chain) <= 1e-2


def test_ffn_config_shape_every_element(dev):
    # Every element of every stage at M=32760, 5120 -> 13824 -> 5120, against
    # the oracle's chain restated in torch (oracle/fp8_torch.py): the up and down
    # linears within the GEMM tolerance, GELU, the requantization and the
    # gate-residual epilogue bit-exact on the kernel's own inputs to them.
    from oracle import fp8_torch as T

    m, h, f = 32760, 5120, 13824
    x, cu, su, bu, cd, sd, bd, gate, res = ffn_inputs(m, h, f)
    d = lambda t: t.to(dev)
    xd, cud, sud, bud, cdd, sdd, bdd, gd, rd = map(d, (x, cu, su, bu, cd, sd, bd, gate, res))
    a, sa = kernels.quantize_rows(xd)
    y = kernels.fp8_gemm(a, sa, cud, sud, m, bud)
    worst, exact = rel_check_device(y, T.w8a8_linear(xd, cud, sud, bud))
    print(f"identical {exact:.6f}, worst {worst:.3g}")
    assert exact > 0.95, (exact, worst)
    hc, hs, g = kernels.gelu_quantize_rows(y, keep_values=True)
    g_ref = T.gelu_tanh(y)
    assert torch.equal(g.float().view(torch.int32), g_ref.view(torch.int32))
    rc, rs = T.quantize_rows(g_ref)
    assert torch.equal(hc.view(torch.uint8), rc) and torch.equal(hs.reshape(-1), rs)
    del g, g_ref
    check_down_projection(hc, hs, cdd, sdd, m, gd, rd, bdd)


def check_down_projection(hc, hs, cd, sd, m, gate, res, bias):
    """The output projection with its gate-residual epilogue at every element:
    the projection (the plain bias epilogue on the same codes runs the same MFMA
    chain) within the GEMM tolerance of the restated oracle, and the epilogue
    bit-exact against the oracle's gate-residual rounding chain applied to it.
    (The residual sum can cancel, so a tolerance relative to the final output
    would not bound the projection.)"""
    from oracle import fp8_torch as T

    out = kernels.fp8_gemm_gate_residual(hc, hs, cd, sd, m, gate, res, bias)
    y = kernels.fp8_gemm(hc, hs, cd, sd, m, bias)
    worst, exact = rel_check_device(y, T.add_bias(T.scaled_mm(hc[:m], hs[:m], cd, sd), bias))
    print(f"down projection identical {exact:.6f}, worst {worst:.3g}")
    assert exact > 0.95, (exact, worst)
    assert torch.equal(out.float().view(torch.int32), T.gate_residual(res, gate, y).view(torch.int32))


def test_swiglu_h3_shape_every_element(dev):
    # The H3 feed-forward (hidden 5376, inner 14336) at 32760 tokens: the SwiGLU
    # tile's output against SwiGLU of the restated oracle linear (value and gate
    # each within the GEMM bound, composed through one product), the row maxima
    # and the requantization exact on the kernel's own h, and the output
    # projection with its gate-residual within the GEMM tolerance.
    from oracle import fp8_torch as T

    m, h, f = 32760, 5376, 14336
    g = torch.Generator().manual_seed(3)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(torch.randn((2 * f, h), generator=g) * 0.02)
    bu = (torch.randn(2 * f, generator=g) * 0.01).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand(h, generator=g).to(torch.bfloat16)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    xd, cud, sud, bud, cdd, sdd, bdd, gd, rd = map(d, (x, cu, su, bu, cd, sd, bd, gate, res))
    a, sa = kernels.quantize_rows(xd)
    hh, amax = kernels.fp8_gemm_swiglu(a, sa, cud, sud, m, bud)
    # The SwiGLU tile's packed projection is the plain GEMM's on the same codes
    # (same K order and epilogue), within the GEMM tolerance of the oracle at
    # every element; h is the oracle's SwiGLU of that projection bit for bit.
    packed = kernels.fp8_gemm(a, sa, cud, sud, m, bud)
    worst, exact = rel_check_device(packed, T.w8a8_linear(xd, cud, sud, bud))
    print(f"packed projection identical {exact:.6f}, worst {worst:.3g}")
    assert torch.equal(hh.float(), T.silu_mul(packed))
    del packed
    assert torch.equal(amax, hh.float().abs().reshape(m, -1, 128).amax(dim=2))
    hc, hs = kernels.requant_rows(hh, amax)
    rc, rs = T.quantize_rows(hh)
    assert torch.equal(hc.view(torch.uint8), rc) and torch.equal(hs.reshape(-1), rs)
    check_down_projection(hc, hs, cdd, sdd, m, gd, rd, bdd)


@pytest.mark.parametrize("m,h,f,token_gate", [(300, 512, 512, False), (77, 256, 384, True)])
def test_swiglu_ffn_chain_stages_against_the_oracle(dev, m, h, f, token_gate):
    # H3 FFN: packed input projection [2F, H] (values, then gates), SwiGLU, requant,
    # output projection [H, F] with the gate-residual epilogue.
    x, cu, su, bu, cd, sd, bd, gate, res = ffn_inputs(m, h, 2 * f, token_gate=token_gate)
    # The output projection maps the F activations back to H.
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=torch.Generator().manual_seed(9)) * 0.02)
    d = lambda t: t.to(dev)
    a, sa = kernels.quantize_rows(d(x))
    hh, amax = kernels.fp8_gemm_swiglu(a, sa, d(cu), d(su), m, d(bu))
    h_np = hh.float().cpu().numpy()
    # Stage 1a: the packed projection inside the SwiGLU tile equals the plain
    # linear (same K order), so SwiGLU of the plain kernel's output pins the
    # epilogue bit for bit.
    packed = kernels.fp8_gemm(a, sa, d(cu), d(su), m, d(bu)).float().cpu().numpy()
    ref_h = O.silu_mul(packed)
    assert np.array_equal(h_np.view(np.uint32), ref_h.view(np.uint32))
    # Stage 1b: the packed projection against the oracle (tolerance), and SwiGLU of it.
    ref_lin = O.w8a8_linear(x.float().numpy(), u8(cu), su.reshape(-1).numpy(), bu.float().numpy())
    rel_check(packed, ref_lin)
    # Row maxima: exact maxima of |h| per 128-column group.
    assert np.array_equal(amax.cpu().numpy(), np.abs(h_np).reshape(m, -1, 128).max(axis=2))
    # Stage 2: requantization bit-exact on the kernel's own h.
    hc, hs = kernels.requant_rows(hh, amax)
    rc, rs = O.quantize_rows(h_np)
    assert np.array_equal(u8(hc), rc) and np.array_equal(hs.reshape(-1).cpu().numpy(), rs)
    # Stage 3: output projection with gate-residual on the same codes.
    out = kernels.fp8_gemm_gate_residual(hc, hs, d(cd), d(sd), m, d(gate), d(res), d(bd))
    y = O.add_bias(O.scaled_mm(rc[:m], rs[:m], u8(cd), sd.reshape(-1).numpy()), bd.float().numpy())
    rel_check(out.float().cpu().numpy(), O.gate_residual(res.float().numpy(), gate.float().numpy(), y))
    # Whole chain through the module-level composition vs the oracle chain.
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    full = fp8_ffn(ex, d(x), d(cu), d(su), d(bu), d(cd), d(sd), d(bd), d(gate), d(res),
                   activation="swiglu")
    assert torch.equal(full, out)
    *_, chain = O.ffn(x.float().numpy(), u8(cu), su.reshape(-1).numpy(), bu.float().numpy(),
                      u8(cd), sd.reshape(-1).numpy(), bd.float().numpy(), gate.float().numpy(),
                      res.float().numpy(), activation="swiglu")
    assert chain_error(full.float().cpu().numpy(), chain) <= 1e-2


def test_swiglu_h3_shape_sampled(dev):
    # H3 feed-forward: hidden 5376, inner 14336 (packed input projection [28672, 5376]).
    m, h, f = 32760, 5376, 14336
    g = torch.Generator().manual_seed(3)
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(torch.randn((2 * f, h), generator=g) * 0.02)
    bu = (torch.randn(2 * f, generator=g) * 0.01).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    a, sa = kernels.quantize_rows(d(x))
    hh, amax = kernels.fp8_gemm_swiglu(a, sa, d(cu), d(su), m, d(bu))
    rows = np.r_[0:8, 16380:16388, 32752:32760]
    h_np = hh.float().cpu().numpy()[rows]
    # The packed projection (the plain GEMM on the same codes) within the GEMM
    # tolerance of the oracle; h its SwiGLU bit for bit.
    packed = kernels.fp8_gemm(a, sa, d(cu), d(su), m, d(bu)).float().cpu().numpy()[rows]
    ref_lin = O.w8a8_linear(x.float().numpy()[rows], u8(cu), su.reshape(-1).numpy(), bu.float().numpy())
    rel_check(packed, ref_lin)
    assert np.array_equal(h_np.view(np.uint32), O.silu_mul(packed).view(np.uint32))
    assert np.array_equal(amax.cpu().numpy()[rows], np.abs(h_np).reshape(len(rows), -1, 128).max(axis=2))
    assert bool(torch.isfinite(hh.float()).all())


@pytest.mark.parametrize("m", [256, 512, 1024])
@pytest.mark.parametrize("n", [1536, 4608, 6144])
@pytest.mark.parametrize("scaling,strength", [(1.0, 1.0), (0.5, 1.375)])
def test_lora_linear_skinny_shapes(dev, m, n, scaling, strength):
    # Every skinny audio-stream shape: M in {256, 512, 1024} x N in {1536, 4608, 6144}, K 1536.
    k, r = 1536, 32
    g = torch.Generator().manual_seed(m + n)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
    lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    out = fp8_linear_lora(ex, d(x), d(c), d(s), d(b), d(la), d(lb), scaling=scaling, strength=strength)
    xf = x.float().numpy()
    t = kernels.lora_down(d(x), d(la)).float().cpu().numpy()
    rel_check(t, O.lora_delta(xf, la.float().numpy(), np.eye(r, dtype=np.float32)))
    base = O.w8a8_linear(xf, u8(c), s.reshape(-1).numpy(), b.float().numpy())
    delta = O.lora_delta(xf, la.float().numpy(), lb.float().numpy(), scaling, strength)
    rel_check(out.float().cpu().numpy(), O.lora_merge(base, delta))
    # Strength 0 disables the adapter (reference hook returns the result unchanged).
    off = fp8_linear_lora(ex, d(x), d(c), d(s), d(b), d(la), d(lb), strength=0.0)
    assert torch.equal(off, ex.linear(d(x), d(c), d(s), d(b)))


@pytest.mark.parametrize("m", [256, 1024])
@pytest.mark.parametrize("r,scaling,strength", [(128, 1.0, 1.0), (16, 0.5, 1.375)])
def test_lora_linear_audio_projection_shapes(dev, m, r, scaling, strength):
    # The audio pass's separate Q/K/V projections: hidden 5376 -> inner 7168 on
    # the live rows, with the shipped adapters' ranks (128 and 16).
    k, n = 5376, 7168
    g = torch.Generator().manual_seed(m * 3 + r)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
    lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")
    out = fp8_linear_lora(ex, d(x), d(c), d(s), d(b), d(la), d(lb), scaling=scaling, strength=strength)
    xf = x.float().numpy()
    t = kernels.lora_down(d(x), d(la)).float().cpu().numpy()
    rel_check(t, O.lora_delta(xf, la.float().numpy(), np.eye(r, dtype=np.float32)))
    base = O.w8a8_linear(xf, u8(c), s.reshape(-1).numpy(), b.float().numpy())
    delta = O.lora_delta(xf, la.float().numpy(), lb.float().numpy(), scaling, strength)
    rel_check(out.float().cpu().numpy(), O.lora_merge(base, delta))
    # The base linear alone, as the hook sees it before the delta.
    base_dev = ex.linear(d(x), d(c), d(s), d(b)).float().cpu().numpy()
    rel_check(base_dev, base)


# Tilings with at most eight 32x32 blocks per wave compute the adapter products
# ahead of the K loop (64x64: 300 x 640, 128x64: 300 x 4112, 128x128:
# 2100 x 3712, 128x192: 1024 x 6144, 256x128: 1024 x 7168), the others in the
# epilogue (256x192: 4096 x 3072, 256x256: 4100 x 3088).
@pytest.mark.parametrize("r", [32, 48, 128])
@pytest.mark.parametrize("m,n,k", [(300, 640, 512), (300, 4112, 512), (2100, 3712, 384),
                                   (1024, 6144, 1536), (1024, 7168, 512), (4096, 3072, 1536),
                                   (4100, 3088, 256)])
def test_lora_epilogue_under_each_tiling(dev, m, n, k, r):
    g = torch.Generator().manual_seed(m + n + k + r)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
    lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    out = fp8_linear_lora(ex, d(x), d(c), d(s), d(b), d(la), d(lb), scaling=0.5, strength=1.375)
    rows = np.r_[0:16, m // 2:m // 2 + 16, m - 16:m]
    xf = x.float().numpy()[rows]
    base = O.w8a8_linear(xf, u8(c), s.reshape(-1).numpy(), b.float().numpy())
    delta = O.lora_delta(xf, la.float().numpy(), lb.float().numpy(), 0.5, 1.375)
    rel_check(out.float().cpu().numpy()[rows], O.lora_merge(base, delta))


@pytest.mark.parametrize("m,k,r", [(1, 16, 16), (37, 1536, 32), (1024, 1536, 32), (300, 1024, 64),
                                   (77, 528, 16), (9, 2048, 32), (256, 5376, 128), (1000, 5376, 16),
                                   (33, 48, 112)])
def test_fused_quantize_and_lora_down_against_the_separate_kernels(dev, m, k, r):
    g = torch.Generator().manual_seed(m * 7 + k + r)
    x = (torch.randn((m, k), generator=g) * torch.rand((m, 1), generator=g) * 8).to(torch.bfloat16)
    if m > 3:
        x[3] = 0  # a zero row: scale 1, codes 0
    la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
    d = lambda t: t.to(dev)
    codes, scales, t = kernels.quantize_rows_lora(d(x), d(la))
    ref_codes, ref_scales = kernels.quantize_rows(d(x))
    assert torch.equal(codes.view(torch.uint8), ref_codes.view(torch.uint8))
    assert torch.equal(scales, ref_scales)
    # t: the same K chunks summed in the same order as the separate kernel.
    t_sep = kernels.lora_down(d(x), d(la))
    assert torch.equal(t, t_sep)
    rel_check(t.float().cpu().numpy(),
              O.lora_delta(x.float().numpy(), la.float().numpy(), np.eye(r, dtype=np.float32)))
    # And the codes against the oracle (padding rows included).
    oc, osc = O.quantize_rows(x.float().numpy())
    assert np.array_equal(u8(codes), oc) and np.array_equal(scales.reshape(-1).cpu().numpy(), osc)


def test_lora_reference_kat_through_the_kernels(dev):
    from tests.conftest import golden

    kat = golden("lora_kat.npz")
    # The reference case is a rank-128 adapter on a 2-wide identity layer; embed it
    # in a 16-wide K (zero padding is exact) to meet the kernel's K % 16 contract.
    x = np.zeros((1, 16), np.float32)
    x[0, :2] = kat["sample"][0]
    la = np.zeros((128, 16), np.float32)
    la[:, :2] = kat["a"]
    lb = np.zeros((16, 128), np.float32)
    lb[:2] = kat["b"]
    t = kernels.lora_down(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                          torch.from_numpy(la).to(torch.bfloat16).to(dev))
    tn = t.float().cpu().numpy()
    assert np.array_equal(tn, O.lora_delta(x, la, np.eye(128, dtype=np.float32)))


def test_gate_rows_gathered_in_place_and_broadcast_over_the_batch(dev):
    # gate_msa / gate_mlp = table[:, j, :].index_select(0, adaln_indices), broadcast
    # over the batch (h3_native_denoiser.py:527-532, 556-561, h3_fused_ops.py:124-170).
    b, s, h, f, r = 2, 96, 512, 384, 7
    g = torch.Generator().manual_seed(41)
    x = torch.randn((b * s, f), generator=g).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    res = torch.randn((b * s, h), generator=g).to(torch.bfloat16)
    table = torch.rand((r, 6, h), generator=g).to(torch.bfloat16).to(dev)
    index = torch.randint(0, r, (s,), generator=g).to(dev)
    d = lambda t: t.to(dev)
    a, sa = kernels.quantize_rows(d(x))
    gate = table[:, 2, :]
    gathered = gate.index_select(0, index)
    run = lambda gt, **kw: kernels.fp8_gemm_gate_residual(a, sa, d(cd), d(sd), b * s, gt, d(res),
                                                           d(bd), **kw)
    ref = run(gathered.repeat(b, 1))
    assert torch.equal(run(gathered), ref)
    assert torch.equal(run(gate, gate_index=index), ref)
    # Through the FFN composition, with the producer's rows as input.
    y = O.gate_residual(res.float().numpy(), gathered.repeat(b, 1).float().cpu().numpy(),
                        O.w8a8_linear(x.float().numpy(), u8(cd), sd.reshape(-1).numpy(), bd.float().numpy()))
    rel_check(ref.float().cpu().numpy(), y)
    # Indices outside the table: NaN rows; every other row unchanged.
    bad = index.clone()
    bad[3], bad[10] = r, -2
    out = run(gate, gate_index=bad).float().cpu()
    nan_rows = torch.isnan(out).all(dim=1)
    expect = torch.zeros(b * s, dtype=torch.bool)
    for t in (3, 10):
        expect[t::s] = True
    assert torch.equal(nan_rows, expect)
    assert torch.equal(out[~expect], ref.float().cpu()[~expect])


def test_ffn_with_gate_index_equals_the_gathered_gate(dev):
    m, h, f = 2 * 64, 256, 384
    x, cu, su, bu, cd, sd, bd, _, res = ffn_inputs(m, h, 2 * f)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=torch.Generator().manual_seed(9)) * 0.02)
    g = torch.Generator().manual_seed(43)
    table = torch.rand((5, 6, h), generator=g).to(torch.bfloat16).to(dev)
    index = torch.randint(0, 5, (64,), generator=g).to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    d = lambda t: t.to(dev)
    args = (ex, d(x), d(cu), d(su), d(bu), d(cd), d(sd), d(bd))
    got = fp8_ffn(*args, table[:, 5, :], d(res), activation="swiglu", gate_index=index)
    ref = fp8_ffn(*args, table[:, 5, :].index_select(0, index).repeat(2, 1), d(res), activation="swiglu")
    assert torch.equal(got, ref)


@pytest.mark.parametrize("m,h,k", [(300, 512, 384), (4096, 5120, 256)])
def test_gate_residual_operand_layouts_give_the_same_bits(dev, m, h, k):
    # The epilogue loads a residual and a gate chunk with one 16-byte load each
    # when both are 16-byte aligned and the gate has unit column stride, and
    # element by element otherwise; the output takes 16-byte stores when it is
    # aligned.  Every layout computes the same bits.  The shapes cover whole
    # and partial 64x64 tiles and the 256x192 tiling's rows past the tile.
    g = torch.Generator().manual_seed(61)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    cw, sw = quantize_weight_rows(torch.randn((h, k), generator=g) * 0.02)
    cw, sw = cw.to(dev), sw.to(dev)
    bias = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16).to(dev)
    gate = torch.rand((m, h), generator=g).to(torch.bfloat16).to(dev)
    a, sa = kernels.quantize_rows(x)
    run = lambda gt, rs, **kw: kernels.fp8_gemm_gate_residual(a, sa, cw, sw, m, gt, rs, bias, **kw)
    ref = run(gate, res)
    gate_cols = gate.t().contiguous().t()            # column stride m
    wide = torch.empty((m, h + 1), dtype=torch.bfloat16, device=dev)
    wide[:, 1:] = res
    res_shifted = wide[:, 1:]                          # 2-byte aligned rows, stride h + 1
    assert gate_cols.stride() == (1, m) and res_shifted.data_ptr() % 16
    assert torch.equal(run(gate_cols, res), ref)
    assert torch.equal(run(gate, res_shifted), ref)
    out_buf = torch.empty((m, h + 4), dtype=torch.bfloat16, device=dev)
    out = out_buf[:, :h]                               # rows 8-byte aligned only
    run(gate_cols, res_shifted, out=out)
    assert torch.equal(out, ref)
