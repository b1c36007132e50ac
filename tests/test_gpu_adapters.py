"""Low-rank residual adapters merged in the GEMM epilogues that combine them
with the other epilogues: the three Q/K/V branches of the merged projection,
the adapted gate-residual and the adapted SwiGLU input projection, against the
oracle.

Two kinds of checks:
* the epilogue on the kernel's own operands: the same GEMM without the adapter
  gives the base bit for bit, the down-projection kernel gives t, and the
  oracle's rounding chain (binary64 sums, oracle/fp8_torch.py) applied to those
  must reproduce the output exactly, up to the rare case where the MFMA's
  binary32 sum of t . B^T rounds to the other bf16 neighbour of the exact sum;
* the whole chain from the bf16 input against the numpy oracle on sampled rows.
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from oracle import fp8_torch as T
from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import (
    FusedQKV,
    LowRankResidual,
    fp8_ffn,
    gate_residual_linear,
    merge_qkv,
    qkv_linear,
    stack_adapters,
)
from vflash_amd.fp8_linear import RowFP8Linear
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def residual_weights(g, rank, k, n, scaling, dev=None):
    down = (torch.randn((rank, k), generator=g) * 0.01).to(torch.bfloat16)
    up = (torch.randn((n, rank), generator=g) * 0.01).to(torch.bfloat16)
    if dev is not None:
        down, up = down.to(dev), up.to(dev)
    return LowRankResidual(down, up, scaling)


def np_adapter(r):
    return (r.down.float().cpu().numpy(), r.up.float().cpu().numpy(), r.scaling)


def assert_chain(got, want, slack, exact_min=0.995):
    """``got`` equals the oracle chain ``want`` on at least ``exact_min`` of the
    elements.  Elsewhere the MFMA's binary32 sum of the adapter product rounded
    the delta to its other bf16 neighbour: one step of the delta, carried
    through the later roundings.  ``slack`` bounds what that step can move the
    output (the delta's magnitude, times the gate where one follows), so every
    element must lie within one bf16 step of ``want`` plus one step of ``slack``
    (bf16 steps are at most 2^-7 of the value)."""
    g, w = got.float(), want.float().to(got.device)
    assert g.shape == w.shape
    assert bool(torch.isfinite(g).all())
    exact = float((g == w).double().mean())
    assert exact >= exact_min, f"only {exact:.5f} of the outputs equal the chain"
    sl = slack.float().abs().to(got.device)
    excess = (g - w).abs() - ((w.abs() + sl) * 2.0**-7 + 2.0**-133)
    worst = int(excess.argmax())
    assert float(excess.reshape(-1)[worst]) <= 0, (
        f"beyond one bf16 step of the chain: got {float(g.reshape(-1)[worst])}, chain "
        f"{float(w.reshape(-1)[worst])}, slack {float(sl.reshape(-1)[worst])}")
    return exact


def gated_slack(gate, projected, delta):
    """Slack of bf16(residual + bf16(gate * bf16(base + delta))): the adapted
    projection moves by one step of itself and of the delta, the gated product
    by the gate times that and one step of its own."""
    return gate.float().abs() * (2 * projected.float().abs() + delta.float().abs())


def _delta(t, up, scaling):
    d = T.bf16_round(t.double() @ up.double().T)
    if scaling != 1.0:
        d = T.bf16_round(d * torch.tensor(scaling, dtype=torch.float32, device=d.device))
    return d


# ---------------------------------------------------------------------------
# Merged QKV with the Q/K/V residual pack.

def qkv_case(m, hidden, inner, ranks, scalings, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
    parts = [quantize_weight_rows(torch.randn((inner, hidden), generator=g) * 0.02) for _ in range(3)]
    bias = (torch.randn(3 * inner, generator=g) * 0.01).to(torch.bfloat16)
    residuals = [residual_weights(g, r, hidden, inner, s, dev) for r, s in zip(ranks, scalings)]
    w, sc = merge_qkv([p[0].to(dev) for p in parts], [p[1].to(dev) for p in parts])
    return x, w, sc, bias.to(dev), residuals


def qkv_expected(ex, xd, w, sc, bias, residuals):
    """The chain on the kernel's operands: plain merged GEMM, then per branch
    lora_merge(base_b, delta_b(t_b))."""
    base = torch.cat(qkv_linear(ex, xd, w, sc, bias), dim=-1).reshape(-1, w.shape[0])
    inner = w.shape[0] // 3
    x2 = xd.reshape(-1, xd.shape[-1])
    chunks, deltas = [], []
    for b, r in enumerate(residuals):
        t = kernels.lora_down(x2, r.down)
        d = _delta(t, r.up, r.scaling)
        chunks.append(T.lora_merge(base[:, b * inner : (b + 1) * inner], d))
        deltas.append(d)
    return torch.cat(chunks, dim=1), torch.cat(deltas, dim=1)


@pytest.mark.parametrize(
    "m,hidden,inner,ranks,scalings",
    [
        (300, 512, 256, (16, 16, 16), (0.0625, 0.0625, 0.0625)),
        (1000, 1024, 512, (32, 8, 24), (1.0, 0.5, 1.375)),
        (77, 256, 160, (1, 100, 128), (0.25, 1.0, 2.0)),
        (4100, 768, 384, (48, 48, 48), (0.0625, 0.125, 0.1)),
    ],
)
def test_qkv_branches_on_the_kernels_operands(dev, m, hidden, inner, ranks, scalings):
    x, w, sc, bias, residuals = qkv_case(m, hidden, inner, ranks, scalings, m + inner, dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    xd = x.to(dev)
    want, delta = qkv_expected(ex, xd, w, sc, bias, residuals)
    q, k, v = qkv_linear(ex, xd, w, sc, bias, residuals=residuals)
    assert_chain(torch.cat((q, k, v), dim=-1), want, delta)
    # The planes give the same bits, and so does the pack stacked once.
    stacked = stack_adapters(residuals, hidden, 3 * inner)
    planes = qkv_linear(ex, xd, w, sc, bias, planes=True, residuals=stacked)
    for got, ref in zip(planes, (q, k, v)):
        assert got.is_contiguous() and torch.equal(got, ref)
    # The branch width decides the tiling: every wave's columns lie in one branch.
    tiling = kernels.gemm_tiling(m, 3 * inner, branch_cols=inner)
    wave_cols = int(tiling.split("x")[1].split()[0]) // 2
    assert inner % wave_cols == 0
    # Against the oracle from the bf16 input, on sampled rows.
    rows = np.r_[0:8, m // 2 : m // 2 + 8, m - 8 : m]
    xs = x.float().numpy()[rows]
    base = O.w8a8_linear(xs, u8(w), sc.reshape(-1).cpu().numpy(), bias.float().cpu().numpy())
    ref = O.qkv_adapted(base, xs, [np_adapter(r) for r in residuals])
    rel_check(torch.cat((q, k, v), dim=-1).float().cpu().numpy()[rows], ref)


def test_qkv_branches_through_the_producer_rows_and_module(dev):
    from vflash_amd import producers

    m, hidden, inner = 256, 512, 256
    x, w, sc, bias, residuals = qkv_case(m, hidden, inner, (32, 32, 32), (0.5, 0.5, 0.5), 5, dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    xd = x.to(dev)
    want = qkv_linear(ex, xd, w, sc, bias, residuals=residuals)
    # Rows a producer quantized and kept in bf16: the same codes and the same t,
    # so the same bits.
    codes, scales = kernels.quantize_rows(xd)
    rows = producers.QuantizedRows(codes, scales, xd.shape, xd)
    got = qkv_linear(ex, rows, w, sc, bias, residuals=residuals)
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    # The module form (no bias, stacked once at construction).
    g = torch.Generator().manual_seed(9)
    mods = []
    for i in range(3):
        lin = torch.nn.Linear(hidden, inner, bias=False)
        mod = RowFP8Linear(lin, ex)
        c, s = quantize_weight_rows(torch.randn((inner, hidden), generator=g) * 0.02)
        mod.weight = torch.nn.Parameter(c.to(dev), requires_grad=False)
        mod.row_scale = s.to(dev)
        mods.append(mod)
    fused = FusedQKV(*mods, planes=True, residuals=residuals)
    wm, sm = merge_qkv([p.weight for p in mods], [p.row_scale for p in mods])
    for a, b in zip(fused(xd), qkv_linear(ex, xd, wm, sm, residuals=residuals)):
        assert torch.equal(a, b)


def test_qkv_branches_row_tiles_equal_the_whole_call(dev):
    m, hidden, inner = 2600, 1024, 640
    x, w, sc, bias, residuals = qkv_case(m, hidden, inner, (32, 16, 48), (0.0625,) * 3, 11, dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    xd = x.to(dev)
    whole = torch.cat(qkv_linear(ex, xd, w, sc, bias, residuals=residuals), dim=-1)
    for tile in (1024, 600):
        parts = [torch.cat(qkv_linear(ex, xd[i : i + tile], w, sc, bias, residuals=residuals), dim=-1)
                 for i in range(0, m, tile)]
        assert torch.equal(torch.cat(parts), whole)


@pytest.mark.parametrize("rank", [16, 32, 128])
def test_qkv_branches_configuration_shape(dev, rank):
    # X [32760, 5120]; merged W [15360, 5120]; a Q/K/V pack of rank `rank`, scaling 1/16.
    m, hidden, inner = 32760, 5120, 5120
    x, w, sc, bias, residuals = qkv_case(m, hidden, inner, (rank,) * 3, (0.0625,) * 3, rank, dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    xd = x.to(dev)
    planes = qkv_linear(ex, xd, w, sc, bias, planes=True, residuals=residuals)
    got = torch.cat(planes, dim=1)
    exact = assert_chain(got, *qkv_expected(ex, xd, w, sc, bias, residuals))
    assert exact > 0.999
    rows = np.r_[0:8, 16380:16388, 32752:32760]
    xs = x.float().numpy()[rows]
    base = O.w8a8_linear(xs, u8(w), sc.reshape(-1).cpu().numpy(), bias.float().cpu().numpy())
    ref = O.qkv_adapted(base, xs, [np_adapter(r) for r in residuals])
    rel_check(got.float().cpu().numpy()[rows], ref)
    # A 16384-row tile gives the whole call's bits.
    tile = torch.cat(qkv_linear(ex, xd[16384:], w, sc, bias, planes=True, residuals=residuals), dim=1)
    assert torch.equal(tile, got[16384:])


# ---------------------------------------------------------------------------
# The adapted gate-residual (attention output and FFN down projections).

def gate_case(m, k, n, rank, scaling, seed, dev, token_gate=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    res = torch.randn((m, n), generator=g).to(torch.bfloat16)
    gate = torch.rand((m, n) if token_gate else (n,), generator=g).to(torch.bfloat16)
    adapter = residual_weights(g, rank, k, n, scaling, dev)
    d = lambda t: t.to(dev)
    return d(x), d(c), d(s), d(b), d(res), d(gate), adapter


# Shapes that route to every tiling (the attention output shapes of the audio
# pass among them), with ranks that end inside an 8-element group.
@pytest.mark.parametrize(
    "m,k,n,rank,scaling,token_gate",
    [
        (300, 512, 640, 16, 0.0625, False),    # 64x64
        (300, 512, 4112, 5, 1.0, True),        # 128x64
        (2100, 384, 3712, 40, 0.5, False),     # 128x128, two per CU
        (1024, 1536, 6144, 32, 1.375, True),   # 128x192
        (1024, 512, 7168, 128, 0.0625, False), # 256x128
        (4096, 1536, 3072, 100, 0.25, False),  # 256x192
        (4100, 256, 3088, 24, 0.0625, True),   # 256x256
    ],
)
def test_adapted_gate_residual_on_the_kernels_operands(dev, m, k, n, rank, scaling, token_gate):
    x, c, s, b, res, gate, adapter = gate_case(m, k, n, rank, scaling, m + n + rank, dev,
                                               token_gate)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    got = gate_residual_linear(ex, x, c, s, b, gate, res, adapter=adapter)
    base = ex.linear(x, c, s, b)
    t = kernels.lora_down(x, adapter.down)
    delta = _delta(t, adapter.up, scaling)
    projected = T.lora_merge(base, delta)
    want = T.gate_residual(res, gate, projected)
    assert_chain(got, want, gated_slack(gate, projected, delta))
    # Without the adapter: the plain gate-residual epilogue.
    plain = gate_residual_linear(ex, x, c, s, b, gate, res)
    assert torch.equal(plain.float(), T.gate_residual(res, gate, base))
    rows = np.r_[0:8, m // 2 : m // 2 + 8, m - 8 : m]
    xs = x.float().cpu().numpy()[rows]
    lin = O.w8a8_linear(xs, u8(c), s.reshape(-1).cpu().numpy(), b.float().cpu().numpy())
    gs = gate.float().cpu().numpy()
    ref = O.adapted_gate_residual(res.float().cpu().numpy()[rows], gs[rows] if token_gate else gs,
                                  lin, xs, np_adapter(adapter))
    rel_check(got.float().cpu().numpy()[rows], ref)


def test_adapted_gate_residual_reads_the_adaln_rows_in_place(dev):
    m, k, n, tokens = 512, 512, 384, 128
    x, c, s, b, res, _, adapter = gate_case(m, k, n, 32, 0.0625, 3, dev)
    table = torch.rand((4, 6, n), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    index = torch.randint(0, 4, (tokens,), generator=torch.Generator().manual_seed(5)).to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    got = gate_residual_linear(ex, x, c, s, b, table[:, 2, :], res, gate_index=index,
                               adapter=adapter)
    gathered = table[:, 2, :].index_select(0, index).repeat(m // tokens, 1)
    want = gate_residual_linear(ex, x, c, s, b, gathered.contiguous(), res, adapter=adapter)
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------
# The FFN with its input and output adapters.

def ffn_case(m, h, f, activation, rank, seed, dev):
    g = torch.Generator().manual_seed(seed)
    up_rows = 2 * f if activation == "swiglu" else f
    x = torch.randn((m, h), generator=g).to(torch.bfloat16)
    cu, su = quantize_weight_rows(torch.randn((up_rows, h), generator=g) * 0.02)
    bu = (torch.randn(up_rows, generator=g) * 0.01).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand(h, generator=g).to(torch.bfloat16)
    res = torch.randn((m, h), generator=g).to(torch.bfloat16)
    up_res = residual_weights(g, rank, h, up_rows, 0.0625, dev)
    down_res = residual_weights(g, rank, f, h, 0.0625, dev)
    d = lambda t: t.to(dev)
    return [d(v) for v in (x, cu, su, bu, cd, sd, bd, gate, res)], up_res, down_res


def ffn_stage_checks(ex, ops, up_res, down_res, activation, out):
    """Every stage on the kernels' own operands: the adapted up projection and
    activation, the requantization, the adapted down projection and epilogue."""
    x, cu, su, bu, cd, sd, bd, gate, res = ops
    m = x.shape[0]
    a, sa = kernels.quantize_rows(x)
    up_base = kernels.fp8_gemm(a, sa, cu, su, m, bu)
    t_up = kernels.lora_down(x, up_res.down)
    d_up = _delta(t_up, up_res.up, up_res.scaling)
    up = T.lora_merge(up_base, d_up)
    # The adapted up projection (the LoRA epilogue on the same operands) is the
    # chain up to the adapter sum's last-bit cases.
    y = kernels.fp8_gemm_lora(a, sa, cu, su, m, t_up, up_res.up, scale=up_res.scaling, bias=bu)
    assert_chain(y, up, d_up)
    if activation == "swiglu":
        # The SwiGLU tile merges the adapter with the same arithmetic, so h is the
        # SwiGLU of that projection bit for bit, and its maxima those of h.
        h, amax = kernels.fp8_gemm_swiglu(a, sa, cu, su, m, bu,
                                          lora=kernels.LoraOperands(t_up, up_res.up, up_res.scaling))
        assert torch.equal(h.float(), T.silu_mul(y))
        assert torch.equal(amax, h.float().abs().reshape(m, -1, 128).amax(dim=2))
        hc, hs = kernels.requant_rows(h, amax)
        g_act = h
    else:
        hc, hs, g_act = kernels.gelu_quantize_rows(y, keep_values=True)
        assert torch.equal(g_act.float(), T.gelu_tanh(y))
    ref_codes, ref_scales = T.quantize_rows(g_act)
    assert torch.equal(hc.view(torch.uint8), ref_codes) and torch.equal(hs.reshape(-1), ref_scales)
    y_down = kernels.fp8_gemm(hc, hs, cd, sd, m, bd)
    t_down = kernels.lora_down(g_act, down_res.down)
    d_down = _delta(t_down, down_res.up, down_res.scaling)
    projected = T.lora_merge(y_down, d_down)
    want = T.gate_residual(res, gate, projected)
    assert_chain(out, want, gated_slack(gate, projected, d_down))


@pytest.mark.parametrize("activation", ["gelu_tanh", "swiglu"])
@pytest.mark.parametrize("m,h,f,rank", [(300, 512, 1024, 16), (1000, 768, 1536, 40)])
def test_ffn_adapters_stage_by_stage(dev, activation, m, h, f, rank):
    ops, up_res, down_res = ffn_case(m, h, f, activation, rank, m + rank, dev)
    x, cu, su, bu, cd, sd, bd, gate, res = ops
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    out = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, activation=activation,
                  up_residual=up_res, down_residual=down_res)
    ffn_stage_checks(ex, ops, up_res, down_res, activation, out)
    # The whole chain from the bf16 input (numpy oracle, binary64 sums).
    n = lambda t: t.float().cpu().numpy()
    *_, chain = O.ffn(n(x), u8(cu), n(su).reshape(-1), n(bu), u8(cd), n(sd).reshape(-1), n(bd),
                      n(gate), n(res), activation=activation, up_adapter=np_adapter(up_res),
                      down_adapter=np_adapter(down_res))
    err = np.abs(n(out).astype(np.float64) - chain)
    # The GEMMs' tolerance, composed through the activation and requantization.
    rms = float(np.sqrt(np.mean(chain.astype(np.float64) ** 2)))
    assert np.all(err <= 2.0**-4 * np.abs(chain) + 2e-2 * rms)
    # Only the input adapter, only the output adapter: each the matching chain.
    for up_r, down_r in ((up_res, None), (None, down_res)):
        part = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, activation=activation,
                       up_residual=up_r, down_residual=down_r)
        *_, chain = O.ffn(n(x), u8(cu), n(su).reshape(-1), n(bu), u8(cd), n(sd).reshape(-1),
                          n(bd), n(gate), n(res), activation=activation,
                          up_adapter=None if up_r is None else np_adapter(up_r),
                          down_adapter=None if down_r is None else np_adapter(down_r))
        err = np.abs(n(part).astype(np.float64) - chain)
        assert np.all(err <= 2.0**-4 * np.abs(chain) + 2e-2 * rms)


def test_ffn_adapters_row_tiles_equal_the_whole_call(dev):
    for activation in ("gelu_tanh", "swiglu"):
        ops, up_res, down_res = ffn_case(2100, 512, 1024, activation, 32, 21, dev)
        x, cu, su, bu, cd, sd, bd, gate, res = ops
        ex = RowFP8Execution("w8a8", activation_quantizer="triton")
        call = lambda lo, hi: fp8_ffn(ex, x[lo:hi], cu, su, bu, cd, sd, bd, gate, res[lo:hi],
                                      activation=activation, up_residual=up_res,
                                      down_residual=down_res)
        whole = call(0, 2100)
        assert torch.equal(torch.cat([call(0, 1024), call(1024, 2048), call(2048, 2100)]), whole)


@pytest.mark.parametrize("rank", [16, 32, 128])
def test_gelu_ffn_adapters_configuration_shape(dev, rank):
    # X [32760, 5120]; up [13824, 5120] + GELU-tanh; down [5120, 13824] + gate-residual;
    # input and output adapters of rank `rank`, scaling 1/16.
    ops, up_res, down_res = ffn_case(32760, 5120, 13824, "gelu_tanh", rank, rank, dev)
    x, cu, su, bu, cd, sd, bd, gate, res = ops
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    out = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, up_residual=up_res,
                  down_residual=down_res)
    ffn_stage_checks(ex, ops, up_res, down_res, "gelu_tanh", out)
    tile = fp8_ffn(ex, x[16384:], cu, su, bu, cd, sd, bd, gate, res[16384:], up_residual=up_res,
                   down_residual=down_res)
    assert torch.equal(tile, out[16384:])


def test_swiglu_ffn_adapters_h3_shape(dev):
    # The H3 feed-forward (hidden 5376, inner 14336) with rank-32 input and output adapters.
    ops, up_res, down_res = ffn_case(32760, 5376, 14336, "swiglu", 32, 4, dev)
    x, cu, su, bu, cd, sd, bd, gate, res = ops
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    out = fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, activation="swiglu",
                  up_residual=up_res, down_residual=down_res)
    ffn_stage_checks(ex, ops, up_res, down_res, "swiglu", out)


def test_lora_linear_refuses_unsupported_adapters_before_counting(dev):
    # A rank above the epilogue's 128 or a non-BF16 adapter is refused before the
    # execution counts the call or launches the quantizer.
    from vflash_amd.fused import fp8_linear_lora

    g = torch.Generator().manual_seed(71)
    cw, sw = quantize_weight_rows(torch.randn((256, 128), generator=g) * 0.02)
    x = torch.randn((32, 128), generator=g).to(torch.bfloat16).to(dev)
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    cases = [
        (torch.zeros((129, 128), dtype=torch.bfloat16), torch.zeros((256, 129), dtype=torch.bfloat16), "ranks"),
        (torch.zeros((16, 128)), torch.zeros((256, 16)), "BF16"),
    ]
    for la, lb, match in cases:
        with pytest.raises(ValueError, match=match):
            fp8_linear_lora(ex, x, cw.to(dev), sw.to(dev), None, la.to(dev), lb.to(dev))
    assert ex.calls == {"weight_only": 0, "w8a8": 0}
    # Strength 0 skips the adapter (the reference hook returns the base result).
    out = fp8_linear_lora(ex, x, cw.to(dev), sw.to(dev), None, cases[1][0].to(dev),
                          cases[1][1].to(dev), strength=0.0)
    assert torch.equal(out, ex.linear(x, cw.to(dev), sw.to(dev), None))
