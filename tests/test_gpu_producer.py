"""RMSNorm + adaLN modulation + E4M3 quantization in one pass on gfx950, vs the oracle."""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import fp8_ffn, fp8_linear_lora, qkv_linear
from vflash_amd.prepare import quantize_weight_rows
from vflash_amd.producers import rmsnorm_modulate_quantize

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def block_input(b, s, h, seed=0, exact=False):
    g = torch.Generator().manual_seed(seed)
    if exact:
        # x = k/16: every partial sum of squares is exact in binary32, so the
        # kernel's summation order cannot change rstd.
        x = (torch.randint(-16, 17, (b, s, h), generator=g).float() / 16).to(torch.bfloat16)
    else:
        x = (torch.randn((b, s, h), generator=g) * 2).to(torch.bfloat16)
    w = (torch.rand(h, generator=g) * 2).to(torch.bfloat16)
    scale = (torch.randn((s, h), generator=g) * 0.5).to(torch.bfloat16)
    shift = torch.randn((s, h), generator=g).to(torch.bfloat16)
    return x, w, scale, shift


def oracle_values(x, w, scale, shift, eps, tokens_of_row):
    h = x.shape[-1]
    n = O.rms_norm(x.float().numpy().reshape(-1, h), None if w is None else w.float().numpy(), eps)
    return O.modulate(n, scale.float().numpy()[tokens_of_row], shift.float().numpy()[tokens_of_row])


def check_codes(q, values_np, m):
    # Bit-exact: the codes and scales are the quantization of the kernel's own y.
    rc, rs = O.quantize_rows(values_np)
    assert np.array_equal(u8(q.codes), rc)
    assert np.array_equal(q.scales.reshape(-1).cpu().numpy(), rs)
    assert q.codes.shape[0] == (m + 15) // 16 * 16


@pytest.mark.parametrize("b,s,h", [(2, 150, 512), (1, 77, 5120), (3, 16, 5376), (1, 5, 8)])
@pytest.mark.parametrize("weighted", [True, False])
def test_values_and_codes_against_the_oracle(dev, b, s, h, weighted):
    x, w, scale, shift = block_input(b, s, h, seed=h + b)
    w = w if weighted else None
    eps = 1e-6
    d = lambda t: None if t is None else t.to(dev)
    q = rmsnorm_modulate_quantize(d(x), d(w), d(scale), d(shift), eps=eps, keep_values=True)
    got = q.values.float().cpu().numpy().reshape(-1, h)
    ref = oracle_values(x, w, scale, shift, eps, np.arange(b * s) % s)
    # Summation order of the sum of squares only: at most one bf16 step of n,
    # carried through the modulation (two more roundings), on few elements.
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= np.abs(ref) * 2.0**-6 + 2.0**-6 * np.abs(shift.float().numpy()).max())
    assert (got != ref).mean() < 1e-3
    check_codes(q, got, b * s)


def test_exact_sums_are_bit_exact_through_the_chain(dev):
    b, s, h = 2, 96, 5120
    x, w, scale, shift = block_input(b, s, h, seed=5, exact=True)
    q = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), scale.to(dev), shift.to(dev), eps=1e-5,
                                  keep_values=True)
    ref = oracle_values(x, w, scale, shift, 1e-5, np.arange(b * s) % s)
    assert np.array_equal(q.values.float().cpu().numpy().reshape(-1, h), ref)
    rc, rs = O.quantize_rows(ref)
    assert np.array_equal(u8(q.codes), rc) and np.array_equal(q.scales.reshape(-1).cpu().numpy(), rs)


def test_table_rows_gathered_in_place_equal_the_materialized_gather(dev):
    # adaLN table [R, 6, H]; token s uses row index[s] (h3_native_denoiser.py:527-532).
    b, s, h, r = 2, 200, 5376, 24
    g = torch.Generator().manual_seed(11)
    x, w, _, _ = block_input(b, s, h, seed=12)
    table = (torch.randn((r, 6, h), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    index = torch.randint(0, r, (s,), generator=g).to(dev)
    xd, wd = x.to(dev), w.to(dev)
    for j in (0, 3):
        scale, shift = table[:, j + 1, :], table[:, j, :]
        q = rmsnorm_modulate_quantize(xd, wd, scale, shift, eps=1e-6, index=index, keep_values=True)
        gathered = [t.index_select(0, index).contiguous() for t in (scale, shift)]
        p = rmsnorm_modulate_quantize(xd, wd, *gathered, eps=1e-6, keep_values=True)
        assert torch.equal(q.values, p.values)
        assert torch.equal(q.codes.view(torch.uint8), p.codes.view(torch.uint8))
        assert torch.equal(q.scales, p.scales)
        # int32 indices (the reference admits both) give the same rows.
        q32 = rmsnorm_modulate_quantize(xd, wd, scale, shift, eps=1e-6, index=index.int())
        assert torch.equal(q32.codes.view(torch.uint8), q.codes.view(torch.uint8))


def run_index(s, r, runs, seed):
    # Token runs of one modulation row each (a packed sequence groups its tokens by
    # modality and frame), with run lengths that are not multiples of four.
    g = torch.Generator().manual_seed(seed)
    cuts = torch.sort(torch.randperm(s - 1, generator=g)[: runs - 1] + 1).values.tolist()
    index = torch.empty(s, dtype=torch.int64)
    for i, (a, b) in enumerate(zip([0] + cuts, cuts + [s])):
        index[a:b] = (7 * i + 3) % r
    return index


@pytest.mark.parametrize("h,weighted", [(5376, True), (1536, False), (5456, True), (5464, True)])
def test_index_runs_share_the_modulation_row(dev, h, weighted):
    # Workgroups whose four rows share a modulation row widen it once (in LDS); the
    # others, and widths past the shared table, take the per-row path.  Both give
    # the materialized gather's bits (which runs row by row).
    b, s, r = 2, 301, 24
    g = torch.Generator().manual_seed(h)
    x, w, _, _ = block_input(b, s, h, seed=h + 1)
    w = w if weighted else None
    table = (torch.randn((r, 6, h), generator=g) * 0.5).to(torch.bfloat16)
    index = run_index(s, r, 9, seed=h + 2)
    d = lambda t: None if t is None else t.to(dev)
    tb = table.to(dev)
    scale, shift = tb[:, 1, :], tb[:, 0, :]
    q = rmsnorm_modulate_quantize(d(x), d(w), scale, shift, eps=1e-6, index=d(index), keep_values=True)
    gathered = [t.index_select(0, d(index)).contiguous() for t in (scale, shift)]
    p = rmsnorm_modulate_quantize(d(x), d(w), *gathered, eps=1e-6, keep_values=True)
    assert torch.equal(q.values, p.values)
    assert torch.equal(q.codes.view(torch.uint8), p.codes.view(torch.uint8))
    assert torch.equal(q.scales, p.scales)
    got = q.values.float().cpu().numpy().reshape(-1, h)
    ref = oracle_values(x, w, table[:, 1, :], table[:, 0, :], 1e-6, index.numpy()[np.arange(b * s) % s])
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= np.abs(ref) * 2.0**-6 + 2.0**-6 * float(table[:, 0, :].float().abs().max()))
    assert (got != ref).mean() < 1e-3
    check_codes(q, got, b * s)


def test_one_token_broadcast_shares_the_row(dev):
    # One modulation row for every row (tokens = 1): the shared path in every full
    # workgroup, the per-row path in the last (m % 4 rows), equal to the same row
    # repeated per token.
    m, h = 1023, 5120
    x, w, scale, shift = block_input(m, 1, h, seed=41)  # x [m, 1, h], one token
    d = lambda t: t.to(dev)
    q = rmsnorm_modulate_quantize(d(x), d(w), d(scale), d(shift), eps=1e-6, keep_values=True)
    p = rmsnorm_modulate_quantize(d(x).view(1, m, h), d(w), d(scale.expand(m, h).contiguous()),
                                  d(shift.expand(m, h).contiguous()), eps=1e-6, keep_values=True)
    assert torch.equal(q.values.view(m, h), p.values.view(m, h))
    assert torch.equal(q.codes.view(torch.uint8), p.codes.view(torch.uint8))
    assert torch.equal(q.scales, p.scales)
    check_codes(q, q.values.float().cpu().numpy().reshape(-1, h), m)


def test_a_run_of_indices_outside_the_table_stays_nan(dev):
    # Four rows with one shared index that lies outside the table: no shared
    # widening of a row that does not exist; the rows get NaN scales.
    s, h, r = 16, 512, 4
    x, w, _, _ = block_input(1, s, h, seed=43)
    table = torch.randn((r, 6, h)).to(torch.bfloat16).to(dev)
    index = torch.tensor([1] * 4 + [7] * 4 + [2] * 4 + [-3] * 4, device=dev)
    q = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), table[:, 1, :], table[:, 0, :], eps=1e-6,
                                  index=index, keep_values=True)
    sc = q.scales.reshape(-1).cpu()
    assert torch.isnan(sc[4:8]).all() and torch.isnan(sc[12:16]).all()
    assert torch.isfinite(sc[0:4]).all() and torch.isfinite(sc[8:12]).all()
    # The valid runs against the materialized gather (the per-row path).
    good = torch.tensor([1] * 4 + [0] * 4 + [2] * 4 + [0] * 4, device=dev)
    gathered = [t.index_select(0, good).contiguous() for t in (table[:, 1, :], table[:, 0, :])]
    p = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), *gathered, eps=1e-6, keep_values=True)
    for rows in (slice(0, 4), slice(8, 12)):
        assert torch.equal(q.values[0, rows], p.values[0, rows])
        assert torch.equal(q.codes.view(torch.uint8)[rows], p.codes.view(torch.uint8)[rows])


def test_modulation_row_offset_beyond_two_to_the_31_elements(dev):
    # Row 66577 of a [66578, 6, 5376] table starts at element 66577 * 32256 > 2^31 - 1
    # (the strided views of h3_fused_ops.py:24-40).
    rows, h = 66578, 5376
    table = torch.empty((rows, 6, h), dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(13)
    for row in (0, rows - 1):
        table[row] = (torch.randn((6, h), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    assert (rows - 1) * 6 * h > 2**31 - 1
    x, w, _, _ = block_input(1, 4, h, seed=14)
    index = torch.tensor([rows - 1, 0, rows - 1, 0], device=dev)
    scale, shift = table[:, 1, :], table[:, 0, :]
    q = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), scale, shift, eps=1e-6, index=index,
                                  keep_values=True)
    gathered = [t.index_select(0, index).contiguous() for t in (scale, shift)]
    p = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), *gathered, eps=1e-6, keep_values=True)
    assert torch.equal(q.values, p.values) and torch.equal(q.scales, p.scales)
    del table


def test_index_outside_the_table_gives_nan_rows(dev):
    b, s, h, r = 1, 8, 512, 4
    x, w, _, _ = block_input(b, s, h, seed=15)
    table = torch.randn((r, 6, h)).to(torch.bfloat16).to(dev)
    index = torch.tensor([0, 1, 4, 2, -1, 3, 0, 1], device=dev)
    q = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), table[:, 1, :], table[:, 0, :], eps=1e-6,
                                  index=index)
    sc = q.scales.reshape(-1).cpu()
    bad = torch.tensor([2, 4])
    assert torch.isnan(sc[bad]).all() and torch.isfinite(sc[[0, 1, 3, 5, 6, 7]]).all()
    assert (q.codes.view(torch.uint8)[bad.to(dev)] == 0).all()


def test_consumers_take_the_rows_in_place_of_the_bf16_activation(dev):
    b, s, h, inner, f = 2, 100, 512, 256, 384
    x, w, scale, shift = block_input(b, s, h, seed=21)
    d = lambda t: t.to(dev)
    q = rmsnorm_modulate_quantize(d(x), d(w), d(scale), d(shift), eps=1e-6, keep_values=True)
    y = q.values
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")
    g = torch.Generator().manual_seed(22)
    cw, sw = quantize_weight_rows(torch.randn((3 * inner, h), generator=g) * 0.02)
    bias = (torch.randn(3 * inner, generator=g) * 0.01).to(torch.bfloat16)
    # The codes are the quantization of y, so every consumer is bit-identical to
    # the same consumer fed y itself.
    assert torch.equal(ex.linear(q, d(cw), d(sw), d(bias)), ex.linear(y, d(cw), d(sw), d(bias)))
    for planes in (False, True):
        for got, ref in zip(qkv_linear(ex, q, d(cw), d(sw), d(bias), planes=planes),
                            qkv_linear(ex, y, d(cw), d(sw), d(bias), planes=planes)):
            assert torch.equal(got, ref)
    cu, su = quantize_weight_rows(torch.randn((2 * f, h), generator=g) * 0.02)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    gate = (torch.rand((s, h), generator=g) * 0.5).to(torch.bfloat16)
    res = torch.randn((b, s, h), generator=g).to(torch.bfloat16)
    ffn = lambda v: fp8_ffn(ex, v, d(cu), d(su), None, d(cd), d(sd), None,
                            d(gate).repeat(b, 1), d(res), activation="swiglu")
    assert torch.equal(ffn(q), ffn(y))
    la = (torch.randn((32, h), generator=g) * 0.05).to(torch.bfloat16)
    lb = (torch.randn((3 * inner, 32), generator=g) * 0.05).to(torch.bfloat16)
    got = fp8_linear_lora(ex, q, d(cw), d(sw), d(bias), d(la), d(lb), scaling=0.5)
    ref = fp8_linear_lora(ex, y, d(cw), d(sw), d(bias), d(la), d(lb), scaling=0.5)
    rel_check(got.float().cpu().numpy().reshape(-1, 3 * inner), ref.float().cpu().numpy().reshape(-1, 3 * inner))
    # End to end against the oracle chain: norm, modulation, quantization, GEMM.
    yo = oracle_values(x, w, scale, shift, 1e-6, np.arange(b * s) % s)
    ref = O.w8a8_linear(yo, u8(cw), sw.reshape(-1).numpy(), bias.float().numpy())
    out = ex.linear(q, d(cw), d(sw), d(bias)).float().cpu().numpy().reshape(-1, 3 * inner)
    rel_check(out, ref)


@pytest.mark.parametrize("runs", [False, True])
def test_metric_shape_sampled(dev, runs):
    # M = 32760 tokens, hidden 5120, modulation rows from a 24-row table: random
    # per token, or in 24 runs (the shared-row path).
    s, h, r = 32760, 5120, 24
    g = torch.Generator().manual_seed(31)
    x = (torch.randn((1, s, h), generator=g) * 2).to(torch.bfloat16)
    w = (torch.rand(h, generator=g) * 2).to(torch.bfloat16)
    table = (torch.randn((r, 6, h), generator=g) * 0.5).to(torch.bfloat16)
    index = run_index(s, r, 24, seed=32) if runs else torch.randint(0, r, (s,), generator=g)
    tb = table.to(dev)
    q = rmsnorm_modulate_quantize(x.to(dev), w.to(dev), tb[:, 1, :], tb[:, 0, :], eps=1e-6,
                                  index=index.to(dev), keep_values=True)
    rows = np.r_[0:16, 20000:20016, 32744:32760]
    got = q.values.float().cpu().numpy().reshape(-1, h)[rows]
    idx = index.numpy()[rows]
    n = O.rms_norm(x.float().numpy().reshape(-1, h)[rows], w.float().numpy(), 1e-6)
    ref = O.modulate(n, table[:, 1, :].float().numpy()[idx], table[:, 0, :].float().numpy()[idx])
    assert (got != ref).mean() < 1e-3
    bound = np.abs(ref) * 2.0**-6 + 2.0**-6 * float(table[:, 0, :].float().abs().max())
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound)
    rc, rs = O.quantize_rows(got, pad=1)
    assert np.array_equal(u8(q.codes)[rows], rc)
    assert np.array_equal(q.scales.reshape(-1).cpu().numpy()[rows], rs)
    assert bool(torch.isfinite(q.scales).all())
