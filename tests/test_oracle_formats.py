"""Pin the oracle's number formats against torch's casts and the spec tables."""

import numpy as np
import torch

from oracle import formats as F
from tests.conftest import golden


def all_bf16_values():
    return F.bf16_from_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))


def test_e4m3_decode_matches_the_torch_table_for_every_code():
    g = golden("e4m3_table.npz")
    ours = F.e4m3_decode(g["codes"])
    ref = g["values"]
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert np.array_equal(np.signbit(ours[ok]), np.signbit(ref[ok]))
    # Spec landmarks: max 448, min subnormal 2^-9, min normal 2^-6, NaN 0x7f/0xff only.
    assert ours[0x7E] == 448 and ours[0x01] == 2.0**-9 and ours[0x08] == 2.0**-6
    assert np.isnan(ours).sum() == 2


def test_e4m3_encode_matches_torch_on_every_bf16_value_and_every_tie():
    v = all_bf16_values().astype(np.float64)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    grid = np.unique(np.abs(F.E4M3_VALUES[~np.isnan(F.E4M3_VALUES)]).astype(np.float64))
    mids = (grid[:-1] + grid[1:]) / 2  # exact ties, both even and odd neighbours
    eps = np.concatenate([mids * (1 + 2.0**-20), mids * (1 - 2.0**-20)])
    rng = np.random.default_rng(0)
    rand = rng.uniform(-448, 448, 200000) * 10.0 ** rng.uniform(-12, 0, 200000)
    x = np.concatenate([v, mids, -mids, eps, -eps, rand, [0.0, -0.0]]).astype(np.float32)
    x = np.clip(x, -448, 448)
    ours = F.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bad = ours != ref
    assert not bad.any(), (x[bad][:8], ours[bad][:8], ref[bad][:8])


def test_bf16_round_matches_torch_including_ties_and_subnormals():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    base = all_bf16_values()
    base = base[np.isfinite(base)]
    # Exact ties halfway between neighbouring bf16 values, plus neighbours.
    ties = (base.view(np.uint32) + np.uint32(0x8000)).view(np.float32)
    ties = ties[np.isfinite(ties)]
    x = np.concatenate([x, base, ties, np.nextafter(ties, np.float32(np.inf))])
    ours = F.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_e2m1_table_and_ties_follow_the_ocp_definition():
    codes = np.arange(16, dtype=np.uint8)
    vals = F.e2m1_decode(codes)
    assert list(vals[:8]) == [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    assert list(vals[8:]) == [-0.0, -0.5, -1, -1.5, -2, -3, -4, -6]
    # Every representable value round trips; ties go to the even mantissa.
    assert np.array_equal(F.e2m1_encode(vals[1:8]), codes[1:8])
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    assert list(F.e2m1_decode(F.e2m1_encode(ties))) == [0, 1, 1, 2, 2, 4, 4]
    assert list(F.e2m1_decode(F.e2m1_encode(-ties))) == [-0.0, -1, -1, -2, -2, -4, -4]
    # Brute force: the code minimises |x - value| on a dense grid.
    x = np.linspace(-6, 6, 24001)
    got = F.e2m1_decode(F.e2m1_encode(x)).astype(np.float64)
    table = np.unique(np.abs(vals).astype(np.float64))
    best = np.min(np.abs(np.abs(x)[:, None] - table[None, :]), axis=1)
    assert np.allclose(np.abs(np.abs(x) - np.abs(got)), best)
