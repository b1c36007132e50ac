"""Pin the NVFP4 oracle (this path's convention; FlashInfer itself is unavailable)."""

import numpy as np
import torch

from oracle import nvfp4 as N
from oracle.formats import e2m1_decode, e4m3_decode
from vflash_amd import prepare


def test_128x4_order_is_a_bijection_with_the_published_tile_formula():
    n, kb = 256, 12
    nn, jj = np.meshgrid(np.arange(n), np.arange(kb), indexing="ij")
    off = N.scale_offset_128x4(nn, jj, kb)
    assert np.array_equal(np.sort(off.reshape(-1)), np.arange(n * kb))
    # Hand-computed positions: (row, block) -> byte.
    assert off[0, 0] == 0 and off[0, 3] == 3 and off[1, 0] == 16 and off[32, 0] == 4
    assert off[0, 4] == 512 and off[128, 0] == 3 * 512 and off[127, 3] == 31 * 16 + 3 * 4 + 3
    plain = np.arange(n * kb, dtype=np.int64).reshape(n, kb) % 251
    assert np.array_equal(N.unswizzle_128x4(N.swizzle_128x4(plain)), plain)


def test_torch_packer_matches_the_oracle_bit_for_bit():
    g = torch.Generator().manual_seed(0)
    w = torch.randn((256, 320), generator=g) * 0.02
    w[3, :16] = 0.0  # an all-zero block
    packed, scales, alpha, ins = prepare.quantize_nvfp4_weight(w)
    rp, rs, ra = N.quantize_weight(w.numpy())
    assert np.array_equal(packed.numpy(), rp)
    assert np.array_equal(scales.numpy(), rs)
    assert alpha.item() == float(ra) and ins.item() == 1.0


def test_packing_round_trip_error_is_bounded_by_the_formats():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((128, 256)) * 0.02).astype(np.float32)
    packed, scales, alpha = N.quantize_weight(w)
    dq = N.dequantize_weight(packed, scales) * float(alpha)
    # Each block's scale is the block max / 6 rounded to E4M3 (<= 2^-4 relative),
    # and E2M1 steps are at most 1/3 of the block scale x 6 range -> |err| <= amax_block / 6.
    blocks = np.abs(w).reshape(128, -1, 16).max(axis=2)
    bound = np.repeat(blocks, 16, axis=1) / 6.0 * 1.07
    assert np.all(np.abs(dq - w) <= bound)
    # The block maximum maps to +-6 (code 7 / 15) unless the scale rounded up.
    q = np.empty((128, 256), np.uint8)
    q[:, 0::2], q[:, 1::2] = packed & 0xF, packed >> 4
    assert np.mean((q & 7) == 7) > 0.03


def test_nvfp4_linear_oracle_matches_brute_force():
    rng = np.random.default_rng(2)
    m, n, k = 5, 128, 64
    a = rng.integers(0, 0x7F, (m, k)).astype(np.uint8) & 0xF7
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales, alpha = N.quantize_weight(w)
    got = N.linear(a, sa, packed, scales, alpha)
    plain = N.unswizzle_128x4(scales)
    for i in range(m):
        for j in range(0, n, 17):
            acc = 0.0
            for t in range(k):
                byte = packed[j, t // 2]
                code = (byte & 0xF) if t % 2 == 0 else (byte >> 4)
                acc += float(e4m3_decode(a[i, t])) * float(e2m1_decode(code)) * float(e4m3_decode(plain[j, t // 16]))
            from oracle.formats import bf16_round

            assert got[i, j] == bf16_round(acc * float(sa[i]) * float(alpha))


def test_activation_quantizer_is_exact_on_scaled_grid_blocks():
    # Blocks of E2M1 grid values with |max| = 6 times 2^e (gsf = 1): the block
    # scale is exactly 2^e (6 * RN(1/6) rounds to 1), the codes are the grid
    # values, and the round trip is exact.  A dropped /6, a transposed scale or
    # a swapped nibble order fails here.
    rng = np.random.default_rng(5)
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float32)
    rows = []
    for e in range(-9, 9):
        v = grid[rng.integers(0, 8, (3, 16))] * np.where(rng.random((3, 16)) < 0.5, -1, 1)
        v[:, rng.integers(0, 16)] = 6.0
        rows.append((v * np.float32(2.0**e)).reshape(1, 48))
    x = np.concatenate(rows).astype(np.float32)
    x = np.concatenate([x, np.zeros((18, 16), np.float32)], axis=1)  # one zero block per row
    packed, tiled = N.quantize_activation(x, np.float32(1.0))
    assert tiled.shape == (128, 4)
    plain = N.unswizzle_128x4(tiled)
    assert np.all(plain[18:] == 0)
    expect_sf = np.array([[0x38 + 8 * e if e >= -6 else 1 << (e + 9) for _ in range(3)] + [0]
                          for e in range(-9, 9)])
    assert np.array_equal(plain[:18], expect_sf)
    assert np.array_equal(N.dequantize_weight(packed, tiled), x.astype(np.float64))


def test_activation_quantizer_invariants_on_calibrated_rows():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((40, 256)) * rng.uniform(0.1, 10, (40, 1))).astype(np.float32)
    gsf = np.float32(2688.0) / np.float32(np.abs(x).max())
    packed, tiled = N.quantize_activation(x, gsf)
    sf = e4m3_decode(N.unswizzle_128x4(tiled)[:40]).astype(np.float64)
    q = np.empty((40, 256), np.uint8)
    q[:, 0::2], q[:, 1::2] = packed & 0xF, packed >> 4
    normal = sf >= 2.0**-6
    # The block maximum always encodes as +-6 when the block scale is normal.
    top = (q.reshape(40, 16, 16) & 7).max(axis=-1)
    assert np.all(top[normal] == 7)
    # Round-trip error: at most half the widest E2M1 step (2) of the block's
    # scale, i.e. amax_block / 6 times the scale rounding (1 + 2^-4).
    dq = N.dequantize_weight(packed, tiled) / float(gsf)
    bmax = np.abs(x).reshape(40, 16, 16).max(axis=-1)
    err = np.abs(dq - x).reshape(40, 16, 16).max(axis=-1)
    assert np.all(err[normal] <= bmax[normal] / 6 * (1 + 2.0**-4) * (1 + 1e-6))
