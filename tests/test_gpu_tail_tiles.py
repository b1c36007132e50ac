"""Partial GEMM tiles next to memory that holds NaN codes.

Each operand sits at the start of a larger buffer whose remaining bytes are
0x7f, the E4M3 NaN code, so the partial last tiles run beside readable memory
that would poison any output it reached.  The outputs must equal those from the
same operands in their own allocations, and the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as O
from tests.conftest import rel_check
from vflash_amd import kernels
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu

NAN_CODE = 0x7F


def nan_tailed(codes, extra_rows, dev):
    """``codes`` ([R, K] E4M3) copied into the first R rows of an [R + extra_rows, K]
    buffer filled with the NaN code; returns the [R, K] view."""
    rows, k = codes.shape
    buf = torch.full((rows + extra_rows, k), NAN_CODE, dtype=torch.uint8, device=dev)
    buf[:rows].copy_(codes.view(torch.uint8).to(dev))
    return buf[:rows].view(torch.float8_e4m3fn)


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def inputs(m, k, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    return x, w, s, b


# 4096 x 3088 runs 208 tiles of 256x256 (one round over 256 CUs) rather than 800
# of 128x128 (two rounds at two per CU), so the 256x256 tiling with the
# scalar-offset DMA (K % 128 == 0) is chosen; its last column of tiles holds
# only 16 weight rows.  M = 4100 adds a last row of tiles with 4 activation
# rows.  1040 x 6160 runs the 128x128 tiling with partial tiles on both edges.
@pytest.mark.parametrize("m,n", [(4096, 3088), (4100, 3088), (4100, 3072), (1040, 6160)])
def test_linear_tail_tiles_match_untailed_operands(dev, m, n):
    k = 384
    x, w, s, b = inputs(m, k, n, seed=1)
    a, sa = kernels.quantize_rows(x.to(dev))
    plain = kernels.fp8_gemm(a, sa, w.to(dev), s.to(dev), m, b.to(dev))
    tailed = kernels.fp8_gemm(nan_tailed(a, 64, dev), sa, nan_tailed(w, 64, dev), s.to(dev), m,
                              b.to(dev))
    assert torch.equal(plain, tailed)
    ref = O.w8a8_linear(x.float().numpy(), u8(w), s.reshape(-1).numpy(), b.float().numpy())
    rel_check(tailed.float().cpu().numpy(), ref)
