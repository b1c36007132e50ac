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


# One shape per GEMM tiling (csrc/fp8_gemm.hip, pick_tiling), each with a
# partial last row and column of tiles; K = 384 is a multiple of 128, so full
# tiles take the scalar-offset DMA and partial ones the vector-offset form.
#   4096 x 3088, 4100 x 3088, 4100 x 3072: 256x256 (16 or 4 weight rows, 4
#   activation rows in the last tiles); 1100 x 8208: 256x192; 1040 x 6160:
#   256x128; 700 x 6032: 128x192; 2100 x 3712: 128x128, two per CU;
#   520 x 4112: 128x128 in one round; 300 x 4112: 128x64; 257 x 528: 64x64.
@pytest.mark.parametrize("m,n", [(4096, 3088), (4100, 3088), (4100, 3072), (1100, 8208),
                                 (1040, 6160), (700, 6032), (2100, 3712), (520, 4112),
                                 (300, 4112), (257, 528)])
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
