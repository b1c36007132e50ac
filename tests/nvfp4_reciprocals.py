"""How far approximate reciprocals can move the NVFP4 activation quantizer.

FlashInfer's nvfp4_quantize (0.6.18, called at h3_nvfp4_linear.py:102) forms,
per 16-element block of a row,
    sf    = e4m3(min(gsf * (amax * r6), 448))        r6    ~ 1/6
    scale = r_out(sf * r_g)                           r_g   ~ 1/gsf, r_out(p) ~ 1/p
    q     = e2m1(clamp(x * scale, -6, 6))
with the GPU's approximate reciprocal for r6, r_g and r_out, whereas the oracle
(oracle/nvfp4.py:quantize_activation) and the HIP kernel use correctly rounded
ones.  The PTX ISA bounds the approximate binary32 reciprocal (rcp.approx) to
one ulp of the exact value, so each of the three is one of RN(1/a) - ulp,
RN(1/a), RN(1/a) + ulp.  ``divergence`` applies all 27 combinations to every
block and counts the blocks whose scale or codes differ from the correctly
rounded result under at least one of them: an upper bound on what the
reciprocal choice can change.

Every step is an exact binary32 operation in torch (products, the E4M3 cast
with ties to even) or a table formed on the host in numpy (the reciprocals of
sf * r_g: sf is one of 127 E4M3 values), so the count is exact on CPU and GPU.
"""

from __future__ import annotations

import numpy as np
import torch

E2M1_LIMIT = 6.0


def _neighbours(r: np.float32):
    return [np.nextafter(r, np.float32(-np.inf)), r, np.nextafter(r, np.float32(np.inf))]


def e2m1_codes(v: torch.Tensor) -> torch.Tensor:
    """OCP E2M1 codes (0..15) of binary32 values already clamped to [-6, 6], ties
    to even: 0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4
    (codes 0..7 are 0, .5, 1, 1.5, 2, 3, 4, 6)."""
    a = v.abs()
    c = ((a > 0.25).to(torch.uint8) + (a >= 0.75) + (a > 1.25) + (a >= 1.75) + (a > 2.5)
         + (a >= 3.5) + (a > 5.0))
    return c | (torch.signbit(v).to(torch.uint8) << 3)


def divergence(x: torch.Tensor, gsf: float):
    """(blocks, blocks whose E4M3 scale can change, blocks whose scale or codes can
    change) for bf16/f32 activations ``x`` [M, K] and the global scale ``gsf``."""
    gsf32 = np.float32(gsf)
    r6s = _neighbours(np.float32(1.0) / np.float32(6.0))
    rgs = _neighbours(np.float32(1.0) / gsf32)
    # scale table [rg variant][r_out variant][sf code 0..127]: code 127 is NaN, never produced.
    sf_values = (torch.arange(128, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy())
    table = np.zeros((3, 3, 128), np.float32)
    with np.errstate(divide="ignore"):
        for i, rg in enumerate(rgs):
            p = (sf_values * rg).astype(np.float32)
            r = (np.float32(1.0) / p).astype(np.float32)
            for j in range(3):
                table[i, j] = np.where(sf_values > 0, [_neighbours(v)[j] for v in r], 0.0)
    table_t = torch.from_numpy(table).to(x.device)
    blocks = x.float().reshape(x.shape[0], -1, 16)
    amax = blocks.abs().amax(dim=-1)
    sf_codes = []
    for r6 in r6s:
        v = torch.clamp_max(torch.tensor(gsf32, device=x.device) * (amax * torch.tensor(r6, device=x.device)), 448.0)
        sf_codes.append(v.to(torch.float8_e4m3fn).view(torch.uint8).long())
    ref_sf = sf_codes[1]
    ref_q = e2m1_codes(torch.clamp(blocks * table_t[1, 1][ref_sf].unsqueeze(-1), -E2M1_LIMIT, E2M1_LIMIT))
    sf_moved = torch.zeros_like(amax, dtype=torch.bool)
    moved = torch.zeros_like(amax, dtype=torch.bool)
    for sf in sf_codes:
        sf_moved |= sf != ref_sf
        for i in range(3):
            for j in range(3):
                q = e2m1_codes(torch.clamp(blocks * table_t[i, j][sf].unsqueeze(-1), -E2M1_LIMIT, E2M1_LIMIT))
                moved |= (q != ref_q).any(dim=-1)
    moved |= sf_moved
    return amax.numel(), int(sf_moved.sum()), int(moved.sum()), ref_sf, ref_q
