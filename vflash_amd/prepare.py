"""Offline weight preparation: FP8 row codes and NVFP4 packed weights.

The reference receives prepared FP8 codes/``row_scale`` and NVFP4 packs as
assets and contains no weight quantizer (src/vflash/native/h3_fp8_runtime.py:1-6,
src/vflash/adapters/h3_qad.py:104-129).  These are the conventions of this
package, written with torch ops (any device); they are not on the per-call
path.

FP8 rows: the activation quantizer's arithmetic applied to each weight row in
binary32: ``s = max(amax / 448, FLT_MIN)`` (1 for a zero row),
``code = e4m3_rne(clamp(w / s, -448, 448))``.

NVFP4 (E2M1 values, E4M3 scale per 16-element K block, fp32 global):
  ``gsf = 2688 / amax(|W|)`` (2688 = 448 * 6)
  ``sf  = e4m3_rne(min(amax_block * (gsf / 6), 448))``
  ``q   = e2m1_rne(clamp(w * (gsf / sf), -6, 6))`` (q = 0 where sf = 0)
  ``alpha = 1 / gsf``, so ``w ~= e2m1(q) * sf * alpha``.
Packing: element 2j in the low nibble of byte j, 2j+1 in the high nibble.
Block scales are stored in the 128x4 tiled order (``swizzle_128x4``).
"""

from __future__ import annotations

import torch

FLT_MIN = torch.finfo(torch.float32).tiny


def quantize_weight_rows(weight: torch.Tensor):
    """E4M3 codes [N, K] and fp32 row scales [N, 1] of a real weight matrix."""
    floats = weight.float()
    maxima = floats.abs().amax(dim=1, keepdim=True)
    # A tensor divisor keeps IEEE division on every device (see _quantize_activation_torch).
    limit = torch.full((), 448.0, dtype=torch.float32, device=floats.device)
    scale = torch.where(maxima > 0, (maxima / limit).clamp_min(FLT_MIN), torch.ones_like(maxima))
    codes = (floats / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return codes, scale


def e2m1_codes(values: torch.Tensor) -> torch.Tensor:
    """Round binary32 values (already within [-6, 6]) to E2M1 codes, ties to even;
    the sign bit follows the input's sign, -0 included."""
    a = values.abs()
    code = (
        (a > 0.25).to(torch.uint8)
        + (a >= 0.75).to(torch.uint8)
        + (a > 1.25).to(torch.uint8)
        + (a >= 1.75).to(torch.uint8)
        + (a > 2.5).to(torch.uint8)
        + (a >= 3.5).to(torch.uint8)
        + (a > 5.0).to(torch.uint8)
    )
    return code | (torch.signbit(values).to(torch.uint8) << 3)


def scale_offsets_128x4(n: int, k_blocks: int, device=None) -> torch.Tensor:
    """Storage offset of each (row, K block) scale in the 128x4 tiled order."""
    rows = torch.arange(n, device=device).unsqueeze(1)
    cols = torch.arange(k_blocks, device=device).unsqueeze(0)
    k_tiles = (k_blocks + 3) // 4
    return (
        (rows // 128) * (k_tiles * 512)
        + (cols // 4) * 512
        + (rows % 32) * 16
        + ((rows % 128) // 32) * 4
        + (cols % 4)
    )


def swizzle_128x4(plain: torch.Tensor) -> torch.Tensor:
    """Row-major [N, K/16] scale bytes -> the same shape in 128x4 tiled storage."""
    n, kb = plain.shape
    if n % 128 or kb % 4:
        raise ValueError("128x4 tiling needs N % 128 == 0 and (K/16) % 4 == 0")
    out = torch.empty(n * kb, dtype=plain.dtype, device=plain.device)
    out[scale_offsets_128x4(n, kb, plain.device).reshape(-1)] = plain.reshape(-1)
    return out.view(n, kb)


def unswizzle_128x4(tiled: torch.Tensor) -> torch.Tensor:
    n, kb = tiled.shape
    return tiled.reshape(-1)[scale_offsets_128x4(n, kb, tiled.device)].contiguous()


def quantize_nvfp4_weight(weight: torch.Tensor, input_scale: float = 1.0):
    """Pack a real [N, K] weight as NVFP4: returns (packed, tiled scales, alpha, input_scale)."""
    n, k = weight.shape
    if n % 128 or k % 64:
        raise ValueError("NVFP4 packing needs N % 128 == 0 and K % 64 == 0")
    w = weight.float()
    amax = w.abs().amax()
    if not bool(amax > 0):
        raise ValueError("an all-zero weight has no NVFP4 global scale")
    gsf = torch.tensor(2688.0, dtype=torch.float32, device=w.device) / amax
    blocks = w.reshape(n, k // 16, 16)
    bmax = blocks.abs().amax(dim=-1)
    sf = (bmax * (gsf / 6.0)).clamp(max=448.0).to(torch.float8_e4m3fn)
    sf_f = sf.float()
    mult = torch.where(sf_f > 0, gsf / sf_f, torch.zeros_like(sf_f))
    q = e2m1_codes((blocks * mult.unsqueeze(-1)).clamp(-6.0, 6.0)).reshape(n, k)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    scales = swizzle_128x4(sf.view(torch.uint8).contiguous())
    alpha = (1.0 / gsf).to(torch.float32).reshape(())
    return packed, scales, alpha, torch.tensor(input_scale, dtype=torch.float32, device=w.device)
