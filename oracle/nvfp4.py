"""NVFP4 path restated on the CPU in numpy (test infrastructure).

The reference's NVFP4 arithmetic lives in FlashInfer 0.6.18 (pyproject.toml:25;
nvfp4_quantize / mm_fp4 with the CUTLASS backend, called at
src/vflash/native/h3_nvfp4_linear.py:102-130), which is not vendored and not
installed here.  PARITY UNPINNED against FlashInfer: the weight packing, the
activation quantization (FlashInfer's published per-block recipe, restated
below with correctly rounded reciprocals where FlashInfer uses the hardware's
approximate ones), the block-scale rounding and the 128x4 order are pinned by
closed forms, the OCP E2M1/E4M3 tables and brute force on small cases, not by
reference vectors.
"""

from __future__ import annotations

import numpy as np

from oracle.formats import bf16_round, e2m1_decode, e2m1_encode, e4m3_decode, e4m3_encode

F32 = np.float32


def scale_offset_128x4(n, j, k_blocks: int):
    """Storage offset of the scale of row n, K block j (16 elements) in the 128x4
    tiled order: 128-row x 4-block tiles of 512 bytes, tiles ordered row-tile
    major; inside a tile, offset (n % 32) * 16 + ((n % 128) // 32) * 4 + j % 4."""
    k_tiles = (k_blocks + 3) // 4
    n = np.asarray(n)
    j = np.asarray(j)
    return (n // 128) * (k_tiles * 512) + (j // 4) * 512 + (n % 32) * 16 + ((n % 128) // 32) * 4 + j % 4


def swizzle_128x4(plain):
    plain = np.asarray(plain)
    n, kb = plain.shape
    out = np.empty(n * kb, dtype=plain.dtype)
    nn, jj = np.meshgrid(np.arange(n), np.arange(kb), indexing="ij")
    out[scale_offset_128x4(nn, jj, kb).reshape(-1)] = plain.reshape(-1)
    return out.reshape(n, kb)


def unswizzle_128x4(tiled):
    tiled = np.asarray(tiled)
    n, kb = tiled.shape
    nn, jj = np.meshgrid(np.arange(n), np.arange(kb), indexing="ij")
    return tiled.reshape(-1)[scale_offset_128x4(nn, jj, kb)]


def quantize_weight(w):
    """NVFP4 packing convention (binary32 arithmetic):
    gsf = 2688 / amax|W|; sf = e4m3(min(amax_block * (gsf / 6), 448));
    q = e2m1(clamp(w * (gsf / sf), -6, 6)) (0 where sf == 0); alpha = 1 / gsf.
    Returns (packed [N, K/2] u8, tiled scales [N, K/16] u8, alpha f32)."""
    w = np.asarray(w, F32)
    n, k = w.shape
    amax = np.max(np.abs(w))
    gsf = F32(2688.0) / F32(amax)
    blocks = w.reshape(n, k // 16, 16)
    bmax = np.max(np.abs(blocks), axis=-1)
    sf = e4m3_encode(np.minimum(bmax * (gsf / F32(6.0)), F32(448.0)))
    sf_f = e4m3_decode(sf)
    with np.errstate(divide="ignore"):
        mult = np.where(sf_f > 0, gsf / sf_f, F32(0.0)).astype(F32)
    q = e2m1_encode(np.clip(blocks * mult[..., None], F32(-6.0), F32(6.0))).reshape(n, k)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, swizzle_128x4(sf), F32(F32(1.0) / gsf)


def dequantize_weight(packed, tiled_scales) -> np.ndarray:
    """Exact e2m1 * e4m3 block-scale values [N, K] (binary64), without alpha.
    ``tiled_scales`` may have more (padding) rows than ``packed``."""
    packed = np.asarray(packed, np.uint8)
    n, half = packed.shape
    q = np.empty((n, 2 * half), dtype=np.uint8)
    q[:, 0::2] = packed & 0xF
    q[:, 1::2] = packed >> 4
    sf = e4m3_decode(unswizzle_128x4(tiled_scales)[:n]).astype(np.float64)
    return e2m1_decode(q).astype(np.float64) * np.repeat(sf, 16, axis=1)


def linear(a_codes, sa, packed, tiled_scales, alpha, bias=None):
    """bf16(bf16(sum_k a * w_dq * sa[m] * alpha) + bias) with an exact sum."""
    a = e4m3_decode(a_codes).astype(np.float64)
    acc = a @ dequantize_weight(packed, tiled_scales).T
    y = bf16_round(acc * np.asarray(sa, np.float64).reshape(-1, 1)[: acc.shape[0]] * float(alpha))
    if bias is None:
        return y
    return bf16_round(y + np.asarray(bias, F32).reshape(1, -1))


SIXTH = F32(1.0) / F32(6.0)  # RN(1/6)


def quantize_activation(x, global_sf):
    """NVFP4 activation quantization of nvfp4_quantize(x, input_scale) as the
    reference calls it (h3_nvfp4_linear.py:102): per row and 16-element block,
    in binary32,
      sf    = e4m3(min(gsf * (amax_block * RN(1/6)), 448))     (RNE, satfinite)
      scale = sf != 0 ? 1 / (sf * (1 / gsf)) : 0
      q     = e2m1(clamp(x * scale, -6, 6))                    (RNE, satfinite)
    FlashInfer forms the two reciprocals with the hardware's approximate
    reciprocal; here they are correctly rounded (parity unpinned: a one-ulp
    difference of ``scale`` moves a code only next to an E2M1 rounding
    boundary).  Returns packed codes [M, K/2] (element 2j in the low nibble)
    and block scales in the 128x4 order with the rows padded to a multiple of
    128 (padding scales 0), the layout h3_nvfp4_linear.py:103-111 checks."""
    x = np.asarray(x, F32)
    m, k = x.shape
    gsf = F32(global_sf)
    blocks = x.reshape(m, k // 16, 16)
    bmax = np.max(np.abs(blocks), axis=-1)
    sf = e4m3_encode(np.minimum(gsf * (bmax * SIXTH), F32(448.0)))
    sf_f = e4m3_decode(sf)
    with np.errstate(divide="ignore", over="ignore"):
        scale = np.where(sf_f > 0, F32(1.0) / (sf_f * (F32(1.0) / gsf)), F32(0.0)).astype(F32)
    q = e2m1_encode(np.clip(blocks * scale[..., None], F32(-6.0), F32(6.0))).reshape(m, k)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    m_pad = -(-m // 128) * 128
    plain = np.zeros((m_pad, k // 16), dtype=np.uint8)
    plain[:m] = sf
    return packed, swizzle_128x4(plain)


def linear_w4a4(a_packed, a_tiled_scales, packed, tiled_scales, alpha, bias=None):
    """mm_fp4 then + bias (h3_nvfp4_linear.py:114-139): bf16(alpha * sum_k a_dq *
    w_dq) with an exact sum, then bf16(y + bias).  ``alpha`` is the output
    scale, weight.alpha / weight.input_scale."""
    acc = dequantize_weight(a_packed, a_tiled_scales) @ dequantize_weight(packed, tiled_scales).T
    y = bf16_round(acc * float(alpha))
    if bias is None:
        return y
    return bf16_round(y + np.asarray(bias, F32).reshape(1, -1))
