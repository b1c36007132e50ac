"""W8A8 path restated on the CPU in numpy (test infrastructure).

Inputs and outputs are numpy arrays; bf16 tensors are carried as binary32
arrays holding bf16-representable values.  Elementwise steps use binary32
arithmetic with a bf16 rounding after each step, as the reference's kernels
do; the GEMM sum is exact (binary64 sums of E4M3 products are exact at these
sizes) and rounded once to bf16 after the two scales.
"""

from __future__ import annotations

import numpy as np

from oracle.formats import FLT_MIN, bf16_round, e4m3_decode, e4m3_encode

F32 = np.float32


def quantize_rows(x, pad: int = 16, scalar_product: bool = False):
    """Per-token E4M3 codes and scales with GEMM row padding.

    Follows src/vflash/native/h3_fp8_linear.py:18-31 (and the fused kernel
    h3_fp8_activation.py:12-28): binary32 row maximum;
    scale = max(amax / 448, FLT_MIN) if amax > 0 else 1 (IEEE binary32
    division); codes = e4m3(clamp(x / scale, -448, 448)); rows padded to a
    multiple of ``pad`` with codes 0 and scale 1.
    ``scalar_product`` forms amax / 448 as amax * RN(1/448) instead: how torch's
    GPU kernels evaluate the reference's portable expression ``maxima / 448.0``
    (a tensor divided by a Python number); its CPU kernels divide.
    Pinned by: the reference KATs (tests/test_fp8_linear.py:99-120, restated in
    tests/golden), torch's float8_e4m3fn cast, and closed-form invariants; the
    product form by torch on the GPU (tests/test_gpu_quant.py).
    """
    x = np.asarray(x, dtype=F32)
    m, k = x.shape
    m_pad = -(-m // pad) * pad if pad > 1 else m
    amax = np.max(np.abs(x), axis=1) if k else np.zeros(m, F32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        base = amax * (F32(1.0) / F32(448.0)) if scalar_product else amax / F32(448.0)
        scale = np.where(amax > 0, np.maximum(base.astype(F32), FLT_MIN), F32(1.0)).astype(F32)
        q = np.clip(x / scale[:, None], F32(-448.0), F32(448.0))
    codes = np.zeros((m_pad, k), dtype=np.uint8)
    codes[:m] = e4m3_encode(q)
    scales = np.ones(m_pad, dtype=F32)
    scales[:m] = scale
    return codes, scales


def gemm_acc(a_codes, w_codes) -> np.ndarray:
    """Exact sum_k a[m,k] * w[n,k] of E4M3 values (binary64)."""
    a = e4m3_decode(a_codes).astype(np.float64)
    w = e4m3_decode(w_codes).astype(np.float64)
    return a @ w.T


def scaled_mm(a_codes, sa, w_codes, sw) -> np.ndarray:
    """bf16(acc * sa[m] * sw[n]): the _scaled_mm call of h3_fp8_linear.py:110-117.

    The scale products are formed in binary64 and rounded once to bf16; the
    reference library's binary32 epilogue order is not observable here, so
    kernel outputs are compared to this within a relative tolerance.
    """
    acc = gemm_acc(a_codes, w_codes)
    sa = np.asarray(sa, dtype=np.float64).reshape(-1, 1)
    sw = np.asarray(sw, dtype=np.float64).reshape(1, -1)
    return bf16_round(acc * sa[: acc.shape[0]] * sw)


def add_bias(y, bias) -> np.ndarray:
    """The second rounding: bf16(y + bias) in binary32 (h3_fp8_linear.py:121)."""
    if bias is None:
        return np.asarray(y, dtype=F32)
    return bf16_round(np.asarray(y, F32) + np.asarray(bias, F32).reshape(1, -1))


def w8a8_linear(x, w_codes, sw, bias=None, scalar_product: bool = False):
    """RowFP8Execution.linear in w8a8 mode (h3_fp8_linear.py:98-121) for a 2-D input;
    ``scalar_product`` selects the portable quantizer as torch evaluates it on a GPU."""
    codes, sa = quantize_rows(x, scalar_product=scalar_product)
    m = np.asarray(x).shape[0]
    return add_bias(scaled_mm(codes[:m], sa[:m], w_codes, sw), bias)


# The binary32 constants a binary32 GELU-tanh kernel multiplies by (torch's
# gelu(approximate="tanh") forms them as float: sqrt(2) * 2/sqrt(pi) * 0.5 and 0.044715).
GELU_BETA = float(F32(0.7978845608028654))
GELU_KAPPA = float(F32(0.044715))


def _bf16_through_f32(v) -> np.ndarray:
    """Real values (binary64) stored as bf16 by a binary32 kernel: rounded to
    binary32, then to bf16, each to nearest with ties to even."""
    with np.errstate(over="ignore"):
        return bf16_round(np.asarray(v, np.float64).astype(F32))


def gelu_tanh(y) -> np.ndarray:
    """GELU with the tanh approximation, 0.5 y (1 + tanh(u)) with
    u = beta (y + kappa y^3), of bf16 values, as a binary32 kernel with correctly
    rounded steps stores it: the function value rounded to binary32, then to
    bf16.  It is evaluated in binary64 as y / (1 + exp(-2u)), the same function
    without the cancellation of 1 + tanh(u) at negative y.  +inf gives +inf,
    -inf gives NaN (-inf * 0 in the tanh form), NaN stays NaN.

    The reference's FFN has no GELU (its activation is SiLU-mul); this is the
    textbook tanh form of torch.nn.functional.gelu(approximate="tanh").  Pinned
    against a 60-digit decimal evaluation over every bf16 value and against
    torch's binary64 gelu (tests/test_oracle_fp8.py)."""
    y = np.asarray(y, dtype=F32).astype(np.float64)
    u = GELU_BETA * (y + GELU_KAPPA * y * y * y)
    with np.errstate(over="ignore", invalid="ignore"):
        v = y / (1.0 + np.exp(-2.0 * u))
    return _bf16_through_f32(v)


def silu(g) -> np.ndarray:
    """bf16(silu(g)) of bf16 values: the reference's binary32 formula
    g / (1 + exp(-g)) (h3_fused_ops.py:205) with each step correctly rounded to
    binary32 -- e = RN(exp(-g)) (infinity where it overflows, below g = -88.72),
    d = RN(1 + e), q = RN(g / d) -- then rounded to bf16.  Overflow gives -0 for
    g <= -89, as the binary32 kernels do; +inf gives +inf, -inf NaN, NaN stays
    NaN.  Pinned by a 60-digit evaluation of the exponential and against torch's
    silu (tests/test_oracle_fp8.py)."""
    g = np.asarray(g, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(F32)
        q = g / (F32(1.0) + e)
    return bf16_round(q)


def silu_mul(packed) -> np.ndarray:
    """H3 SwiGLU activation of a packed bf16 [.., 2F] projection output:
    value, gate = packed.chunk(2, -1); bf16(value * bf16(silu(gate)))
    (h3_native_denoiser.py:369-373 with eager bf16 tensors; the fused kernel
    h3_fused_ops.py:184-224 keeps the same two roundings).  The product of two
    bf16 values is exact in binary32, so its only rounding is the one to bf16."""
    packed = np.asarray(packed, F32)
    f = packed.shape[-1] // 2
    value, gate = packed[..., :f], packed[..., f:]
    with np.errstate(invalid="ignore"):
        return bf16_round(value.astype(np.float64) * silu(gate).astype(np.float64))


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """torch.nn.functional.rms_norm of a bf16 [.., H] input with a bf16 weight,
    as the reference calls it (src/vflash/native/h3_native_denoiser.py:231-243):
    rstd = 1 / sqrt(sum(x^2) / H + eps) in binary32, n = bf16(x * rstd * w), one
    rounding; ``weight`` None leaves out the weight.  The sum of squares is
    formed in binary64 and rounded once to binary32 (any binary32 summation
    order agrees with it to a few units in the last place).  Pinned against
    torch's CPU rms_norm: bit-exact where the sum is exact in binary32, within
    one bf16 step otherwise."""
    x = np.asarray(x, F32)
    h = x.shape[-1]
    ss = F32((x.astype(np.float64) ** 2).sum(-1, keepdims=True))
    rstd = F32(1.0) / np.sqrt(ss / F32(h) + F32(eps))
    t = x * rstd
    return bf16_round(t if weight is None else t * np.asarray(weight, F32))


def modulate(n, scale, shift) -> np.ndarray:
    """adaLN modulation n * (1 + scale) + shift with eager bf16 tensors
    (h3_native_denoiser.py:363-364; the fused kernel h3_fused_ops.py:52-122 keeps
    its three roundings): bf16(bf16(n * bf16(1 + scale)) + shift).  Pinned
    against torch's eager bf16 expression."""
    one_plus = bf16_round(F32(1.0) + np.asarray(scale, F32))
    return bf16_round(bf16_round(np.asarray(n, F32) * one_plus) + np.asarray(shift, F32))


def gate_residual(residual, gate, y) -> np.ndarray:
    """bf16(residual + bf16(gate * y)) in binary32 (h3_fused_ops.py:153-170)."""
    gated = bf16_round(np.asarray(gate, F32) * np.asarray(y, F32))
    return bf16_round(np.asarray(residual, F32) + gated)


def lora_delta(x, lora_a, lora_b, scaling: float = 1.0, strength: float = 1.0):
    """The adapter hook's delta (src/vflash/adapters/h3_reference_lora.py:80-89):
    t = bf16(x A^T); d = bf16(t B^T); bf16(d * scaling) if scaling != 1;
    bf16(d * strength) if strength != 1.  Sums exact in binary64."""
    t = bf16_round(np.asarray(x, np.float64) @ np.asarray(lora_a, np.float64).T)
    d = bf16_round(t.astype(np.float64) @ np.asarray(lora_b, np.float64).T)
    if scaling != 1.0:
        d = bf16_round(d * F32(scaling))
    if strength != 1.0:
        d = bf16_round(d * F32(strength))
    return d


def lora_merge(base, delta) -> np.ndarray:
    """bf16(result + delta) (h3_reference_lora.py:90)."""
    return bf16_round(np.asarray(base, F32) + np.asarray(delta, F32))


def adapted(base, x, adapter, strength: float = 1.0) -> np.ndarray:
    """A projection with a low-rank residual merged in, bf16(base + delta) with
    delta = lora_delta(x, down, up, scaling): the native block's _adapted_linear
    (src/vflash/native/h3_native_denoiser.py:280-299, 318-325) and its fused
    merges (h3_fused_ops.py:297-340, 765-800), which round the scaled delta and
    the sum the same way.  ``adapter`` is (down [r, K], up [N, r], scaling) or
    None (the base unchanged)."""
    if adapter is None:
        return np.asarray(base, F32)
    down, up, scaling = adapter
    return lora_merge(base, lora_delta(x, down, up, scaling, strength))


def qkv_adapted(base, x, adapters) -> np.ndarray:
    """The merged QKV projection with its Q/K/V residual pack: third b of the
    output takes adapter b (h3_native_denoiser.py:301-316; the fused merges
    h3_fused_ops.py:802-838, 954-980 round each branch the same way)."""
    base = np.asarray(base, F32)
    third = base.shape[1] // 3
    return np.concatenate(
        [adapted(base[:, b * third : (b + 1) * third], x, adapters[b]) for b in range(3)], axis=1
    )


def adapted_gate_residual(residual, gate, base, x, adapter) -> np.ndarray:
    """bf16(residual + bf16(gate * bf16(base + delta))): _adapted_gate_residual
    (h3_native_denoiser.py:327-338) and strict_adapter_gate_residual_kernel
    (h3_fused_ops.py:341-418)."""
    return gate_residual(residual, gate, adapted(base, x, adapter))


def ffn(x, up_codes, up_scale, up_bias, down_codes, down_scale, down_bias, gate, residual,
        activation: str = "gelu_tanh", up_adapter=None, down_adapter=None):
    """The FFN chain of this path: up + bias (+ the input adapter), activation
    (GELU-tanh, or the H3 SwiGLU on a packed [2F, H] up projection), per-token
    requant, down + bias (+ the output adapter on the activation), gate-residual
    (h3_native_denoiser.py:375-382, 563-576).  Returns (g, h_codes, h_scales, out)."""
    x = np.asarray(x, F32)
    m = x.shape[0]
    up = adapted(w8a8_linear(x, up_codes, up_scale, up_bias), x, up_adapter)
    g = silu_mul(up) if activation == "swiglu" else gelu_tanh(up)
    h_codes, h_scales = quantize_rows(g)
    y = add_bias(scaled_mm(h_codes[:m], h_scales[:m], down_codes, down_scale), down_bias)
    return g, h_codes, h_scales, gate_residual(residual, gate, adapted(y, g, down_adapter))
