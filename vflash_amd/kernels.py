"""Tensor-level wrappers of the HIP kernels (one call = one C-ABI entry).

Each wrapper checks dtypes, devices and layouts, allocates its outputs with
``torch.empty`` on the input's device and enqueues on the current stream.
No wrapper synchronizes.  Unsupported devices raise ``ValueError``.
"""

from __future__ import annotations

import ctypes

import torch

from vflash_amd import _lib
from vflash_amd._lib import call, ptr, stream_of

E4M3 = torch.float8_e4m3fn


def require_device(*tensors: torch.Tensor) -> torch.device:
    device = tensors[0].device
    for t in tensors[1:]:
        if t is not None and t.device != device:
            raise ValueError("all operands must share one device")
    if not _lib.is_gfx950(device):
        raise ValueError("the HIP quantized-linear kernels require a gfx950 (MI355X) device")
    return device


def padded_rows(rows: int) -> int:
    return (rows + 15) // 16 * 16


def quantize_rows(matrix: torch.Tensor, pad_to: int = 16):
    """Per-token E4M3 codes [ceil16(M), K] and fp32 scales [ceil16(M), 1]."""
    if matrix.dtype != torch.bfloat16 or matrix.ndim != 2 or matrix.stride(1) != 1:
        raise ValueError("row quantization requires a 2-D BF16 matrix with unit column stride")
    device = require_device(matrix)
    m, k = matrix.shape
    m_pad = (m + pad_to - 1) // pad_to * pad_to
    codes = torch.empty((m_pad, k), device=device, dtype=E4M3)
    scales = torch.empty((m_pad, 1), device=device, dtype=torch.float32)
    if m_pad:
        call("vflash_quantize_rows_e4m3", ptr(matrix), m, k, matrix.stride(0), ptr(codes),
             ptr(scales), m_pad, stream_of(device))
    return codes, scales


def rmsnorm_modulate_quantize(matrix, norm_weight, scale, shift, *, eps, index=None,
                              keep_values=False, pad_to: int = 16):
    """RMSNorm + adaLN modulation + per-token E4M3 quantization in one pass.

    ``matrix`` is bf16 ``[M, K]`` with unit column stride, ``norm_weight`` bf16
    ``[K]`` or None.  ``scale`` and ``shift`` are bf16 ``[R, K]`` with unit column
    stride and any row stride (for instance ``table[:, j, :]`` of a ``[R, 6, K]``
    adaLN table).  Row r of ``matrix`` uses modulation row ``r % R``, or
    ``index[r % T]`` for an int64 ``index`` of length T.  Returns codes
    ``[ceil16(M), K]``, scales ``[ceil16(M), 1]`` and, with ``keep_values``, the
    modulated bf16 ``[M, K]`` (else None).
    """
    if matrix.dtype != torch.bfloat16 or matrix.ndim != 2 or matrix.stride(1) != 1:
        raise ValueError("the fused norm/modulation needs a 2-D BF16 matrix with unit column stride")
    m, k = matrix.shape
    for t in (scale, shift):
        if t.dtype != torch.bfloat16 or t.ndim != 2 or t.shape[1] != k or t.stride(1) != 1:
            raise ValueError("modulation rows must be BF16 [R, K] with unit column stride")
    if scale.shape != shift.shape:
        raise ValueError("scale and shift must have the same rows")
    if norm_weight is not None and (
        norm_weight.dtype != torch.bfloat16 or norm_weight.shape != (k,) or not norm_weight.is_contiguous()
    ):
        raise ValueError("the RMSNorm weight must be a contiguous BF16 [K] vector")
    if m == 0:
        # No tokens (an empty sequence gathers no modulation rows): empty outputs.
        device = require_device(matrix, scale, shift, norm_weight, index)
        codes = torch.empty((0, k), device=device, dtype=E4M3)
        scales = torch.empty((0, 1), device=device, dtype=torch.float32)
        values = torch.empty((0, k), device=device, dtype=torch.bfloat16) if keep_values else None
        return codes, scales, values
    if index is not None:
        if index.dtype != torch.int64 or index.ndim != 1 or not index.is_contiguous() or index.numel() < 1:
            raise ValueError("modulation indices must be a contiguous int64 vector")
        tokens = index.numel()
    else:
        tokens = scale.shape[0]
    if tokens < 1 or m % tokens:
        raise ValueError("activation rows must be a whole number of modulated token blocks")
    device = require_device(matrix, scale, shift, norm_weight, index)
    m_pad = (m + pad_to - 1) // pad_to * pad_to
    codes = torch.empty((m_pad, k), device=device, dtype=E4M3)
    scales = torch.empty((m_pad, 1), device=device, dtype=torch.float32)
    values = torch.empty((m, k), device=device, dtype=torch.bfloat16) if keep_values else None
    call("vflash_rmsnorm_modulate_quantize_e4m3", ptr(matrix), m, k, matrix.stride(0),
         ptr(norm_weight), float(eps), ptr(scale), scale.stride(0), ptr(shift), shift.stride(0),
         tokens, ptr(index), scale.shape[0], ptr(values), k, ptr(codes), ptr(scales), m_pad,
         stream_of(device))
    return codes, scales, values


def _gemm_operands(codes, act_scale, weight, w_scale, rows, bias):
    if codes.dtype != E4M3 or weight.dtype != E4M3 or codes.ndim != 2 or weight.ndim != 2:
        raise ValueError("E4M3 GEMM operands must be 2-D float8_e4m3fn matrices")
    if codes.stride(1) != 1 or weight.stride(1) != 1 or codes.shape[1] != weight.shape[1]:
        raise ValueError("E4M3 GEMM operands must share K with unit column stride")
    if act_scale.dtype != torch.float32 or w_scale.dtype != torch.float32:
        raise ValueError("GEMM scales must be fp32")
    if not act_scale.is_contiguous() or not w_scale.is_contiguous():
        raise ValueError("GEMM scales must be contiguous")
    if act_scale.numel() < rows or w_scale.numel() != weight.shape[0] or codes.shape[0] < rows:
        raise ValueError("GEMM scales do not cover the operands")
    if bias is not None and (
        bias.dtype != torch.bfloat16 or bias.shape != (weight.shape[0],) or not bias.is_contiguous()
    ):
        raise ValueError("GEMM bias must be a contiguous BF16 vector of the output width")
    return require_device(codes, act_scale, weight, w_scale, bias)


def fp8_gemm(codes, act_scale, weight, w_scale, rows, bias=None, out=None):
    """out[rows, N] = bf16(bf16(codes . weight^T * act_scale * w_scale) + bias)."""
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    if out is None:
        out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
    if (out.dtype != torch.bfloat16 or out.shape != (rows, n) or out.stride(1) != 1
            or out.device != device):
        raise ValueError("GEMM output must be BF16 [rows, N] with unit column stride")
    if rows:
        call("vflash_fp8_linear", ptr(codes), ptr(act_scale), codes.stride(0), ptr(weight),
             ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(out), out.stride(0),
             stream_of(device))
    return out


def fp8_gemm_planes(codes, act_scale, weight, w_scale, rows, planes, bias=None):
    """Merged projection written as ``planes`` contiguous [rows, N / planes] matrices.

    Returns a tensor of shape [planes, rows, N / planes].
    """
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    if planes < 1 or n % planes:
        raise ValueError("the merged width must split evenly into planes")
    cols = n // planes
    out = torch.empty((planes, rows, cols), device=device, dtype=torch.bfloat16)
    if rows:
        call("vflash_fp8_linear_planes", ptr(codes), ptr(act_scale), codes.stride(0), ptr(weight),
             ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(out), cols, cols,
             rows * cols, stream_of(device))
    return out


def gelu_quantize_rows(y, pad_to: int = 16, keep_values: bool = False):
    """E4M3 codes [ceil16(M), K] and fp32 scales [ceil16(M), 1] of g = bf16(gelu_tanh(y)),
    and g itself (bf16 [M, K]) with ``keep_values`` (else None)."""
    if y.dtype != torch.bfloat16 or y.ndim != 2 or y.stride(1) != 1:
        raise ValueError("the GELU quantizer requires a 2-D BF16 matrix with unit column stride")
    m, k = y.shape
    if k % 8 or k > 16384 or y.stride(0) % 8 or y.data_ptr() % 16:
        raise ValueError("the GELU quantizer needs K % 8 == 0, K <= 16384 and 16-byte aligned rows")
    device = require_device(y)
    m_pad = (m + pad_to - 1) // pad_to * pad_to
    codes = torch.empty((m_pad, k), device=device, dtype=E4M3)
    scales = torch.empty((m_pad, 1), device=device, dtype=torch.float32)
    g = torch.empty((m, k), device=device, dtype=torch.bfloat16) if keep_values else None
    if m:
        call("vflash_gelu_quantize_rows_e4m3", ptr(y), m, k, y.stride(0), ptr(g), k, ptr(codes),
             ptr(scales), m_pad, stream_of(device))
    return codes, scales, g


def swiglu_parts(n: int) -> int:
    return int(_lib.library().vflash_swiglu_parts(n))


def fp8_gemm_swiglu(codes, act_scale, weight, w_scale, rows, bias=None, lora=None):
    """h = bf16(value * bf16(silu(gate))) of the packed projection ``weight``
    ([2F, K]: value rows, then gate rows), plus per-row |h| maxima per
    128-column group.  ``lora`` (``LoraOperands``, B of shape [2F, rank]) merges
    the adapter delta into value and gate columns before the activation."""
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    if n % 256:
        raise ValueError("SwiGLU projections need 2F rows with F a multiple of 128")
    h = torch.empty((rows, n // 2), device=device, dtype=torch.bfloat16)
    amax = torch.empty((rows, swiglu_parts(n)), device=device, dtype=torch.float32)
    if rows:
        if lora is None:
            call("vflash_fp8_linear_swiglu", ptr(codes), ptr(act_scale), codes.stride(0), ptr(weight),
                 ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(h), h.stride(0),
                 ptr(amax), stream_of(device))
        else:
            t, ldt, b, ldb = lora.operands(rows, n, device)
            call("vflash_fp8_linear_swiglu_lora", ptr(codes), ptr(act_scale), codes.stride(0),
                 ptr(weight), ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(t), ldt,
                 ptr(b), ldb, lora.rank, float(lora.scale), float(lora.strength), ptr(h),
                 h.stride(0), ptr(amax), stream_of(device))
    return h, amax


def fp8_gemm_swiglu_quantize_noalloc(codes, act_scale, weight, w_scale, rows, bias, h, h_codes,
                                     h_scales):
    """fp8_gemm_swiglu + requant_rows in one C-ABI call that allocates nothing: the
    per-row partial maxima stay in the library's static device scratch.  The
    outputs are the caller's: ``h`` bf16 [rows, F], ``h_codes`` E4M3 [ceil16(rows), F]
    and ``h_scales`` fp32 [ceil16(rows), 1]; this wrapper allocates nothing either.
    Calls that overlap on one GPU share the scratch and must be serialized."""
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    f = n // 2
    m_pad = h_codes.shape[0]
    if n % 256 or h.dtype != torch.bfloat16 or h.shape != (rows, f) or h.stride(1) != 1:
        raise ValueError("SwiGLU output must be BF16 [rows, F] with F a multiple of 128")
    if h_codes.dtype != E4M3 or h_codes.shape[1] != f or not h_codes.is_contiguous() or m_pad < rows:
        raise ValueError("requantized codes must be a contiguous E4M3 [>= rows, F] matrix")
    if (h_scales.dtype != torch.float32 or h_scales.numel() != m_pad
            or not h_scales.is_contiguous()):
        raise ValueError("requantization scales must be contiguous fp32, one per code row")
    require_device(h, h_codes, h_scales)
    if rows:
        call("vflash_fp8_linear_swiglu_quantize_noalloc", ptr(codes), ptr(act_scale), codes.stride(0),
             ptr(weight), ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(h), h.stride(0),
             ptr(h_codes), ptr(h_scales), m_pad, stream_of(device))
    return h, h_codes, h_scales


def requant_rows(g, amax_part, pad_to: int = 16):
    """E4M3 codes/scales of ``g`` using its epilogue row maxima."""
    if g.dtype != torch.bfloat16 or g.ndim != 2 or g.stride(1) != 1:
        raise ValueError("requantization requires a 2-D BF16 matrix with unit column stride")
    if amax_part.dtype != torch.float32 or amax_part.shape[0] != g.shape[0]:
        raise ValueError("row maxima must be fp32 [rows, parts]")
    if not amax_part.is_contiguous():
        raise ValueError("row maxima must be contiguous")
    device = require_device(g, amax_part)
    m, k = g.shape
    m_pad = (m + pad_to - 1) // pad_to * pad_to
    codes = torch.empty((m_pad, k), device=device, dtype=E4M3)
    scales = torch.empty((m_pad, 1), device=device, dtype=torch.float32)
    if m:
        call("vflash_requant_rows_e4m3", ptr(g), m, k, g.stride(0), ptr(amax_part),
             amax_part.shape[1], ptr(codes), ptr(scales), m_pad, stream_of(device))
    return codes, scales


def fp8_gemm_gate_residual(codes, act_scale, weight, w_scale, rows, gate, residual, bias=None,
                           out=None, gate_index=None, lora=None):
    """out = bf16(residual + bf16(gate * linear)), with ``lora`` (``LoraOperands``)
    linear -> bf16(linear + delta) first (the adapted gate-residual).

    ``gate`` is ``[N]`` (one row for every token), ``[T, N]`` with ``rows`` a
    multiple of T (row m uses gate row m % T: ``[rows, N]`` per row, ``[S, N]``
    broadcast over a batch), or with ``gate_index`` (int64 ``[T]``) any ``[R, N]``
    of which row m uses ``gate_index[m % T]`` (an adaLN table view gathered in
    place).  Any strides.
    """
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    if gate.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16:
        raise ValueError("gate and residual must be BF16")
    if gate.ndim == 1:
        if gate.shape != (n,) or gate_index is not None:
            raise ValueError("a broadcast gate must have the output width")
        gts, ghs, tokens, gate_rows = 0, gate.stride(0), 1, 1
    elif gate.ndim == 2 and gate.shape[1] == n:
        gts, ghs, gate_rows = gate.stride(0), gate.stride(1), gate.shape[0]
        if gate_index is not None:
            if gate_index.dtype != torch.int64 or gate_index.ndim != 1 or not gate_index.is_contiguous():
                raise ValueError("gate indices must be a contiguous int64 vector")
            tokens = gate_index.numel()
        else:
            tokens = gate.shape[0]
        if tokens < 1 or rows % tokens:
            raise ValueError("output rows must be a whole number of gated token blocks")
    else:
        raise ValueError("gate must be [N] or [T, N]")
    if residual.shape != (rows, n) or residual.stride(1) != 1:
        raise ValueError("residual must be [rows, N] with unit column stride")
    require_device(gate, residual, gate_index)
    if out is None:
        out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
    elif (out.dtype != torch.bfloat16 or out.shape != (rows, n) or out.stride(1) != 1
          or out.device != device):
        raise ValueError("out must be a BF16 [rows, N] matrix with unit column stride")
    if rows:
        t = ldt = b = ldb = None
        rank, scale, strength = 0, 1.0, 1.0
        if lora is not None:
            t, ldt, b, ldb = lora.operands(rows, n, device)
            rank, scale, strength = lora.rank, float(lora.scale), float(lora.strength)
        call("vflash_fp8_linear_lora_gate_residual", ptr(codes), ptr(act_scale), codes.stride(0),
             ptr(weight), ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(gate), gts,
             ghs, tokens, ptr(gate_index), gate_rows, ptr(residual), residual.stride(0), ptr(t),
             ldt or 0, ptr(b), ldb or 0, rank, scale, strength, ptr(out), out.stride(0),
             stream_of(device))
    return out


LORA_MAX_RANK = 128  # per adapter (branch) in the GEMM epilogues
LORA_DOWN_MAX_RANK = 512  # stacked adapters in one down-projection


def _round_up(v: int, q: int) -> int:
    return -(-v // q) * q


def _lora_a(x, lora_a):
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("LoRA input must be a 2-D BF16 matrix with unit column stride")
    if lora_a.dtype != torch.bfloat16 or lora_a.ndim != 2:
        raise ValueError("LoRA A must be a BF16 [rank, K] matrix")
    if lora_a.shape[1] != x.shape[1]:
        raise ValueError("LoRA A does not match the input width")
    if not 1 <= lora_a.shape[0] <= LORA_DOWN_MAX_RANK:
        raise ValueError(f"LoRA rank must be 1..{LORA_DOWN_MAX_RANK}")
    if not lora_a.is_contiguous() or lora_a.data_ptr() % 16:
        lora_a = lora_a.contiguous().clone()  # the kernel reads whole contiguous rows
    return lora_a


def lora_down(x, lora_a):
    """t = bf16(x . lora_a^T) for a BF16 activation matrix and a BF16 [rank, K]
    adapter.  Returns a [M, rank] view of a [M, ceil16(rank)] buffer whose extra
    columns are zero (the GEMM epilogues read whole 8-element groups)."""
    lora_a = _lora_a(x, lora_a)
    device = require_device(x, lora_a)
    m, k = x.shape
    rank = lora_a.shape[0]
    ldt = _round_up(rank, 16)
    t = torch.empty((m, ldt), device=device, dtype=torch.bfloat16)
    if m:
        call("vflash_lora_down", ptr(x), m, k, x.stride(0), ptr(lora_a), rank, ptr(t), ldt,
             stream_of(device))
    return t[:, :rank]


def quantize_lora_supported(k: int, rank: int) -> bool:
    """Shapes of the fused quantize + LoRA-down kernel (those of ``lora_down``)."""
    return k % 16 == 0 and k >= 16 and 1 <= rank <= LORA_DOWN_MAX_RANK


def quantize_rows_lora(x, lora_a, pad_to: int = 16):
    """Codes/scales of ``quantize_rows(x)`` and the ``t`` of ``lora_down(x, lora_a)``
    (both bit-identical) from one launch; see ``quantize_lora_supported`` for the shapes."""
    lora_a = _lora_a(x, lora_a)
    device = require_device(x, lora_a)
    m, k = x.shape
    rank = lora_a.shape[0]
    ldt = _round_up(rank, 16)
    m_pad = (m + pad_to - 1) // pad_to * pad_to
    codes = torch.empty((m_pad, k), device=device, dtype=E4M3)
    scales = torch.empty((m_pad, 1), device=device, dtype=torch.float32)
    t = torch.empty((m, ldt), device=device, dtype=torch.bfloat16)
    if m:
        call("vflash_quantize_rows_lora_e4m3", ptr(x), m, k, x.stride(0), ptr(codes), ptr(scales),
             m_pad, ptr(lora_a), rank, ptr(t), ldt, stream_of(device))
    return codes, scales, t[:, :rank]


def _rows_for_lora(matrix, rows, cols):
    """``matrix`` ([rows, >= cols] BF16) as the epilogues read it: unit column
    stride, a row stride that is a multiple of 8 and 16-byte alignment; a copy
    (zero-padded to a multiple of 8 columns) when it is not.  Returns
    (tensor, row stride)."""
    if matrix.dtype != torch.bfloat16 or matrix.ndim != 2 or matrix.shape[0] != rows:
        raise ValueError("LoRA operands must be BF16 matrices of the declared rows")
    if matrix.shape[1] < cols:
        raise ValueError("LoRA operands do not cover the rank")
    if matrix.stride(1) == 1 and matrix.stride(0) % 8 == 0 and matrix.data_ptr() % 16 == 0:
        # The epilogue reads each row up to cols rounded up to 8: those elements
        # must lie inside the tensor's storage (a view [:, :rank] of lora_down's
        # padded buffer does; a tensor ending at column `cols` of its last row may not).
        end = matrix.storage_offset() + (rows - 1) * matrix.stride(0) + _round_up(cols, 8)
        if rows == 0 or end * 2 <= matrix.untyped_storage().nbytes():
            return matrix, matrix.stride(0)
    padded = torch.zeros((rows, _round_up(cols, 8)), device=matrix.device, dtype=torch.bfloat16)
    padded[:, :cols] = matrix[:, :cols]
    return padded, padded.shape[1]


class LoraOperands:
    """One adapter's operands for a GEMM epilogue: t = bf16(x A^T) ``[rows, rank]``
    (as ``lora_down`` returns it), B ``[N, rank]``, the scale and the strength
    (h3_reference_lora.py:80-90: delta = bf16(t B^T), then bf16(delta * scale) if
    scale != 1 and bf16(delta * strength) if strength != 1)."""

    __slots__ = ("t", "b", "rank", "scale", "strength")

    def __init__(self, t, b, scale=1.0, strength=1.0):
        if t.ndim != 2 or b.ndim != 2 or t.shape[1] != b.shape[1]:
            raise ValueError("LoRA operands do not match the projection")
        self.t, self.b, self.rank = t, b, int(b.shape[1])
        if not 1 <= self.rank <= LORA_MAX_RANK:
            raise ValueError(f"LoRA rank must be 1..{LORA_MAX_RANK} per adapter")
        self.scale, self.strength = float(scale), float(strength)

    def operands(self, rows, n, device):
        if self.b.shape[0] != n or self.t.shape[0] != rows:
            raise ValueError("LoRA operands do not match the projection")
        if self.t.device != device or self.b.device != device:
            raise ValueError("all operands must share one device")
        t, ldt = _rows_for_lora(self.t, rows, self.rank)
        b, ldb = _rows_for_lora(self.b, n, self.rank)
        return t, ldt, b, ldb


def fp8_gemm_lora(codes, act_scale, weight, w_scale, rows, t, lora_b, *, scale=1.0,
                  strength=1.0, bias=None):
    """out = bf16(linear + delta) with delta = bf16(t . lora_b^T) [* scale] [* strength]."""
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    if t.dtype != torch.bfloat16 or lora_b.dtype != torch.bfloat16:
        raise ValueError("LoRA operands must be BF16")
    rank = lora_b.shape[1]
    if t.shape != (rows, rank) or lora_b.shape != (n, rank):
        raise ValueError("LoRA operands do not match the projection")
    lora = LoraOperands(t, lora_b, scale, strength)
    out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
    if rows:
        tt, ldt, bb, ldb = lora.operands(rows, n, device)
        call("vflash_fp8_linear_lora", ptr(codes), ptr(act_scale), codes.stride(0), ptr(weight),
             ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(tt), ldt, ptr(bb), ldb,
             rank, float(scale), float(strength), ptr(out), out.stride(0), stream_of(device))
    return out


def fp8_gemm_lora_branches(codes, act_scale, weight, w_scale, rows, t, t_branch, lora_b, rank,
                           scales, *, strength=1.0, bias=None, planes=0):
    """The LoRA linear with ``len(scales)`` (1..3) adapter branches over equal runs
    of output columns: column c of branch b = c // (N / branches) takes
    delta = bf16(t[:, b * t_branch : b * t_branch + rank] . lora_b[c]^T), then
    bf16(delta * scales[b]) and the strength step.  ``t`` is [rows, >= (branches-1)
    * t_branch + rank] with a row stride that is a multiple of 8; ``lora_b`` is
    [N, >= rank].  ``planes`` > 0 writes [planes, rows, N / planes] (as
    ``fp8_gemm_planes``), else [rows, N]."""
    device = _gemm_operands(codes, act_scale, weight, w_scale, rows, bias)
    n, k = weight.shape
    branches = len(scales)
    if not 1 <= branches <= 3 or n % branches or (branches > 1 and (n // branches) % 32):
        raise ValueError("adapter branches must split the output into runs of 32-column multiples")
    if not 1 <= rank <= LORA_MAX_RANK:
        raise ValueError(f"LoRA rank must be 1..{LORA_MAX_RANK} per adapter")
    if branches > 1 and (t_branch < rank or t_branch % 8):
        raise ValueError("t branches must be at least the rank wide, a multiple of 8")
    if t.device != device or lora_b.device != device:
        raise ValueError("all operands must share one device")
    tt, ldt = _rows_for_lora(t, rows, (branches - 1) * t_branch + rank if branches > 1 else rank)
    if tt is not t and branches > 1:
        raise ValueError("stacked adapter rows need a row stride that is a multiple of 8")
    bb, ldb = _rows_for_lora(lora_b, n, rank)
    if planes:
        if n % planes:
            raise ValueError("the merged width must split evenly into planes")
        cols = n // planes
        out = torch.empty((planes, rows, cols), device=device, dtype=torch.bfloat16)
        ldo, plane_cols, plane_stride = cols, cols, rows * cols
    else:
        out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
        ldo, plane_cols, plane_stride = n, 0, 0
    if rows:
        sc = (ctypes.c_float * branches)(*[float(v) for v in scales])
        call("vflash_fp8_linear_lora_branches", ptr(codes), ptr(act_scale), codes.stride(0),
             ptr(weight), ptr(w_scale), weight.stride(0), rows, n, k, ptr(bias), ptr(tt), ldt,
             t_branch if branches > 1 else 0, ptr(bb), ldb, rank, branches, sc, float(strength),
             ptr(out), ldo, plane_cols, plane_stride, stream_of(device))
    return out


def gemm_tiling(m: int, n: int, compute_units: int = 256, branch_cols: int = 0) -> str:
    """Name of the tiling the E4M3 GEMM entries use for an m x n output
    (``vflash_fp8_gemm_tiling``; a host-side query)."""
    index = _lib.library().vflash_fp8_gemm_tiling(m, n, compute_units, branch_cols)
    if index < 0:
        raise ValueError("no tiling for these arguments")
    return GEMM_TILINGS[index]


# The tilings in the order of vflash_fp8_gemm_tiling's result.
GEMM_TILINGS = ("256x256", "256x192", "256x128", "128x192", "128x128", "128x128 one round",
                "128x64", "64x64")


def nvfp4_gemm(codes, act_scale, packed, block_scales, alpha, rows, bias=None):
    """W4A8 NVFP4-weight GEMM: out[rows, N] bf16."""
    if codes.dtype != E4M3 or codes.ndim != 2 or codes.stride(1) != 1:
        raise ValueError("NVFP4 activation codes must be a 2-D float8_e4m3fn matrix")
    if packed.dtype != torch.uint8 or block_scales.dtype != torch.uint8:
        raise ValueError("NVFP4 weights and block scales must be uint8")
    if packed.ndim != 2 or not packed.is_contiguous():
        raise ValueError("NVFP4 packed weights must be a contiguous uint8 [N, K/2] matrix")
    n, half_k = packed.shape
    k = 2 * half_k
    if codes.shape[1] != k or codes.shape[0] < rows:
        raise ValueError("NVFP4 activation width differs from the weight")
    if block_scales.shape != (n, k // 16) or not block_scales.is_contiguous():
        raise ValueError("NVFP4 block scales must be a contiguous uint8 [N, K/16] matrix")
    if act_scale.dtype != torch.float32 or not act_scale.is_contiguous() or act_scale.numel() < rows:
        raise ValueError("NVFP4 activation scales must be contiguous fp32 covering the rows")
    if alpha.dtype != torch.float32 or alpha.numel() != 1:
        raise ValueError("NVFP4 alpha must be an fp32 scalar tensor")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (n,) or not bias.is_contiguous()):
        raise ValueError("NVFP4 bias must be a contiguous BF16 vector of the output width")
    if block_scales.data_ptr() % 16:
        block_scales = block_scales.clone()  # the kernel copies scale runs with 16-byte DMA
    device = require_device(codes, act_scale, packed, block_scales, alpha,
                            *([bias] if bias is not None else []))
    out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
    if rows:
        call("vflash_nvfp4_linear", ptr(codes), ptr(act_scale), codes.stride(0), ptr(packed),
             ptr(block_scales), ptr(alpha), rows, n, k, ptr(bias), ptr(out), out.stride(0),
             stream_of(device))
    return out


def nvfp4_quantize_rows(matrix, global_sf):
    """NVFP4 activation quantization (the W4A4 input).

    ``matrix`` is bf16 or f16 ``[M, K]`` (K % 64 == 0, unit column stride),
    ``global_sf`` an fp32 scalar tensor on the same device.  Returns packed E2M1
    codes ``[M, K/2]`` (uint8) and E4M3 block scales ``[ceil128(M), K/16]``
    (uint8, 128x4 order, padding rows 0).
    """
    if matrix.dtype not in (torch.bfloat16, torch.float16) or matrix.ndim != 2 or matrix.stride(1) != 1:
        raise ValueError("NVFP4 quantization requires a 2-D BF16/F16 matrix with unit column stride")
    if global_sf.dtype != torch.float32 or global_sf.numel() != 1:
        raise ValueError("the NVFP4 global scale must be an fp32 scalar tensor")
    m, k = matrix.shape
    if k % 64:
        raise ValueError("NVFP4 quantization needs K % 64 == 0")
    device = require_device(matrix, global_sf)
    m_pad = (m + 127) // 128 * 128
    codes = torch.empty((m, k // 2), device=device, dtype=torch.uint8)
    scales = torch.empty((m_pad, k // 16), device=device, dtype=torch.uint8)
    if m:
        call("vflash_nvfp4_quantize_rows", ptr(matrix), int(matrix.dtype == torch.float16), m, k,
             matrix.stride(0), ptr(global_sf), ptr(codes), codes.stride(0), ptr(scales), m_pad,
             stream_of(device))
    return codes, scales


def nvfp4_w4a4_gemm(codes, act_scales, packed, block_scales, alpha, rows, bias=None):
    """W4A4 NVFP4 GEMM: out[rows, N] = bf16(bf16(alpha * a . w^T) + bias)."""
    if codes.dtype != torch.uint8 or codes.ndim != 2 or codes.stride(1) != 1:
        raise ValueError("NVFP4 activation codes must be a 2-D uint8 matrix")
    if packed.dtype != torch.uint8 or block_scales.dtype != torch.uint8 or act_scales.dtype != torch.uint8:
        raise ValueError("NVFP4 codes and block scales must be uint8")
    if packed.ndim != 2 or not packed.is_contiguous():
        raise ValueError("NVFP4 packed weights must be a contiguous uint8 [N, K/2] matrix")
    n, half_k = packed.shape
    k = 2 * half_k
    if codes.shape != (rows, half_k):
        raise ValueError("NVFP4 activation width differs from the weight")
    if block_scales.shape != (n, k // 16) or not block_scales.is_contiguous():
        raise ValueError("NVFP4 block scales must be a contiguous uint8 [N, K/16] matrix")
    if block_scales.data_ptr() % 16:
        block_scales = block_scales.clone()  # the kernel copies scale runs with 16-byte DMA
    if act_scales.shape != ((rows + 127) // 128 * 128, k // 16) or not act_scales.is_contiguous():
        raise ValueError("NVFP4 activation scales must be the padded 128x4 layout")
    if alpha.dtype != torch.float32 or alpha.numel() != 1:
        raise ValueError("NVFP4 alpha must be an fp32 scalar tensor")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (n,) or not bias.is_contiguous()):
        raise ValueError("NVFP4 bias must be a contiguous BF16 vector of the output width")
    device = require_device(codes, act_scales, packed, block_scales, alpha,
                            *([bias] if bias is not None else []))
    out = torch.empty((rows, n), device=device, dtype=torch.bfloat16)
    if rows:
        call("vflash_nvfp4_w4a4_linear", ptr(codes), codes.stride(0), ptr(act_scales), ptr(packed),
             ptr(block_scales), ptr(alpha), rows, n, k, ptr(bias), ptr(out), out.stride(0),
             stream_of(device))
    return out
