"""Fused W8A8 compositions: merged QKV, the GELU-tanh FFN, and the LoRA linear.

Each runs on the HIP kernels of this package and keeps the rounding boundaries
of the reference's unfused sequence:

* merged QKV (src/vflash/adapters/h3_reference_execution.py:141-192): one
  linear over ``cat(Wq, Wk, Wv)`` and ``cat(scales)``; returns the three column
  chunks, either as views of one ``[.., 3*inner]`` output (the reference's
  ``.chunk(3, -1)``) or as three contiguous planes (the copy done by
  src/vflash/native/h3_tiled_block.py:45-60), written directly by the epilogue;
* FFN: up-projection + bias + GELU-tanh in the GEMM epilogue, which also emits
  per-row |g| maxima; per-token E4M3 requantization of ``g`` (the down
  projection's own activation quantization); down-projection + bias + adaLN
  gate + residual in the epilogue (h3_fused_ops.py:124-170 rounding);
* LoRA (src/vflash/adapters/h3_reference_lora.py:75-90): ``t = bf16(x A^T)``,
  then the base linear with ``bf16(t B^T)`` merged in its epilogue;
* the native block's low-rank residuals (``LowRankResidual``, the reference's
  H3LowRankResidualWeights, src/vflash/native/h3_native_denoiser.py:50-54)
  merged in the epilogues of the projections they adapt: the three Q/K/V
  branches with their own scalings in the merged QKV projection
  (h3_native_denoiser.py:301-316), the attention-output and FFN-down adapters
  before the gate-residual (``_adapted_gate_residual``, :327-338), and the FFN
  input adapter before the activation (``_ffn_input``, :375-382).

Each also accepts, as ``value``, the ``QuantizedRows`` of a fused producer
(vflash_amd.producers), whose codes and scales take the place of its own
activation quantization.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from vflash_amd import kernels
from vflash_amd.fp8_linear import RowFP8Execution, _quantize_activation_torch, w8a8_supported
from vflash_amd.producers import QuantizedRows


def _quantize(execution: RowFP8Execution, matrix):
    if execution.activation_quantizer == "torch":
        return _quantize_activation_torch(matrix)
    with execution.measure("linear.activation_quantize"):
        return kernels.quantize_rows(matrix)


def _activation(execution: RowFP8Execution, value):
    """(codes, scales, rows) of a bf16 ``[.., K]`` activation, or of the rows a
    fused producer already quantized (``QuantizedRows``)."""
    if isinstance(value, QuantizedRows):
        return value.codes, value.scales, value.rows
    matrix = value.reshape(-1, value.shape[-1])
    codes, act_scale = _quantize(execution, matrix)
    return codes, act_scale, matrix.shape[0]


def _check_w8a8(execution: RowFP8Execution, value, weight, scale, bias=None):
    if execution.mode != "w8a8":
        raise ValueError("fused FP8 compositions require a w8a8 execution")
    if (
        weight.ndim != 2
        or value.ndim < 1
        or value.shape[-1] != weight.shape[1]
        or weight.dtype != torch.float8_e4m3fn
        or scale.dtype != torch.float32
        or scale.shape != (weight.shape[0], 1)
        or weight.device != value.device
        or scale.device != value.device
    ):
        raise ValueError("FP8 codes/scales differ from the declared layout")
    if bias is not None and (
        bias.shape != (weight.shape[0],) or bias.device != value.device or bias.dtype != value.dtype
    ):
        raise ValueError("FP8 bias differs from the declared output")
    if not w8a8_supported(value):
        raise ValueError("W8A8 requires gfx950 (MI355X) BF16 inputs")


@dataclass(frozen=True)
class LowRankResidual:
    """A low-rank residual adapter of one projection: ``down`` bf16 ``[rank, K]``,
    ``up`` bf16 ``[N, rank]``, ``scaling`` a float (the reference's
    H3LowRankResidualWeights, h3_native_denoiser.py:50-54).  Its contribution is
    ``bf16(bf16(bf16(x down^T) up^T) * scaling)``, added to the projection with
    one bf16 rounding (``_residual_linear``, h3_native_denoiser.py:280-299)."""

    down: torch.Tensor
    up: torch.Tensor
    scaling: float


def _check_residual(residual, k: int, n: int):
    if not isinstance(residual, LowRankResidual):
        raise ValueError("adapters must be LowRankResidual weights")
    down, up = residual.down, residual.up
    if down.ndim != 2 or up.ndim != 2 or down.shape[0] < 1 or up.shape[1] != down.shape[0]:
        raise ValueError("Adapter projection requires compatible nonempty A/B matrices")
    if down.shape[1] != k or up.shape[0] != n:
        raise ValueError("Adapter projection does not match the target model")
    if down.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("the fused adapter epilogues take BF16 adapters")
    if not math.isfinite(residual.scaling) or isinstance(residual.scaling, bool):
        raise ValueError("Adapter scale must be finite")
    if down.shape[0] > kernels.LORA_MAX_RANK:
        raise ValueError(f"the fused adapter epilogues take ranks up to {kernels.LORA_MAX_RANK}")


@dataclass(frozen=True)
class StackedAdapters:
    """The Q/K/V adapters of a merged projection laid out for one down-projection
    and one epilogue: ``down`` ``[B * R, K]`` (branch b's rows at b * R, zero rows
    up to R), ``up`` ``[N, rank]`` (each branch's rows in column order, zero
    columns up to ``rank``), ``rank`` the largest branch rank, ``width`` R =
    ceil16(rank) and one scaling per branch."""

    down: torch.Tensor
    up: torch.Tensor
    rank: int
    width: int
    scalings: tuple


def stack_adapters(residuals, k: int, n: int) -> StackedAdapters:
    """Stack 1..3 ``LowRankResidual`` branches (equal output widths n / branches)
    for ``qkv_linear``; build it once per set of weights and pass it in place of
    the tuple to skip the per-call copy."""
    residuals = tuple(residuals)
    branches = len(residuals)
    if not 1 <= branches <= 3 or n % branches:
        raise ValueError("H3 QKV residual pack must contain three branches")
    width_n = n // branches
    for r in residuals:
        _check_residual(r, k, width_n)
    rank = max(r.down.shape[0] for r in residuals)
    width = -(-rank // 16) * 16
    device = residuals[0].down.device
    down = torch.zeros((branches * width, k), device=device, dtype=torch.bfloat16)
    # Rows of B padded to a multiple of 8 columns, as the epilogue reads them.
    up = torch.zeros((n, -(-rank // 8) * 8), device=device, dtype=torch.bfloat16)
    for b, r in enumerate(residuals):
        down[b * width : b * width + r.down.shape[0]] = r.down
        up[b * width_n : (b + 1) * width_n, : r.up.shape[1]] = r.up
    return StackedAdapters(down, up[:, :rank], rank, width,
                           tuple(float(r.scaling) for r in residuals))


def _adapter_t(execution, value, down):
    """t = bf16(x down^T) of the activation (bf16 rows, or the bf16 values a fused
    producer kept), and the rows' codes and scales; one launch when the HIP
    quantizer and the fused quantize + down-projection kernel apply."""
    if isinstance(value, QuantizedRows):
        if value.values is None:
            raise ValueError("an adapter on pre-quantized rows needs the producer's bf16 values")
        matrix = value.values.reshape(-1, value.values.shape[-1])
        return value.codes, value.scales, value.rows, kernels.lora_down(matrix, down)
    matrix = value.reshape(-1, value.shape[-1])
    if matrix.stride(1) != 1 or matrix.stride(0) % 8:
        matrix = matrix.contiguous()
    if (execution.activation_quantizer != "torch"
            and kernels.quantize_lora_supported(matrix.shape[1], down.shape[0])):
        with execution.measure("linear.activation_quantize"):
            codes, act_scale, t = kernels.quantize_rows_lora(matrix, down)
        return codes, act_scale, matrix.shape[0], t
    codes, act_scale = _quantize(execution, matrix)
    return codes, act_scale, matrix.shape[0], kernels.lora_down(matrix, down)


def merge_qkv(weights, scales):
    """Concatenate per-projection codes [inner, hidden] and row scales [inner, 1]."""
    if len(weights) != 3 or len(scales) != 3:
        raise ValueError("merged QKV needs exactly three projections")
    if any(w.shape != weights[0].shape or w.dtype != torch.float8_e4m3fn for w in weights):
        raise ValueError("QKV fusion requires matching cached row-FP8 projections")
    return torch.cat([w.detach() for w in weights]), torch.cat(list(scales))


def qkv_linear(execution: RowFP8Execution, value, weight, scale, bias=None, *, planes=False,
               residuals=()):
    """One W8A8 linear over the merged [3*inner, hidden] matrix.

    ``planes=False`` returns ``.chunk(3, -1)`` views of one output, exactly as
    the reference; ``planes=True`` returns three contiguous ``[.., inner]``
    tensors (views into one [3, rows, inner] buffer) written by the epilogue.
    ``residuals``: the Q/K/V pack of three ``LowRankResidual`` (or their
    ``stack_adapters``), each merged into its third of the output with its own
    scaling, ``chunk_b + bf16(bf16(t_b up_b^T) * scaling_b)`` rounded once
    (h3_native_denoiser.py:301-316; the fused merges of h3_fused_ops.py:802-838,
    954-980 keep the same roundings).
    """
    _check_w8a8(execution, value, weight, scale, bias)
    if weight.shape[0] % 3:
        raise ValueError("a merged QKV matrix has 3 * inner rows")
    stacked = None
    if isinstance(residuals, StackedAdapters):
        stacked = residuals
    elif residuals:
        if len(residuals) != 3:
            raise ValueError("H3 QKV residual pack must contain three branches")
        stacked = stack_adapters(residuals, weight.shape[1], weight.shape[0])
    if stacked is not None and (
        len(stacked.scalings) != 3 or stacked.up.shape[0] != weight.shape[0]
        or stacked.down.shape[1] != weight.shape[1]
    ):
        raise ValueError("H3 QKV residual pack must contain three branches")
    if execution.observer is not None and sum(execution.calls.values()) % 200 == 0:
        execution.observer()
    execution.calls["w8a8"] += 1
    shape = value.shape
    inner = weight.shape[0] // 3
    if stacked is not None:
        codes, act_scale, rows, t = _adapter_t(execution, value, stacked.down)
        with execution.measure("linear.fp8_gemm"):
            out = kernels.fp8_gemm_lora_branches(
                codes, act_scale, weight, scale, rows, t, stacked.width, stacked.up, stacked.rank,
                stacked.scalings, bias=bias, planes=3 if planes else 0,
            )
        if planes:
            return tuple(out[i].view(*shape[:-1], inner) for i in range(3))
        return out.reshape(*shape[:-1], 3 * inner).chunk(3, dim=-1)
    codes, act_scale, rows = _activation(execution, value)
    with execution.measure("linear.fp8_gemm"):
        if planes:
            out = kernels.fp8_gemm_planes(codes, act_scale, weight, scale, rows, 3, bias)
            return tuple(out[i].view(*shape[:-1], inner) for i in range(3))
        out = kernels.fp8_gemm(codes, act_scale, weight, scale, rows, bias)
    return out.reshape(*shape[:-1], 3 * inner).chunk(3, dim=-1)


class FusedQKV(torch.nn.Module):
    """Merged Q/K/V projection built from three row-FP8 projections without bias.

    Mirrors the construction checks of h3_reference_execution.py:141-160: the
    three parts must share shape, dtype and execution, and carry no bias.
    """

    def __init__(self, to_q, to_k, to_v, *, planes=False, residuals=()):
        super().__init__()
        parts = [to_q, to_k, to_v]
        if not all(
            hasattr(p, "execution")
            and hasattr(p, "row_scale")
            and p.bias is None
            and p.weight.shape == parts[0].weight.shape
            and p.execution is parts[0].execution
            for p in parts
        ):
            raise ValueError("QKV fusion requires matching cached row-FP8 projections")
        weight, scale = merge_qkv([p.weight for p in parts], [p.row_scale for p in parts])
        self.weight = torch.nn.Parameter(weight, requires_grad=False)
        self.register_buffer("row_scale", scale)
        self.execution = parts[0].execution
        self.planes = planes
        # The Q/K/V adapter pack, stacked once for the merged epilogue.
        self.adapters = (
            stack_adapters(residuals, weight.shape[1], weight.shape[0]) if residuals else None
        )

    def forward(self, value):
        return qkv_linear(self.execution, value, self.weight, self.row_scale, planes=self.planes,
                          residuals=self.adapters or ())


def _lora(execution, rows_bf16, residual, n):
    """LoraOperands of a ``LowRankResidual`` on bf16 rows [M, K] (t computed here)."""
    _check_residual(residual, rows_bf16.shape[1], n)
    t = kernels.lora_down(rows_bf16, residual.down)
    return kernels.LoraOperands(t, residual.up, residual.scaling)


def fp8_ffn(
    execution: RowFP8Execution,
    value,
    up_weight,
    up_scale,
    up_bias,
    down_weight,
    down_scale,
    down_bias,
    gate,
    residual,
    *,
    activation: str = "gelu_tanh",
    gate_index=None,
    up_residual=None,
    down_residual=None,
):
    """residual + gate * down(requant(act(up(value)))) with reference rounding.

    ``value`` and ``residual`` are ``[.., hidden]``; ``gate`` is ``[hidden]``
    (broadcast over tokens), ``[T, hidden]`` with the rows a multiple of T (row
    m uses gate row m % T), or, with ``gate_index`` (int64 ``[T]``, the
    reference's ``adaln_indices``), the ungathered adaLN rows ``table[:, j, :]``
    of which row m uses ``gate_index[m % T]`` (h3_native_denoiser.py:556-576
    without the ``index_select`` copy).  Any strides.
    ``activation`` is ``"gelu_tanh"`` (up projection ``[F, hidden]``) or
    ``"swiglu"``, the H3 feed-forward (h3_native_denoiser.py:369-382, 563-576):
    the up projection is the packed ``[2F, hidden]`` value/gate matrix and the
    activation is ``value * silu(gate)`` with the eager bf16 rounding of
    h3_fused_ops.py:184-224.
    ``up_residual`` / ``down_residual`` (``LowRankResidual``): the block's FFN
    adapters, merged into the up projection before the activation (``_ffn_input``,
    h3_native_denoiser.py:375-382; h3_fused_ops.py:229-286) and into the down
    projection before the gate-residual (``_adapted_gate_residual``,
    h3_native_denoiser.py:327-338, 570; h3_fused_ops.py:341-418).  The down
    adapter reads the bf16 activation, so that path keeps it.
    """
    if activation not in ("gelu_tanh", "swiglu"):
        raise ValueError("unknown FFN activation")
    _check_w8a8(execution, value, up_weight, up_scale, up_bias)
    hidden = up_weight.shape[1]
    inner = up_weight.shape[0] // (2 if activation == "swiglu" else 1)
    if activation == "swiglu" and up_weight.shape[0] % 256:
        raise ValueError("SwiGLU projections need 2F rows with F a multiple of 128")
    if down_weight.shape[1] != inner or down_weight.shape[0] != hidden:
        raise ValueError("FFN up/down projections do not chain")
    if up_residual is not None:
        _check_residual(up_residual, hidden, up_weight.shape[0])
    if down_residual is not None:
        _check_residual(down_residual, inner, hidden)
    shape = value.shape
    rows = shape.numel() // hidden
    res = residual.reshape(-1, down_weight.shape[0])
    if res.shape[0] != rows:
        raise ValueError("residual rows differ from the FFN input rows")
    if execution.observer is not None and sum(execution.calls.values()) % 200 == 0:
        execution.observer()
    execution.calls["w8a8"] += 2
    up_lora = None
    if up_residual is not None:
        codes, act_scale, rows, t = _adapter_t(execution, value, up_residual.down)
        up_lora = kernels.LoraOperands(t, up_residual.up, up_residual.scaling)
    else:
        codes, act_scale, rows = _activation(execution, value)
    g = None
    if activation == "swiglu":
        # value * silu(gate) in the up projection's epilogue, with row maxima.
        with execution.measure("linear.fp8_gemm"):
            g, amax = kernels.fp8_gemm_swiglu(codes, act_scale, up_weight, up_scale, rows, up_bias,
                                              lora=up_lora)
        with execution.measure("linear.activation_quantize"):
            h_codes, h_scale = kernels.requant_rows(g, amax)
    else:
        # The up projection, then GELU-tanh fused with the down linear's quantization.
        with execution.measure("linear.fp8_gemm"):
            if up_lora is None:
                y = kernels.fp8_gemm(codes, act_scale, up_weight, up_scale, rows, up_bias)
            else:
                y = kernels.fp8_gemm_lora(codes, act_scale, up_weight, up_scale, rows, up_lora.t,
                                          up_lora.b, scale=up_lora.scale, bias=up_bias)
        with execution.measure("linear.activation_quantize"):
            h_codes, h_scale, g = kernels.gelu_quantize_rows(
                y, keep_values=down_residual is not None)
    down_lora = None if down_residual is None else _lora(execution, g, down_residual, hidden)
    with execution.measure("linear.fp8_gemm"):
        out = kernels.fp8_gemm_gate_residual(
            h_codes, h_scale, down_weight, down_scale, rows, gate, res, down_bias,
            gate_index=gate_index, lora=down_lora,
        )
    return out.reshape(shape)


def gate_residual_linear(execution: RowFP8Execution, value, weight, scale, bias, gate, residual,
                         *, gate_index=None, adapter=None):
    """``residual + gate * linear(value)`` with the reference's strict bf16 rounding,
    and with ``adapter`` (``LowRankResidual``) the adapted form
    ``bf16(residual + bf16(gate * bf16(linear + bf16(bf16(t up^T) * scaling))))``:
    the attention-output projection of the native block (``_adapted_gate_residual``,
    h3_native_denoiser.py:327-338, 551; h3_fused_ops.py:124-170, 341-418), one GEMM
    launch.  ``gate`` and ``gate_index`` as in ``fp8_ffn``."""
    _check_w8a8(execution, value, weight, scale, bias)
    n, k = weight.shape
    shape = value.shape
    res = residual.reshape(-1, n)
    if res.shape[0] * k != shape.numel():
        raise ValueError("residual rows differ from the projection's input rows")
    if adapter is not None:
        _check_residual(adapter, k, n)
    if execution.observer is not None and sum(execution.calls.values()) % 200 == 0:
        execution.observer()
    execution.calls["w8a8"] += 1
    lora = None
    if adapter is not None:
        codes, act_scale, rows, t = _adapter_t(execution, value, adapter.down)
        lora = kernels.LoraOperands(t, adapter.up, adapter.scaling)
    else:
        codes, act_scale, rows = _activation(execution, value)
    with execution.measure("linear.fp8_gemm"):
        out = kernels.fp8_gemm_gate_residual(codes, act_scale, weight, scale, rows, gate, res, bias,
                                             gate_index=gate_index, lora=lora)
    return out.reshape(*shape[:-1], n)


class FP8FeedForward(torch.nn.Module):
    """FFN block of two row-FP8 projections with a GELU-tanh or SwiGLU activation."""

    def __init__(self, up, down, activation: str = "gelu_tanh"):
        super().__init__()
        if up.execution is not down.execution:
            raise ValueError("FFN projections must share one execution")
        if activation not in ("gelu_tanh", "swiglu"):
            raise ValueError("unknown FFN activation")
        self.up, self.down, self.execution = up, down, up.execution
        self.activation = activation

    def forward(self, value, gate, residual, gate_index=None, up_residual=None,
                down_residual=None):
        return fp8_ffn(
            self.execution,
            value,
            self.up.weight,
            self.up.row_scale,
            self.up.bias,
            self.down.weight,
            self.down.row_scale,
            self.down.bias,
            gate,
            residual,
            activation=self.activation,
            gate_index=gate_index,
            up_residual=up_residual,
            down_residual=down_residual,
        )


def fp8_linear_lora(
    execution: RowFP8Execution,
    value,
    weight,
    scale,
    bias,
    lora_a,
    lora_b,
    *,
    scaling: float = 1.0,
    strength: float = 1.0,
):
    """W8A8 linear plus an activation-space LoRA delta merged in the epilogue.

    Same result as the reference hook applied to ``execution.linear``:
    ``result + bf16(bf16(bf16(x A^T) B^T) [* scaling] [* strength])``;
    strength 0 skips the adapter (h3_reference_lora.py:75-78).
    """
    _check_w8a8(execution, value, weight, scale, bias)
    if strength == 0.0:
        return execution.linear(value, weight, scale, bias)
    if lora_a.ndim != 2 or lora_b.ndim != 2 or lora_a.shape[1] != weight.shape[1]:
        raise ValueError("Adapter projection does not match the target model")
    if lora_b.shape != (weight.shape[0], lora_a.shape[0]):
        raise ValueError("Adapter projection does not match the target model")
    # Refused before any counter moves or kernel runs.
    if lora_a.dtype != torch.bfloat16 or lora_b.dtype != torch.bfloat16:
        raise ValueError("the fused adapter epilogue takes BF16 adapters")
    if not 1 <= lora_a.shape[0] <= kernels.LORA_MAX_RANK:
        raise ValueError(f"the fused adapter epilogue takes ranks 1..{kernels.LORA_MAX_RANK}")
    if execution.observer is not None and sum(execution.calls.values()) % 200 == 0:
        execution.observer()
    execution.calls["w8a8"] += 1
    shape = value.shape
    if isinstance(value, QuantizedRows):
        # The producer quantized the rows; the adapter reads the bf16 rows it kept.
        if value.values is None:
            raise ValueError("an adapter on pre-quantized rows needs the producer's bf16 values")
        t = kernels.lora_down(value.values.reshape(-1, shape[-1]), lora_a)
        with execution.measure("linear.fp8_gemm"):
            out = kernels.fp8_gemm_lora(
                value.codes, value.scales, weight, scale, value.rows, t, lora_b, scale=scaling,
                strength=strength, bias=bias,
            )
        return out.reshape(*shape[:-1], weight.shape[0])
    matrix = value.reshape(-1, shape[-1])
    rows = matrix.shape[0]
    if matrix.stride(1) != 1 or matrix.stride(0) % 8:
        matrix = matrix.contiguous()
    fused_pass = (
        execution.activation_quantizer != "torch"
        and kernels.quantize_lora_supported(matrix.shape[1], lora_a.shape[0])
        and matrix.stride(0) % 8 == 0
        and lora_a.is_contiguous()
    )
    if fused_pass:
        # One pass over the rows: activation codes/scales and t = bf16(x A^T).
        with execution.measure("linear.activation_quantize"):
            codes, act_scale, t = kernels.quantize_rows_lora(matrix, lora_a)
    else:
        codes, act_scale = _quantize(execution, matrix)
        t = kernels.lora_down(matrix, lora_a)
    with execution.measure("linear.fp8_gemm"):
        out = kernels.fp8_gemm_lora(
            codes, act_scale, weight, scale, rows, t, lora_b, scale=scaling, strength=strength,
            bias=bias,
        )
    return out.reshape(*shape[:-1], weight.shape[0])
