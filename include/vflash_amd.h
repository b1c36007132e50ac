/*
 * vflash_amd: C-ABI of the MI355X (gfx950) quantized-linear path.
 *
 * Every entry point enqueues work on the given HIP stream (`stream` is a
 * hipStream_t; NULL is the legacy default stream) and returns immediately.
 * None allocates memory, synchronizes, or keeps a pointer after it returns.
 * All pointers are device pointers owned by the caller.  Element types:
 *   e4m3  : OCP FP8 E4M3 ("fn": no infinities, max 448), one byte per value
 *   bf16  : bfloat16, two bytes
 *   fp32  : IEEE binary32
 * Strides (ld*) are in elements of the pointed-to type.
 *
 * Return value: VFLASH_OK, or a negative status; no work was enqueued when a
 * negative status is returned.  vflash_status_string() names a status.
 */
#ifndef VFLASH_AMD_H
#define VFLASH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VFLASH_OK 0
#define VFLASH_EINVAL (-1)  /* an argument is outside the declared contract */
#define VFLASH_ELAUNCH (-2) /* the HIP runtime refused the launch */
#define VFLASH_ESCRATCH (-3) /* the call needs more than the allocation-free entry's scratch */

/* Bytes of the static device scratch of vflash_fp8_linear_swiglu_quantize_noalloc. */
#define VFLASH_NOALLOC_SCRATCH_BYTES (16 << 20)

/* Version of this interface; bumped when a signature changes. */
int vflash_abi_version(void);

/* Static string for a status code. */
const char* vflash_status_string(int status);

/*
 * Per-token E4M3 activation quantization.
 * Replaces quantize_activation / _rows_fp8
 *   (src/vflash/native/h3_fp8_activation.py:12-55) and its portable twin
 *   _quantize_activation_torch (src/vflash/native/h3_fp8_linear.py:18-31).
 *   x      bf16 [m, k], row stride ldx (>= k), unit column stride
 *   codes  e4m3 [m_pad, k] contiguous;  scales fp32 [m_pad]
 *   scale[r] = amax_r > 0 ? max(amax_r / 448, FLT_MIN) : 1
 *   code     = e4m3_rne(clamp(x / scale[r], -448, 448))
 *   Rows m..m_pad-1 are padding: codes 0, scale 1.  Requires 1 <= k, m <= m_pad.
 */
int vflash_quantize_rows_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx, void* codes,
                              float* scales, int64_t m_pad, void* stream);

/*
 * W8A8 linear with per-token and per-output-channel scales and bias.
 * Replaces the w8a8 branch of RowFP8Execution.linear
 *   (src/vflash/native/h3_fp8_linear.py:98-121): torch._scaled_mm(codes,
 *   weight.t(), scale_a, scale_b, out_dtype=bf16) then "+ bias".
 *   a   e4m3 [m, k] row stride lda;  sa fp32 [m]
 *   w   e4m3 [n, k] row stride ldw;  sw fp32 [n]
 *   bias bf16 [n] or NULL;  out bf16 [m, n] row stride ldo
 *   out = bf16(bf16(sum_k a*w * sa[m] * sw[n]) + bias[n])   (binary32 accumulation)
 *   Requires k % 16 == 0, n % 16 == 0, lda/ldw % 16 == 0, ldo % 4 == 0 (elements),
 *   a, w 16-byte aligned; bias, out 8-byte aligned.
 */
int vflash_fp8_linear(const void* a, const float* sa, int64_t lda, const void* w,
                      const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                      const void* bias, void* out, int64_t ldo, void* stream);

/*
 * Merged QKV projection into separate planes.
 * Replaces the fused to_q/to_k/to_v forward of dense_reference_execution
 *   (src/vflash/adapters/h3_reference_execution.py:141-192: one linear over
 *   cat(Wq, Wk, Wv) then .chunk(3, -1)) and the plane copy of tiled_forward
 *   (src/vflash/native/h3_tiled_block.py:45-60).
 *   Arithmetic is vflash_fp8_linear's; output column c is written to
 *   out[(c / plane_cols) * plane_stride + row * ldo + c % plane_cols].
 *   Requires plane_cols % 16 == 0 and n % plane_cols == 0.
 */
int vflash_fp8_linear_planes(const void* a, const float* sa, int64_t lda, const void* w,
                             const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                             const void* bias, void* out, int64_t ldo, int64_t plane_cols,
                             int64_t plane_stride, void* stream);

/*
 * GELU-tanh of the FFN hidden rows fused with the down linear's per-token E4M3
 * quantization: the step between the GELU FFN's two linears.
 * Replaces the FFN activation (the GELU-tanh form of
 *   src/vflash/native/h3_native_denoiser.py:369-382, whose reference
 *   activation is SiLU-mul) and the down linear's quantize_activation
 *   (src/vflash/native/h3_fp8_activation.py:12-55).
 *   y      bf16 [m, k] (ldy): the up linear's output (vflash_fp8_linear)
 *   g      = bf16(gelu_tanh(y)), the real function 0.5 y (1 + tanh(u)),
 *            u = beta (y + kappa y^3) with beta, kappa the binary32 constants of
 *            sqrt(2/pi) and 0.044715, rounded to binary32 and then to bf16 (a
 *            table of all 65536 bf16 inputs); written to g [m, k] (ldg) when g is
 *            not NULL.  +inf gives +inf, -inf NaN, a NaN input stays NaN.
 *   codes  e4m3 [m_pad, k] contiguous;  scales fp32 [m_pad]: the arithmetic of
 *          vflash_quantize_rows_e4m3 applied to g.  Rows m..m_pad-1: codes 0, scale 1.
 *   Requires k % 8 == 0, k <= 16384, ldy and ldg multiples of 8, y and g 16-byte
 *   aligned, codes 8-byte aligned.
 */
int vflash_gelu_quantize_rows_e4m3(const void* y, int64_t m, int64_t k, int64_t ldy, void* g,
                                   int64_t ldg, void* codes, float* scales, int64_t m_pad,
                                   void* stream);

/*
 * FFN input projection with the SwiGLU epilogue (the H3 feed-forward input).
 * Replaces RowFP8Execution.linear on the packed projection followed by
 * value * silu(gate) (src/vflash/native/h3_native_denoiser.py:369-376) or its
 * fused form triton_strict_bf16_silu_mul (src/vflash/native/h3_fused_ops.py:184-224,
 * 660-700).  w holds n = 2F rows: rows [0, F) give the value columns and rows
 * [F, 2F) the gate columns of the packed output, as .chunk(2, dim=-1) splits it.
 *   p   = bf16(bf16(acc * sa * sw) + bias)            (the packed [m, 2F] output)
 *   h   = bf16(p[:, f] * bf16(silu(p[:, F + f])))     written to h [m, F] (ldh), with
 *         silu(x) = x / (1 + exp(-x)) in binary32 with each step correctly
 *         rounded (the exponential, the sum and the quotient), then rounded to bf16
 *   amax_part fp32 [m, vflash_swiglu_parts(n)]: max |h| of each row over each
 *   128-column group, consumed by vflash_requant_rows_e4m3.
 *   Requires n % 256 == 0, ldh % 8 == 0, h and sw (and bias) 16-byte aligned.
 */
int vflash_fp8_linear_swiglu(const void* a, const float* sa, int64_t lda, const void* w,
                             const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                             const void* bias, void* h, int64_t ldh, float* amax_part,
                             void* stream);

/*
 * vflash_fp8_linear_swiglu with the FFN input adapter merged into the packed
 * projection before the activation (t, lora_b NULL: no adapter, the plain entry).
 * Replaces triton_strict_bf16_ffn_adapter_silu and its eager twin
 *   (src/vflash/native/h3_fused_ops.py:229-286, 703-763;
 *   src/vflash/native/h3_native_denoiser.py:318-325, 375-382, 1081-1101):
 *   p'  = bf16(p + delta) for value and gate columns alike, with
 *         delta = bf16(t . B^T), then bf16(delta * scale) if scale != 1 and
 *         bf16(delta * strength) if strength != 1 (the adapter chain of
 *         vflash_fp8_linear_lora)
 *   h   = bf16(p'[:, f] * bf16(silu(p'[:, F + f]))), amax_part as in
 *         vflash_fp8_linear_swiglu.
 *   t bf16 [m, >= rank] (ldt);  lora_b bf16 [n, >= rank] (ldb): value rows, then
 *   gate rows, of the adapter's up-projection;  1 <= rank <= 128; ldt, ldb
 *   multiples of 8; t, lora_b 16-byte aligned.
 */
int vflash_fp8_linear_swiglu_lora(const void* a, const float* sa, int64_t lda, const void* w,
                                  const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                                  const void* bias, const void* t, int64_t ldt,
                                  const void* lora_b, int64_t ldb, int64_t rank, float scale,
                                  float strength, void* h, int64_t ldh, float* amax_part,
                                  void* stream);

/* Number of 128-column groups per row in the SwiGLU amax_part: ceil(n / 2 / 128). */
int64_t vflash_swiglu_parts(int64_t n);

/*
 * The tiling vflash_fp8_linear and the other E4M3 GEMM entries use for an
 * m x n output on a device with `compute_units` CUs (a host-side query; no
 * device work).  0: 256x256, 1: 256x192, 2: 256x128, 3: 128x192, 4: 128x128
 * (two workgroups per CU), 5: 128x128 (one per CU, grids of one round),
 * 6: 128x64, 7: 64x64.  The SwiGLU entries always use 256x256.  No tiling
 * changes a result bit; this exists so that tests can aim shapes at each one.
 * branch_cols > 0 (a multiple of 32): the choice of a LoRA entry with adapter
 * branches that wide, which takes only tilings whose wave width (half the tile
 * width) divides branch_cols.
 */
int vflash_fp8_gemm_tiling(int64_t m, int64_t n, int64_t compute_units, int64_t branch_cols);

/*
 * vflash_fp8_linear_swiglu followed by vflash_requant_rows_e4m3 in one call
 * that allocates nothing.  It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid allocation).  The per-row partial maxima that
 * vflash_fp8_linear_swiglu returns in amax_part stay in a static device array
 * of VFLASH_NOALLOC_SCRATCH_BYTES (16 MiB) that each GPU the library runs on
 * holds until the process ends; the caller passes only inputs and outputs.
 *   h       bf16 [m, n/2] (ldh): h of vflash_fp8_linear_swiglu
 *   codes   e4m3 [m_pad, n/2] contiguous, scales fp32 [m_pad]: the requantized h
 *           (vflash_requant_rows_e4m3 on h), rows m..m_pad-1 codes 0, scale 1
 *   Requires the contracts of both entries and m * vflash_swiglu_parts(n) <=
 *   VFLASH_NOALLOC_SCRATCH_BYTES / 4; larger calls return VFLASH_ESCRATCH before
 *   any launch.  Calls that overlap on one GPU share the array and race; a
 *   caller serializes them (one stream per GPU, or its own ordering).
 */
int vflash_fp8_linear_swiglu_quantize_noalloc(const void* a, const float* sa, int64_t lda,
                                              const void* w, const float* sw, int64_t ldw,
                                              int64_t m, int64_t n, int64_t k, const void* bias,
                                              void* h, int64_t ldh, void* codes, float* scales,
                                              int64_t m_pad, void* stream);

/*
 * RMSNorm + adaLN modulation fused with the consuming linear's per-token E4M3
 * quantization: the producer of the QKV and FFN-input activations.
 * Replaces _rms_norm + _modulate (src/vflash/native/h3_native_denoiser.py:231-243,
 *   363-364, called at :535-540 and :565-566) or its fused form
 *   triton_strict_bf16_modulate (src/vflash/native/h3_fused_ops.py:52-122, 575-611),
 *   followed by the activation quantization of the next linear
 *   (src/vflash/native/h3_fp8_activation.py:12-55).
 *   x       bf16 [m, k] (ldx)
 *   norm_w  bf16 [k], or NULL (an RMSNorm without weight)
 *   rstd    = 1 / sqrt(sum_k x^2 / k + eps)                       (binary32)
 *   y       = bf16(bf16(bf16(x * rstd * norm_w) * bf16(1 + scale)) + shift)
 *   Modulation rows: x's row r uses t = r % tokens, or index[t] when index is
 *   not NULL (int64 [tokens], each < mod_rows; the in-place form of the gather
 *   table[:, j, :].index_select(0, adaln_indices), h3_native_denoiser.py:527-532).
 *   Row i of scale is scale + i * ld_scale elements, likewise shift.  A row whose
 *   index is outside [0, mod_rows) gets codes 0 and scale NaN.
 *   values  optional bf16 [m, k] (ldv) copy of y, for a consumer that needs it.
 *   codes   e4m3 [m_pad, k] contiguous;  scales fp32 [m_pad]: the arithmetic of
 *   vflash_quantize_rows_e4m3 applied to y.  Rows m..m_pad-1: codes 0, scale 1.
 *   Requires k % 8 == 0, k <= 16384, ldx/ld_scale/ld_shift/ldv multiples of 8,
 *   x, norm_w, scale, shift, values 16-byte aligned, eps finite and >= 0.
 */
int vflash_rmsnorm_modulate_quantize_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx,
                                          const void* norm_w, float eps, const void* scale,
                                          int64_t ld_scale, const void* shift, int64_t ld_shift,
                                          int64_t tokens, const int64_t* index, int64_t mod_rows,
                                          void* values, int64_t ldv, void* codes, float* scales,
                                          int64_t m_pad, void* stream);

/*
 * Per-token E4M3 requantization from epilogue row maxima.
 * Same arithmetic as vflash_quantize_rows_e4m3 (the down projection's own
 * activation quantization, src/vflash/native/h3_fp8_linear.py:102-108), with
 * amax taken as the maximum of amax_part[row, 0..parts).
 *   g bf16 [m, k] (ldg);  codes e4m3 [m_pad, k];  scales fp32 [m_pad]
 *   Requires k % 8 == 0, ldg % 8 == 0, g 16-byte aligned.
 */
int vflash_requant_rows_e4m3(const void* g, int64_t m, int64_t k, int64_t ldg,
                             const float* amax_part, int64_t parts, void* codes, float* scales,
                             int64_t m_pad, void* stream);

/*
 * FFN down-projection with the adaLN gate-residual epilogue.
 * Replaces RowFP8Execution.linear + triton_strict_bf16_gate_residual
 *   (src/vflash/native/h3_fused_ops.py:124-170, 614-657), including the gather
 *   of the gate rows, table[:, j, :].index_select(0, adaln_indices)
 *   (src/vflash/native/h3_native_denoiser.py:527-532, 556-561), read in place.
 *   y   = bf16(bf16(acc * sa * sw) + bias)
 *   out = bf16(residual[m, n] + bf16(gate[g * gate_ts + n * gate_hs] * y))
 *   g   = m % gate_tokens, or gate_index[m % gate_tokens] when gate_index is not
 *         NULL (int64, each < gate_rows; a row whose index is outside gets NaN).
 *   gate_ts = 0 broadcasts one gate row over all tokens; gate_tokens = m gives
 *   one gate row per output row.  out may alias residual only when ldo == ldr.
 */
int vflash_fp8_linear_gate_residual(const void* a, const float* sa, int64_t lda, const void* w,
                                    const float* sw, int64_t ldw, int64_t m, int64_t n,
                                    int64_t k, const void* bias, const void* gate,
                                    int64_t gate_ts, int64_t gate_hs, int64_t gate_tokens,
                                    const int64_t* gate_index, int64_t gate_rows,
                                    const void* residual, int64_t ldr, void* out, int64_t ldo,
                                    void* stream);

/*
 * vflash_fp8_linear_gate_residual with an adapter merged before the gate: the
 * adapted gate-residual of the attention output and FFN down projections.
 * Replaces _adapted_gate_residual and triton_strict_bf16_adapter_gate_residual
 *   (src/vflash/native/h3_native_denoiser.py:327-338, 551, 570, 1271-1290;
 *   src/vflash/native/h3_fused_ops.py:341-418, 982-1028):
 *   y'  = bf16(y + delta), delta as in vflash_fp8_linear_lora
 *   out = bf16(residual + bf16(gate * y'))
 *   t, lora_b NULL: no adapter (vflash_fp8_linear_gate_residual).  The adapter
 *   operands follow vflash_fp8_linear_lora; the gate and residual
 *   vflash_fp8_linear_gate_residual.
 */
int vflash_fp8_linear_lora_gate_residual(
    const void* a, const float* sa, int64_t lda, const void* w, const float* sw, int64_t ldw,
    int64_t m, int64_t n, int64_t k, const void* bias, const void* gate, int64_t gate_ts,
    int64_t gate_hs, int64_t gate_tokens, const int64_t* gate_index, int64_t gate_rows,
    const void* residual, int64_t ldr, const void* t, int64_t ldt, const void* lora_b,
    int64_t ldb, int64_t rank, float scale, float strength, void* out, int64_t ldo,
    void* stream);

/*
 * LoRA down-projection t = bf16(x . A^T) (binary32 accumulation).
 * Replaces the inner F.linear of the activation-adapter hook
 *   (src/vflash/adapters/h3_reference_lora.py:80-82).
 *   x bf16 [m, k] (ldx);  lora_a bf16 [rank, k] contiguous;  t bf16 [m, ldt]:
 *   columns [0, rank) hold t, columns [rank, ceil16(rank)) are written as zeros.
 *   Requires 1 <= rank <= 512 (three stacked Q/K/V adapters of rank 128 fit),
 *   ldt >= ceil16(rank), ldt % 8 == 0, k % 16 == 0, ldx % 8 == 0; x, lora_a, t
 *   16-byte aligned.
 * Sum order: K is cut into 8 chunks of 32-element steps, [S c / 8, S (c + 1) / 8)
 * with S = ceil(k / 32), each accumulated from zero; t = bf16 of the chunk
 * sums added in chunk order.  The order depends on k only, never on m or rank.
 */
int vflash_lora_down(const void* x, int64_t m, int64_t k, int64_t ldx, const void* lora_a,
                     int64_t rank, void* t, int64_t ldt, void* stream);

/*
 * Per-token E4M3 quantization and the LoRA down-projection of the same rows in
 * one launch: the codes and scales of vflash_quantize_rows_e4m3 bit for bit, and
 * the t of vflash_lora_down bit for bit.  Replaces quantize_activation
 * (src/vflash/native/h3_fp8_activation.py:12-55) plus the adapter hook's inner
 * F.linear (src/vflash/adapters/h3_reference_lora.py:80-82) for the adapter
 * linears.
 *   Requires k % 16 == 0, ldx % 8 == 0, m_pad >= m, the rank and t layout of
 *   vflash_lora_down; x, lora_a, t 16-byte aligned; codes 8-byte aligned.
 */
int vflash_quantize_rows_lora_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx,
                                   void* codes, float* scales, int64_t m_pad,
                                   const void* lora_a, int64_t rank, void* t, int64_t ldt,
                                   void* stream);

/*
 * W8A8 linear with a fused LoRA up-projection and merge.
 * Replaces the outer F.linear and merge of the adapter hook
 *   (src/vflash/adapters/h3_reference_lora.py:80-90):
 *   base  = vflash_fp8_linear's output
 *   delta = bf16(t . B^T); if scale != 1: bf16(delta * scale);
 *           if strength != 1: bf16(delta * strength)
 *   out   = bf16(base + delta)
 *   t bf16 [m, >= rank] (ldt);  lora_b bf16 [n, >= rank] (ldb);  1 <= rank <= 128;
 *   ldt, ldb multiples of 8 (reads stop at the rank rounded up to 8; positions
 *   at or past the rank count as zero); t, lora_b 16-byte aligned.
 */
int vflash_fp8_linear_lora(const void* a, const float* sa, int64_t lda, const void* w,
                           const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                           const void* bias, const void* t, int64_t ldt, const void* lora_b,
                           int64_t ldb, int64_t rank, float scale, float strength, void* out,
                           int64_t ldo, void* stream);

/*
 * vflash_fp8_linear_lora with up to three adapter branches, each with its own
 * scale, over equal runs of output columns: the Q/K/V adapters of a merged
 * projection.  Replaces the QKV residual pack and its merges
 *   (src/vflash/native/h3_native_denoiser.py:301-316, 1153-1194;
 *   src/vflash/native/h3_fused_ops.py:297-340, 802-838, 900-980):
 *   column c belongs to branch b = c / (n / branches);
 *   delta = bf16(t[:, b * t_branch .. + rank] . B^T) then bf16(delta * scales[b])
 *           if scales[b] != 1 and bf16(delta * strength) if strength != 1;
 *   out  = bf16(base + delta), written as one matrix (plane_cols 0, ldo) or
 *          into planes as vflash_fp8_linear_planes (plane_cols, plane_stride).
 *   lora_b bf16 [n, >= rank]: branch b's up-projection rows stacked in column
 *   order; a branch of smaller rank has zero columns up to `rank`.
 *   scales: host array of `branches` floats (read before the call returns).
 *   Requires 1 <= branches <= 3, n % branches == 0, (n / branches) % 32 == 0
 *   when branches > 1, t_branch >= rank and a multiple of 8, ldt >=
 *   (branches - 1) * t_branch + rank, and the operand rules of vflash_fp8_linear_lora.
 */
int vflash_fp8_linear_lora_branches(const void* a, const float* sa, int64_t lda, const void* w,
                                    const float* sw, int64_t ldw, int64_t m, int64_t n,
                                    int64_t k, const void* bias, const void* t, int64_t ldt,
                                    int64_t t_branch, const void* lora_b, int64_t ldb,
                                    int64_t rank, int64_t branches, const float* scales,
                                    float strength, void* out, int64_t ldo, int64_t plane_cols,
                                    int64_t plane_stride, void* stream);

/*
 * NVFP4-weight linear (W4A8: E4M3 per-token activations, E2M1 weights with
 * E4M3 scales per 16-element K block and an fp32 output multiplier).  A more
 * accurate alternative to the reference's W4A4 arithmetic
 * (vflash_nvfp4_w4a4_linear), taking the place of the same mm_fp4 call
 *   (src/vflash/native/h3_nvfp4_linear.py:118-139).
 *   a        e4m3 [m, k] (lda);  sa fp32 [m]
 *   w_packed u8 [n, k/2]: element 2j in the low nibble, 2j+1 in the high nibble
 *   w_scales u8 (e4m3) [n, k/16] in the 128x4 tiled order of NVFP4Weight
 *            (h3_nvfp4_linear.py:22-33)
 *   alpha    fp32 device scalar (NVFP4Weight.alpha; read on the device, no host sync)
 *   out = bf16(bf16(sum_k a * e2m1(w) * e4m3(s_blk) * sa[m] * alpha) + bias[n])
 *   Requires n % 128 == 0, k % 64 == 0, lda % 16 == 0, a, w_packed and w_scales
 *   16-byte aligned.
 */
int vflash_nvfp4_linear(const void* a, const float* sa, int64_t lda, const void* w_packed,
                        const void* w_scales, const float* alpha, int64_t m, int64_t n, int64_t k,
                        const void* bias, void* out, int64_t ldo, void* stream);

/*
 * NVFP4 activation quantization, the W4A4 input of the reference's NVFP4 linear.
 * Replaces nvfp4_quantize(x, input_scale, sfLayout=128x4, do_shuffle=False)
 *   (FlashInfer 0.6.18) as called at src/vflash/native/h3_nvfp4_linear.py:102-111.
 *   x          bf16 [m, k] (f16 when x_is_f16), row stride ldx
 *   global_sf  fp32 device scalar (NVFP4Weight.input_scale)
 *   per 16-element K block, binary32:
 *     sf    = e4m3(min(gsf * (amax * RN(1/6)), 448)),  scale = sf ? 1 / (sf * (1/gsf)) : 0
 *     code  = e2m1(clamp(x * scale, -6, 6))  (round to nearest even, sign kept)
 *   codes  u8 [m, k/2] (ldc bytes): element 2j in the low nibble
 *   scales u8 (e4m3) [m_pad, k/16] in the 128x4 tiled order; m_pad is a multiple
 *          of 128 >= m, and the padding rows' scales are 0 (the layout
 *          h3_nvfp4_linear.py:103-111 checks).
 *   Requires k % 64 == 0, ldx % 8 == 0, ldc % 16 == 0, ldc >= k/2, x and codes
 *   16-byte aligned, scales and global_sf 4-byte aligned.
 */
int vflash_nvfp4_quantize_rows(const void* x, int x_is_f16, int64_t m, int64_t k, int64_t ldx,
                               const float* global_sf, void* codes, int64_t ldc, void* scales,
                               int64_t m_pad, void* stream);

/*
 * W4A4 NVFP4 linear: E2M1 activations and weights, each with E4M3 scales per
 * 16-element K block in the 128x4 order, and one fp32 output scale.
 * Replaces mm_fp4(codes, W^T, scales, W_scales^T, alpha, bf16, block_size=16,
 *   backend="cutlass", use_nvfp4=True) followed by + bias
 *   (src/vflash/native/h3_nvfp4_linear.py:114-139).
 *   a        u8 [m, k/2] (lda bytes);  a_scales: as vflash_nvfp4_quantize_rows writes them
 *   w_packed u8 [n, k/2];  w_scales u8 [n, k/16], 128x4 order (NVFP4Weight)
 *   alpha    fp32 device scalar: NVFP4Weight.alpha / NVFP4Weight.input_scale
 *   out = bf16(bf16(alpha * sum_k e2m1(a) e4m3(sa_blk) e2m1(w) e4m3(sw_blk)) + bias[n])
 *   Requires n % 128 == 0, k % 64 == 0, lda % 16 == 0, a, w_packed, a_scales and
 *   w_scales 16-byte aligned.
 */
int vflash_nvfp4_w4a4_linear(const void* a, int64_t lda, const void* a_scales, const void* w_packed,
                             const void* w_scales, const float* alpha, int64_t m, int64_t n,
                             int64_t k, const void* bias, void* out, int64_t ldo, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VFLASH_AMD_H */
