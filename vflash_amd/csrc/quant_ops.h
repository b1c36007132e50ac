// Per-row E4M3 quantization arithmetic shared by the quantization kernels
// (reference: src/vflash/native/h3_fp8_activation.py:12-28,
// src/vflash/native/h3_fp8_linear.py:18-31).  Kernel-side only.
#pragma once
#include "common.h"

namespace vfa {

__device__ __forceinline__ float absmax8(v4i v) {
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t w = (uint32_t)v[j];
    m = fmaxf(m, fabsf(bf16_to_f32(w & 0xffffu)));
    m = fmaxf(m, fabsf(bf16_to_f32(w >> 16)));
  }
  return m;
}

__device__ __forceinline__ float row_scale(float amax) {
  return amax > 0.0f ? fmaxf(amax / 448.0f, VFA_FLT_MIN) : 1.0f;
}

__device__ __forceinline__ float clamped_quotient(float x, float scale) {
  return fminf(fmaxf(x / scale, -448.0f), 448.0f);
}

__device__ __forceinline__ uint32_t quant1(float x, float scale) {
  return f32_to_e4m3(clamped_quotient(x, scale));
}

// Division of a row by its scale.
//
// The IEEE quotient x / s costs about ten VALU instructions per element, which
// makes the row kernels instruction-bound.  The divisor is fixed per row, so
// rows with 2^-72 <= s <= FLT_MAX use Markstein's correction on the correctly
// rounded reciprocal y = RN(1/s), formed once per row:
//   q0 = RN(x y),  r = x - q0 s (exact, one fma),  q = RN(q0 + r y).
// The residual is formed negated, r' = RN(q0 s - x) = -r, and the correction
// as RN(q0 + r' (-y)): the same value (RN is symmetric) with the sign of a
// zero quotient right (x = -0 gives -0), at no extra instruction.  For every
// bf16 x with |x| <= amax,
// the E4M3 code of clamp(q) equals that of clamp(x / s): an exhaustive check
// over all pairs of bf16 values finds the first disagreement at amax near
// 2^-104.7, in rows whose residual underflows, far below the bound here
// (s >= 2^-72 means amax > 2^-64).  Rows outside the bound, including
// non-finite scales, divide exactly.  The on-device probe
// tests/probes/row_division.hip repeats the comparison on the GPU.
struct RowDivisor {
  float s, y;
  bool fast;  // uniform over the wave: the scale must be
};

__device__ __forceinline__ RowDivisor row_divisor(float s) {
  RowDivisor d;
  d.s = s;
  d.y = 1.0f / s;
  d.fast = __builtin_amdgcn_readfirstlane((s >= 0x1p-72f && s <= 3.40282347e38f) ? 1 : 0) != 0;
  return d;
}

template <bool FAST>
__device__ __forceinline__ float row_quotient(float x, const RowDivisor& d) {
  if constexpr (FAST) {
    const float q0 = x * d.y;
    const float r = __builtin_fmaf(q0, d.s, -x);
    return __builtin_fmaf(r, -d.y, q0);
  } else {
    return x / d.s;
  }
}

template <bool FAST>
__device__ __forceinline__ float clamped_row_quotient(float x, const RowDivisor& d) {
  return fminf(fmaxf(row_quotient<FAST>(x, d), -448.0f), 448.0f);
}

// 8 bf16 values (one 16-byte vector) -> 8 E4M3 codes packed little-endian.
// The conversion is the hardware v_cvt_pk_fp8_f32 (two values per
// instruction).  On the clamped range it is the OCP E4M3 round-to-nearest-even
// of f32_to_e4m3: an exhaustive on-device comparison over every binary32 with
// |x| <= 448, both signs, found no difference.
template <bool FAST>
__device__ __forceinline__ uint2 quant8(v4i v, const RowDivisor& d) {
  float q[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)v[j];
    q[2 * j] = clamped_row_quotient<FAST>(bf16_lo(w), d);
    q[2 * j + 1] = clamped_row_quotient<FAST>(bf16_hi(w), d);
  }
  uint2 r;
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
  r.x = (uint32_t)lo;
  r.y = (uint32_t)hi;
  return r;
}

// Codes of one row held in registers: vector i of this lane is element
// vector lane + 64 i of the row (i < VPL, lane + 64 i < nvec).
template <int VPL>
__device__ __forceinline__ void quant_row_regs(uint2* cr, const v4i (&v)[VPL], int lane, int nvec,
                                               float scale) {
  const RowDivisor d = row_divisor(scale);
  if (d.fast) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < nvec) cr[j] = quant8<true>(v[i], d);
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < nvec) cr[j] = quant8<false>(v[i], d);
    }
  }
}

}  // namespace vfa
