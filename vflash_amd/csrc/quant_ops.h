// Per-row E4M3 quantization arithmetic shared by the quantization kernels
// (reference: src/vflash/native/h3_fp8_activation.py:12-28,
// src/vflash/native/h3_fp8_linear.py:18-31).  Kernel-side only.
#pragma once
#include "common.h"

namespace vfa {

// GEMM padding row [m, m_pad): codes 0, scale 1 (one wave).
__device__ __forceinline__ void pad_row(uint8_t* codes, float* scales, int64_t row, int64_t k,
                                        int lane) {
  uint8_t* c = codes + row * k;
  for (int64_t j = lane; j < k; j += 64) c[j] = 0;
  if (lane == 0) scales[row] = 1.0f;
}

// max |x| over 8 bf16 values (one 16-byte vector), NaN propagated (abs_max_pk).
__device__ __forceinline__ float absmax8(v4i v) {
  uint32_t acc = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = abs_max_pk(acc, (uint32_t)v[j]);
  return abs_max_value(acc);
}

// amax > 0 ? max(amax / 448, FLT_MIN) : 1.  A NaN maximum gives 1 (NaN > 0 is
// false) and an infinite one gives infinity, as the reference's torch.where does.
__device__ __forceinline__ float row_scale(float amax) {
  return amax > 0.0f ? fmaxf(amax / 448.0f, VFA_FLT_MIN) : 1.0f;
}

// clamp(q, -448, 448) with NaN kept (torch.clamp), for rows that may hold NaN.
__device__ __forceinline__ float clamp448_keep_nan(float q) {
  return q != q ? q : fminf(fmaxf(q, -448.0f), 448.0f);
}

__device__ __forceinline__ uint32_t quant1(float x, float scale) {
  return f32_to_e4m3(clamp448_keep_nan(x / scale));
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
  bool fast;  // uniform over the wave: the scale and the row maximum must be
};

// Rows whose maximum is NaN or infinite take the exact path, where the clamp
// keeps NaN and the software encoder gives it the NaN code (the reference's
// torch.clamp and float8 cast); every finite row with a scale in range takes
// the fast path, where no x can be NaN.
__device__ __forceinline__ RowDivisor row_divisor(float s, float amax) {
  RowDivisor d;
  d.s = s;
  d.y = 1.0f / s;
  const bool fast = amax <= 3.40282347e38f && s >= 0x1p-72f && s <= 3.40282347e38f;
  d.fast = __builtin_amdgcn_readfirstlane(fast ? 1 : 0) != 0;
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
  if constexpr (FAST) return fminf(fmaxf(row_quotient<true>(x, d), -448.0f), 448.0f);
  return clamp448_keep_nan(row_quotient<false>(x, d));
}

// 8 bf16 values (one 16-byte vector) -> 8 E4M3 codes packed little-endian.
// The conversion is the hardware v_cvt_pk_fp8_f32 (two values per
// instruction).  On the clamped range it is the OCP E4M3 round-to-nearest-even
// of f32_to_e4m3: an exhaustive on-device comparison over every binary32 with
// |x| <= 448, both signs, found no difference.
template <bool FAST>
__device__ __forceinline__ uint2 quant8(v4i v, const RowDivisor& d) {
  if constexpr (!FAST) {
    // Exact path: IEEE division, NaN kept, software encoder (NaN -> 0x7f | sign).
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = (uint32_t)v[j];
      c[2 * j] = f32_to_e4m3(clamped_row_quotient<false>(bf16_lo(w), d));
      c[2 * j + 1] = f32_to_e4m3(clamped_row_quotient<false>(bf16_hi(w), d));
    }
    return make_uint2(c[0] | c[1] << 8 | c[2] << 16 | c[3] << 24,
                      c[4] | c[5] << 8 | c[6] << 16 | c[7] << 24);
  }
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
                                               float scale, float amax) {
  const RowDivisor d = row_divisor(scale, amax);
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
