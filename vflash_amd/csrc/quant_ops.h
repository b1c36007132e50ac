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

// 8 bf16 values (one 16-byte vector) -> 8 E4M3 codes packed little-endian.
// The conversion is the hardware v_cvt_pk_fp8_f32 (two values per
// instruction).  On the clamped range it is the OCP E4M3 round-to-nearest-even
// of f32_to_e4m3: an exhaustive on-device comparison over every binary32 with
// |x| <= 448, both signs, found no difference.
__device__ __forceinline__ uint2 quant8(v4i v, float scale) {
  float q[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)v[j];
    q[2 * j] = clamped_quotient(bf16_to_f32(w & 0xffffu), scale);
    q[2 * j + 1] = clamped_quotient(bf16_to_f32(w >> 16), scale);
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

}  // namespace vfa
