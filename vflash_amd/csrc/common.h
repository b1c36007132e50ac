// Device helpers shared by the gfx950 kernels of the quantized-linear path.
//
// Number formats follow the OCP 8-bit floating point specification (E4M3 with
// no infinities, max 448, NaN = S.1111.111) and the OCP MX specification for
// E2M1 (values 0, 0.5, 1, 1.5, 2, 3, 4, 6).  bfloat16 is the upper half of an
// IEEE binary32.  All conversions here are written from those definitions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace vfa {

// Compile-time loop: f(std::integral_constant<int, i>) for i in [0, N).  Keeps
// every index into accumulator arrays a constant, so they stay in registers.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

// The binary32 value of FLT_MIN (2^-126), the floor of every row scale.
#define VFA_FLT_MIN 1.1754943508222875e-38f

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// binary32 -> bfloat16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950);
// NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two binary32 values -> one packed bf16 pair (low half = a), RNE, one
// v_cvt_pk_bf16_f32.  Written as an instruction the compiler keeps whole:
// when the two halves of a pair are read back separately it would otherwise
// convert each value on its own and re-extract it with shifts and masks.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// bf16(f) widened back to binary32 by one v_cvt_pk_bf16_f32: the rounded
// value lands in the high half and zero in the low half, so no shift or mask
// extracts it.
__device__ __forceinline__ float round_bf16_wide(float f) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(f));
  return __uint_as_float(r);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round a binary32 to the nearest bfloat16 and widen it back.
__device__ __forceinline__ float round_bf16(float f) { return (float)(__bf16)f; }

// binary32 -> E4M3 (OCP "fn" variant) with round to nearest even.  The caller
// has already clamped |f| <= 448, so the result never overflows; NaN maps to
// the NaN code with the input's sign.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  uint32_t code;
  if (a < 0x3c800000u) {
    // Below 2^-6 the format is uniform with step 2^-9: scale by 2^9 (exact)
    // and round to an integer 0..8; 8 is the encoding of 2^-6 itself.
    code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    // Normal range: re-bias the exponent (127 -> 7) and round the 23-bit
    // mantissa to 3 bits; a carry moves into the exponent field as it should.
    uint32_t t = a - (120u << 23);
    t += 0x7ffffu + ((t >> 20) & 1u);
    code = t >> 20;
  }
  return sign | code;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu;
  uint32_t m = c & 7u;
  float v;
  if ((c & 0x7fu) == 0x7fu) return __uint_as_float(s | 0x7fc00000u);
  if (e == 0) v = (float)m * (1.0f / 512.0f);
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(v) | s);
}

// The lane's index in its wave, computed afresh: the volatile statement is not
// merged with an earlier computation, so a value needed before and after a long
// loop is recomputed instead of holding a register through the loop.
__device__ __forceinline__ int lane_id_fresh() {
  int lo, lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0" : "=v"(lo));
  asm volatile("v_mbcnt_hi_u32_b32 %0, -1, %1" : "=v"(lane) : "v"(lo));
  return lane;
}

// Raw buffer resources: loads outside [0, num_records) return zero and stores
// there are dropped, which gives free bounds checks at tile edges.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// LDS tiles store rows of eight 16-byte chunks; chunk j of row r sits in slot
// j ^ lds_swizzle(r).  For the rows read together by one ds_read_b128 (16
// consecutive rows for a 64-bank LDS, 8 for a 32-bank one) the slots, taken
// modulo the bank width, are all distinct, so fragment reads are conflict free.
// The key depends on row bits 0..3 only: rows congruent modulo 16 share it.
__device__ __forceinline__ int lds_swizzle(int row) { return (row ^ ((row >> 3) & 1)) & 7; }

// An offset that is always past num_records (num_records < 2^31 by construction).
#define VFA_OOB 0x80000000u

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Wave-wide buffer load straight into LDS (buffer_load_dwordx4 ... lds): the
// 16 bytes lane l reads at `voffset` land at LDS byte address lds_dst + 16 * l,
// where lds_dst (wave-uniform) is an address from lds_addr().  Out-of-range
// offsets deliver zeros.  It is written as inline assembly so that the
// compiler inserts no waits for it: the caller waits with vmcnt (and a barrier
// for other waves' loads) before it reads the destination, and must not let
// the kernel end with one pending.  The statement has no memory clobber, so
// LDS reads of other buffers may be scheduled around it; ordering against
// reads of the destination comes from the caller's barrier, which is fenced
// by "memory"-clobbering volatile statements that volatile DMAs never cross.
// lds_dst must be wave-uniform in the compiler's analysis (derived from
// scalars or readfirstlane), since it is passed in an SGPR.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds_dst,
                                          uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_dst), "v"(voffset), "s"(r)
               : "m0");
}

// lds_dma16 with a scalar byte offset added to the lane offset (soffset): the
// K advance of a stage then costs no vector instruction.  The resource's range
// check covers the lane offset only, not soffset, so it no longer protects the
// bytes soffset reaches: callers use this form only where every lane offset +
// soffset they form lies inside the operand (the GEMM's full tiles).
__device__ __forceinline__ void lds_dma16_so(__amdgpu_buffer_rsrc_t r, uint32_t lds_dst,
                                             uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_dst), "v"(voffset), "s"(r), "s"(soffset)
               : "m0");
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8); LGKM selects
// whether outstanding LDS/scalar operations must also drain.
template <int VMCNT, bool LGKM>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(VMCNT >= 0 && VMCNT < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VMCNT & 15) | ((VMCNT >> 4) << 14) | (7 << 4) |
                             ((LGKM ? 0 : 15) << 8));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Row maxima with NaN propagated, as torch's amax does: the bit patterns of
// |x| (sign cleared) order like |x| with every NaN above infinity, so an
// unsigned maximum of patterns is the maximum of |x|, or NaN when any x is NaN.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Maximum of v over each 16-lane row of the wave, in every lane of the row:
// DPP quad permutations [1,0,3,2] and [2,3,0,1], then the half-row and row
// mirrors (lane i with 7 - i, then with 15 - i).  All lanes must be active.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

// acc (two 16-bit |bf16| patterns) updated with the two bf16 of word w.
__device__ __forceinline__ uint32_t abs_max_pk(uint32_t acc, uint32_t w) {
  const u16x2 a = __builtin_bit_cast(u16x2, acc), b = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}

// binary32 value of the larger of the two halves of abs_max_pk's accumulator.
__device__ __forceinline__ float abs_max_value(uint32_t acc) {
  return __uint_as_float(max(acc & 0xffffu, acc >> 16) << 16);
}

// Maximum of two non-negative binary32 values (NaN with the sign cleared included).
__device__ __forceinline__ float nan_max(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

__device__ __forceinline__ float wave_nan_max(float v) {
  uint32_t u = __float_as_uint(v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) u = max(u, (uint32_t)__shfl_xor((int)u, o, 64));
  return __uint_as_float(u);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// E2M1 (OCP MX): bit 3 sign, bits 2..1 exponent (bias 1), bit 0 mantissa.
// Codes 0..7 are 0, .5, 1, 1.5, 2, 3, 4, 6.  Built as binary32 bits directly.
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
  uint32_t e = (c >> 1) & 3u, m = c & 1u;
  uint32_t bits = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3f000000u : 0u);
  return __uint_as_float(bits | ((c & 8u) << 28));
}

// binary32 -> OCP E2M1 code, round to nearest even on the clamped range
// |f| <= 6 (values 0, 0.5, 1, 1.5, 2, 3, 4, 6; ties 0.25 -> 0, 0.75 -> 1,
// 1.25 -> 1, 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4), sign in bit 3 (-0 keeps
// it).  The reference encoder of the on-device conversion check.
__device__ __forceinline__ uint32_t f32_to_e2m1(float f) {
  const float a = fabsf(f);
  const uint32_t c = (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) +
                     (a >= 3.5f) + (a > 5.0f);
  return c | ((__float_as_uint(f) >> 28) & 8u);
}

}  // namespace vfa
