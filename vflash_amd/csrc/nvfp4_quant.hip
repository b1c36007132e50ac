// NVFP4 activation quantization for the W4A4 linear: the contract of
// nvfp4_quantize(x, input_scale, sfLayout=128x4) as the reference calls it
// (src/vflash/native/h3_nvfp4_linear.py:102-111; FlashInfer 0.6.18).
//
// Per row and 16-element K block, in binary32 (gsf = the global input scale):
//   sf    = e4m3(min(gsf * (amax_block * RN(1/6)), 448))      RNE
//   scale = sf != 0 ? 1 / (sf * (1 / gsf)) : 0                 IEEE reciprocals
//   q     = e2m1(clamp(x * scale, -6, 6))                      RNE, sign kept
// FlashInfer forms the two reciprocals with the hardware's approximate
// reciprocal; here they are correctly rounded.
//
// Layout: codes [m, k/2] (element 2j in the low nibble of byte j), scales in
// the 128x4 tiled order with the rows padded to m_pad (a multiple of 128,
// padding scales 0): tile (row / 128, block / 4) of 512 bytes, byte
// (row % 32) * 16 + ((row % 128) / 32) * 4 + block % 4 inside it.  Conversions: the hardware v_cvt_pk_fp8_f32 (E4M3)
// and v_cvt_scalef32_pk_fp4_f32 at scale 1 (E2M1), each checked exhaustively
// against a software round-to-nearest-even encoder on the device.
#include "common.h"

namespace vfa {

template <bool F16>
__device__ __forceinline__ float half_lo(uint32_t w) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  return bf16_lo(w);
}

template <bool F16>
__device__ __forceinline__ float half_hi(uint32_t w) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  return bf16_hi(w);
}

// One wave per row, four rows per workgroup.  Lane l of pass t reads the 8
// elements 512 t + 8 l .. +7 (16 bytes; the wave reads 1 KB contiguously), so
// a 16-element block is a lane pair: the block maximum takes one shuffle, and
// each lane writes its 4 packed bytes.  The four scales of a 128x4 word (four
// consecutive blocks) come from lanes 8u, 8u + 2, 8u + 4, 8u + 6 and are
// written by lane 8u.
template <bool F16>
__global__ void __launch_bounds__(256) nvfp4_quant_rows(const uint16_t* __restrict__ x, int64_t m,
                                                        int64_t k, int64_t ldx,
                                                        const float* __restrict__ global_sf,
                                                        uint8_t* __restrict__ codes, int64_t ldc,
                                                        uint8_t* __restrict__ scales,
                                                        int64_t m_pad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m_pad) return;
  const int64_t groups = k / 64;  // 128x4 scale words per row
  uint8_t* srow = scales + (row / 128) * groups * 512 + (row % 32) * 16 + ((row % 128) / 32) * 4;
  if (row >= m) {
    for (int64_t gi = lane; gi < groups; gi += 64) *reinterpret_cast<uint32_t*>(srow + gi * 512) = 0u;
    return;
  }
  const float gsf = *global_sf;
  const float inv_gsf = 1.0f / gsf;
  constexpr float SIXTH = 1.0f / 6.0f;
  const v4i* xr = reinterpret_cast<const v4i*>(x + row * ldx);
  uint32_t* cr = reinterpret_cast<uint32_t*>(codes + row * ldc);
  const int nvec = (int)(k / 8);
  for (int base = 0; base < nvec; base += 64) {  // uniform over the wave: shuffles below
    const int j = base + lane;
    const bool live = j < nvec;  // k % 64 == 0: whole 8-lane groups are live together
    const v4i v = live ? __builtin_nontemporal_load(xr + j) : v4i{};
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = (uint32_t)v[e];
      amax = fmaxf(amax, fmaxf(fabsf(half_lo<F16>(w)), fabsf(half_hi<F16>(w))));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));  // the block: this lane and its pair
    const float sff = fminf(gsf * (amax * SIXTH), 448.0f);
    const uint32_t sfc = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(sff, sff, 0, false) & 0xffu;
    const float sf = e4m3_to_f32(sfc);
    const float scale = sf != 0.0f ? 1.0f / (sf * inv_gsf) : 0.0f;
    uint32_t word = 0u;
    static_for<4>([&](auto e) {
      const uint32_t w = (uint32_t)v[(int)e];
      const float lo = fminf(fmaxf(half_lo<F16>(w) * scale, -6.0f), 6.0f);
      const float hi = fminf(fmaxf(half_hi<F16>(w) * scale, -6.0f), 6.0f);
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, lo, hi, 1.0f, (int)e);
    });
    const uint32_t s2 = (uint32_t)__shfl_down((int)sfc, 2, 64);
    const uint32_t s4 = (uint32_t)__shfl_down((int)sfc, 4, 64);
    const uint32_t s6 = (uint32_t)__shfl_down((int)sfc, 6, 64);
    if (live) {
      cr[j] = word;
      if ((lane & 7) == 0)
        *reinterpret_cast<uint32_t*>(srow + (int64_t)(j / 8) * 512) =
            sfc | (s2 << 8) | (s4 << 16) | (s6 << 24);
    }
  }
}

hipError_t launch_nvfp4_quant(const uint16_t* x, bool f16, int64_t m, int64_t k, int64_t ldx,
                              const float* global_sf, uint8_t* codes, int64_t ldc,
                              uint8_t* scales, int64_t m_pad, hipStream_t s) {
  const dim3 grid((unsigned)((m_pad + 3) / 4));
  if (f16)
    nvfp4_quant_rows<true><<<grid, 256, 0, s>>>(x, m, k, ldx, global_sf, codes, ldc, scales, m_pad);
  else
    nvfp4_quant_rows<false><<<grid, 256, 0, s>>>(x, m, k, ldx, global_sf, codes, ldc, scales, m_pad);
  return hipGetLastError();
}

}  // namespace vfa
