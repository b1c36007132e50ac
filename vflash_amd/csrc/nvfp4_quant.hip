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
// (row % 32) * 16 + ((row % 128) / 32) * 4 + block % 4 inside it.  One thread
// owns 64 elements of a row, i.e. the four blocks whose scales form one
// 32-bit word of a tile.  Conversions: the hardware v_cvt_pk_fp8_f32 (E4M3)
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

template <bool F16>
__global__ void __launch_bounds__(256) nvfp4_quant_rows(const uint16_t* __restrict__ x, int64_t m,
                                                        int64_t k, int64_t ldx,
                                                        const float* __restrict__ global_sf,
                                                        uint8_t* __restrict__ codes, int64_t ldc,
                                                        uint8_t* __restrict__ scales,
                                                        int64_t m_pad) {
  const int64_t groups = k / 64;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t / groups, g = t - row * groups;
  if (row >= m_pad) return;
  uint32_t* sw = reinterpret_cast<uint32_t*>(scales + (row / 128) * groups * 512 + g * 512 +
                                             (row % 32) * 16 + ((row % 128) / 32) * 4);
  if (row >= m) {
    *sw = 0u;
    return;
  }
  const float gsf = *global_sf;
  const float inv_gsf = 1.0f / gsf;
  constexpr float SIXTH = 1.0f / 6.0f;
  const v4i* xr = reinterpret_cast<const v4i*>(x + row * ldx + g * 64);
  v4i v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __builtin_nontemporal_load(xr + i);
  uint32_t sfw = 0u;
  uint32_t out[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float amax = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (uint32_t)v[2 * b + h][e];
        amax = fmaxf(amax, fmaxf(fabsf(half_lo<F16>(w)), fabsf(half_hi<F16>(w))));
      }
    }
    const float sff = fminf(gsf * (amax * SIXTH), 448.0f);
    const uint32_t sfc = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(sff, sff, 0, false) & 0xffu;
    const float sf = e4m3_to_f32(sfc);
    const float scale = sf != 0.0f ? 1.0f / (sf * inv_gsf) : 0.0f;
    sfw |= sfc << (8 * b);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t word = 0u;
      static_for<4>([&](auto e) {
        const uint32_t w = (uint32_t)v[2 * b + h][(int)e];
        const float lo = fminf(fmaxf(half_lo<F16>(w) * scale, -6.0f), 6.0f);
        const float hi = fminf(fmaxf(half_hi<F16>(w) * scale, -6.0f), 6.0f);
        word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, lo, hi, 1.0f, (int)e);
      });
      out[2 * b + h] = word;
    }
  }
  v4i* cr = reinterpret_cast<v4i*>(codes + row * ldc + g * 32);
  cr[0] = v4i{(int)out[0], (int)out[1], (int)out[2], (int)out[3]};
  cr[1] = v4i{(int)out[4], (int)out[5], (int)out[6], (int)out[7]};
  *sw = sfw;
}

hipError_t launch_nvfp4_quant(const uint16_t* x, bool f16, int64_t m, int64_t k, int64_t ldx,
                              const float* global_sf, uint8_t* codes, int64_t ldc,
                              uint8_t* scales, int64_t m_pad, hipStream_t s) {
  const int64_t threads = m_pad * (k / 64);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (f16)
    nvfp4_quant_rows<true><<<grid, 256, 0, s>>>(x, m, k, ldx, global_sf, codes, ldc, scales, m_pad);
  else
    nvfp4_quant_rows<false><<<grid, 256, 0, s>>>(x, m, k, ldx, global_sf, codes, ldc, scales, m_pad);
  return hipGetLastError();
}

}  // namespace vfa
