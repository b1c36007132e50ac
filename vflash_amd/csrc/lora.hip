// LoRA down-projection t = bf16(x . A^T) for gfx950.
//
// Reference: the inner F.linear of the activation-adapter hook
// (src/vflash/adapters/h3_reference_lora.py:80-82), bf16 operands with a
// binary32 accumulator and one bf16 rounding of the result.
//
// The adapter rank is small (16..128) and K is the model width, so the work per
// row is a few dot products of length K: the kernel is latency-bound, not
// compute-bound.  One 1024-thread workgroup owns 32 rows of x; its 16 waves
// split K sixteen ways and issue all loads of a chunk of K-steps (8 at rank 32)
// before the MFMAs that consume them (v_mfma_f32_32x32x16_bf16, adapter rows
// as operand A, activation rows as operand B).  The 16 partial accumulators
// are summed through LDS in a fixed order (wave 0, 1, ..., 15), one 32-column
// rank block at a time.
#include "common.h"

namespace vfa {

constexpr int LORA_WAVES = 16;

template <int RB>  // rank / 32 blocks (rank 16 uses one half-filled block)
__global__ void __launch_bounds__(64 * LORA_WAVES) lora_down_kernel(
    const uint16_t* __restrict__ x, int64_t m, int64_t k, int64_t ldx,
    const uint16_t* __restrict__ a, int rank, uint16_t* __restrict__ t) {
  // K-steps (16 elements) whose loads are in flight together; 1024-thread
  // workgroups leave 128 VGPRs per lane.
  constexpr int LORA_CHUNK = RB == 1 ? 8 : (RB == 2 ? 4 : 2);
  __shared__ float red[LORA_WAVES][16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 32;
  const int fr = lane & 31, fh = lane >> 5;
  const int64_t mrow = m0 + fr;
  const bool mok = mrow < m;

  // K range of this wave, in 16-element steps.
  const int64_t steps = k / 16;
  const int64_t s0 = steps * wave / LORA_WAVES, s1 = steps * (wave + 1) / LORA_WAVES;

  v16f acc[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) acc[b] = v16f{};
  for (int64_t c0 = s0; c0 < s1; c0 += LORA_CHUNK) {
    v8s xf[LORA_CHUNK], af[LORA_CHUNK][RB];
#pragma unroll
    for (int i = 0; i < LORA_CHUNK; ++i) {
      const int64_t s = c0 + i;
      const int64_t kk = s * 16 + fh * 8;
      const bool sok = s < s1;
      xf[i] = (sok && mok) ? *reinterpret_cast<const v8s*>(x + mrow * ldx + kk) : v8s{};
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int r = b * 32 + fr;
        af[i][b] = (sok && r < rank) ? *reinterpret_cast<const v8s*>(a + (int64_t)r * k + kk)
                                     : v8s{};
      }
    }
#pragma unroll
    for (int i = 0; i < LORA_CHUNK; ++i)
#pragma unroll
      for (int b = 0; b < RB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, af[i][b]),
                                                         __builtin_bit_cast(v8bf, xf[i]), acc[b],
                                                         0, 0, 0);
  }
  // Lane holds t[m0 + fr, b*32 + 8*(q/4) + 4*fh + q%4] in acc[b][q].
#pragma unroll
  for (int b = 0; b < RB; ++b) {
#pragma unroll
    for (int q = 0; q < 16; ++q) red[wave][q][lane] = acc[b][q];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = b * 32 + g * 8 + fh * 4;
        if (!mok || r >= rank) continue;
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = g * 4 + i;
          float v = red[0][q][lane];
#pragma unroll
          for (int w = 1; w < LORA_WAVES; ++w) v += red[w][q][lane];
          o[i] = f32_to_bf16(v);
        }
        *reinterpret_cast<uint2*>(t + mrow * rank + r) =
            make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
      }
    }
    __syncthreads();
  }
}

hipError_t launch_lora_down(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                            const uint16_t* a, int rank, uint16_t* t, hipStream_t s) {
  const dim3 grid((unsigned)((m + 31) / 32)), block(64 * LORA_WAVES);
  switch ((rank + 31) / 32) {
    case 1: lora_down_kernel<1><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 2: lora_down_kernel<2><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 3: lora_down_kernel<3><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 4: lora_down_kernel<4><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace vfa
