// LoRA down-projection t = bf16(x . A^T) for gfx950, alone or fused with the
// per-token E4M3 quantization of the same rows.
//
// Reference: the inner F.linear of the activation-adapter hook
// (src/vflash/adapters/h3_reference_lora.py:80-82), bf16 operands with a
// binary32 accumulator and one bf16 rounding of the result; the fused form
// also produces the codes and scales of quantize_activation
// (src/vflash/native/h3_fp8_activation.py:12-55) for the base linear, so the
// activation rows are read once for both.
//
// lora_rows_kernel: the adapter rank is small (16..128) and K is the model
// width, so the work per row is a few dot products of length K and the kernel
// is latency-bound.  One 512-thread workgroup owns 32 rows of x; its 8 waves
// split K eight ways and issue the loads of several K-steps before the MFMAs
// that consume them (v_mfma_f32_32x32x16_bf16, adapter rows as operand A,
// activation rows as operand B).  The 8 partial accumulators are summed
// through LDS in a fixed order (wave 0, 1, ..., 7), one 32-column rank block
// at a time.
#include "quant_ops.h"

namespace vfa {

constexpr int LORA_WAVES = 8;

template <int RB>  // RB = rank / 32 blocks (rank 16 uses one half-filled block)
__global__ void __launch_bounds__(64 * LORA_WAVES) lora_rows_kernel(
    const uint16_t* __restrict__ x, int64_t m, int64_t k, int64_t ldx,
    const uint16_t* __restrict__ a, int rank, uint16_t* __restrict__ t) {
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
  auto load_x = [&](int64_t s) {
    return (s < s1 && mok) ? *reinterpret_cast<const v8s*>(x + mrow * ldx + s * 16 + fh * 8)
                           : v8s{};
  };
  auto load_a = [&](int64_t s, int b) {
    const int r = b * 32 + fr;
    return (s < s1 && r < rank)
               ? *reinterpret_cast<const v8s*>(a + (int64_t)r * k + s * 16 + fh * 8)
               : v8s{};
  };
  auto mma = [&](const v8s& xf, const v8s (&af)[RB]) {
#pragma unroll
    for (int b = 0; b < RB; ++b)
      acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, af[b]),
                                                       __builtin_bit_cast(v8bf, xf), acc[b],
                                                       0, 0, 0);
  };

  {
    // K-steps whose loads are in flight together (512-thread workgroups leave
    // 256 VGPRs per lane).
    constexpr int CHUNK = RB <= 2 ? 8 : 4;
    for (int64_t c0 = s0; c0 < s1; c0 += CHUNK) {
      v8s xf[CHUNK], af[CHUNK][RB];
#pragma unroll
      for (int i = 0; i < CHUNK; ++i) {
        xf[i] = load_x(c0 + i);
#pragma unroll
        for (int b = 0; b < RB; ++b) af[i][b] = load_a(c0 + i, b);
      }
#pragma unroll
      for (int i = 0; i < CHUNK; ++i)
        if (c0 + i < s1) mma(xf[i], af[i]);
    }
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

// Row-parallel fused pass for the skinny adapter linears: one wave per row, 4
// rows per workgroup, so every CU gets rows at M = 1024.  The adapter matrix A
// [R, K] is copied into LDS once per workgroup (buffer-load-to-LDS DMA) while
// the wave loads its row into registers.  Each lane forms R partial dot
// products over its 8-element K vectors (binary32 FMAs), a halving butterfly reduces them across the wave (R = 32: 32
// shuffles) and the same registers are quantized exactly as
// vflash_quantize_rows_e4m3 does.  t is bf16 of a binary32 sum in another
// order than the MFMA kernel, so it can differ from vflash_lora_down where the
// dot product cancels; the codes and scales are identical.
constexpr int QL_VPL = 4;        // 8-element vectors per lane: K <= 2048
constexpr int QL_LDS = 131072;   // bytes of A in LDS: rank * K <= 65536

template <int R>  // rank: 16, 32 or 64
__global__ void __launch_bounds__(256) quant_lora_rows(
    const uint16_t* __restrict__ x, int64_t m, int64_t k, int64_t ldx,
    const uint16_t* __restrict__ a, uint16_t* __restrict__ t, uint8_t* __restrict__ codes,
    float* __restrict__ scales, int64_t m_pad) {
  __shared__ __attribute__((aligned(1024))) uint8_t a_lds[QL_LDS];  // A: R x k bf16
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  const int nvec = (int)(k >> 3);

  // Row into registers (zeros past the matrix: padding rows quantize to code 0, scale 1).
  v4i v[QL_VPL];
  const bool live = row < m;
  const v4i* xr = reinterpret_cast<const v4i*>(x + (live ? row : 0) * ldx);
  static_for<QL_VPL>([&](auto i) {
    const int j = lane + 64 * i;
    v[i] = (live && j < nvec) ? __builtin_nontemporal_load(xr + j) : v4i{};
  });
  // A into LDS: 1 KB per DMA instruction, blocks spread over the 4 waves.
  const uint32_t a_bytes = (uint32_t)(R * k * 2);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, a_bytes);
  const uint32_t a_base = __builtin_amdgcn_readfirstlane(lds_addr(a_lds));
  for (uint32_t blk = wave; blk * 1024 < a_bytes; blk += 4)
    lds_dma16(ra, a_base + blk * 1024, blk * 1024 + (uint32_t)lane * 16);
  wait_vmcnt<0, true>();
  __syncthreads();

  // Partial dot products of this lane's vectors with every adapter row.
  float part[R];
  static_for<R>([&](auto r) { part[r] = 0.0f; });
  static_for<QL_VPL>([&](auto i) {
    const int j = lane + 64 * i;
    if (j < nvec) {
      float xv[8];
      static_for<4>([&](auto h) {
        xv[2 * h] = bf16_lo((uint32_t)v[i][(int)h]);
        xv[2 * h + 1] = bf16_hi((uint32_t)v[i][(int)h]);
      });
      static_for<R>([&](auto r) {
        const v4i av = *reinterpret_cast<const v4i*>(a_lds + ((int64_t)r * k + 8 * j) * 2);
        float acc = part[r];
        static_for<4>([&](auto h) {
          acc = __builtin_fmaf(xv[2 * h], bf16_lo((uint32_t)av[(int)h]), acc);
          acc = __builtin_fmaf(xv[2 * h + 1], bf16_hi((uint32_t)av[(int)h]), acc);
        });
        part[r] = acc;
      });
    }
  });
  // Halving butterfly: after the step with lane bit b, a lane keeps the half of
  // its values selected by that bit, summed with its partner's copy.
  constexpr int LG = R == 16 ? 4 : (R == 32 ? 5 : 6);
  static_for<LG>([&](auto st) {
    constexpr int n = R >> (st + 1);  // values kept after this step
    constexpr int o = 32 >> st;       // partner lane offset
    const bool up = (lane & o) != 0;
    static_for<n>([&](auto i2) {
      const float mine = up ? part[i2 + n] : part[i2];
      const float other = up ? part[i2] : part[i2 + n];
      part[i2] = mine + __shfl_xor(other, o, 64);
    });
  });
  float tv = part[0];
  // Lanes that differ only in the low 6 - LG bits hold partial sums of one value.
  static_for<6 - LG>([&](auto st) { tv += __shfl_xor(tv, 1 << st, 64); });
  // Lane bits 5 .. 6-LG select the value, most significant first.
  const int r_idx = lane >> (6 - LG);
  if (live && (lane & ((1 << (6 - LG)) - 1)) == 0) t[row * R + r_idx] = (uint16_t)f32_to_bf16(tv);

  // Quantization of the same registers (the arithmetic of quant_rows_vec).
  if (row < m_pad) {
    float amax = 0.0f;
    static_for<QL_VPL>([&](auto i) { amax = nan_max(amax, absmax8(v[i])); });
    amax = wave_nan_max(amax);
    const float scale = row_scale(amax);
    quant_row_regs<QL_VPL>(reinterpret_cast<uint2*>(codes + row * k), v, lane, nvec, scale, amax);
    if (lane == 0) scales[row] = scale;
  }
}

hipError_t launch_lora_down(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                            const uint16_t* a, int rank, uint16_t* t, hipStream_t s) {
  const dim3 grid((unsigned)((m + 31) / 32)), block(64 * LORA_WAVES);
  switch ((rank + 31) / 32) {
    case 1: lora_rows_kernel<1><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 2: lora_rows_kernel<2><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 3: lora_rows_kernel<3><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    case 4: lora_rows_kernel<4><<<grid, block, 0, s>>>(x, m, k, ldx, a, rank, t); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_quant_lora(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                             const uint16_t* a, int rank, uint16_t* t, uint8_t* codes,
                             float* scales, int64_t m_pad, hipStream_t s) {
  const dim3 grid((unsigned)((m_pad + 3) / 4)), block(256);
  if (rank * k * 2 > QL_LDS || k > 512 * QL_VPL) return hipErrorInvalidValue;
  switch (rank) {
    case 16: quant_lora_rows<16><<<grid, block, 0, s>>>(x, m, k, ldx, a, t, codes, scales, m_pad); break;
    case 32: quant_lora_rows<32><<<grid, block, 0, s>>>(x, m, k, ldx, a, t, codes, scales, m_pad); break;
    case 64: quant_lora_rows<64><<<grid, block, 0, s>>>(x, m, k, ldx, a, t, codes, scales, m_pad); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace vfa
