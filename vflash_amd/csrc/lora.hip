// LoRA down-projection t = bf16(x . A^T) for gfx950, alone or fused with the
// per-token E4M3 quantization of the same rows.
//
// Reference: the inner F.linear of the activation-adapter hook
// (src/vflash/adapters/h3_reference_lora.py:80-82), bf16 operands with a
// binary32 accumulator and one bf16 rounding of the result; the fused form
// also produces the codes and scales of quantize_activation
// (src/vflash/native/h3_fp8_activation.py:12-55) for the base linear, so the
// adapter's rows need no separate quantization launch.
//
// The adapter rank is small (at most a few hundred, three stacked Q/K/V
// adapters of rank 128 at most) and K is the model width, so each output
// is a dot product of length K and the work per row is tiny: the kernel is
// latency-bound, and its parallelism has to come from splitting rows, ranks
// and K.  One 512-thread workgroup owns a 16-row x 16-rank block of t; its 8
// waves take K in 8 fixed chunks (chunk c = 32-element steps
// [S c / 8, S (c + 1) / 8), S = ceil(K / 32)), each an accumulation chain of
// v_mfma_f32_16x16x32_bf16 (adapter rows as operand A, activation rows as
// operand B) from k = 0 upwards, and wave 0 adds the 8 partial blocks in chunk
// order, t = bf16(((p0 + p1) + p2) + ... + p7).  The chunks depend on K only,
// so t does not depend on M, on the row block or on the launch.  A rank that is
// not a multiple of 16 reads the adapter rows past it as zeros: t columns
// [rank, ceil16(rank)) are written as zeros (t's row stride covers them).
//
// Fused form: every workgroup of a row block loads all of K for its 16 rows,
// so each takes the rows' maximum |x| (bit-pattern maximum, NaN propagated, as
// quant_rows_vec) from the vectors it loads for the products.  The rank blocks
// then split the codes: rank block b of R re-reads (from L2) the 16-byte
// vectors [V b / R, V (b + 1) / R) of each row (V = K / 8) and writes their
// codes, each wave two rows, with the arithmetic of quant_rows_vec; rank block
// 0 writes the scales and the padding rows.  Codes and scales are
// bit-identical to vflash_quantize_rows_e4m3.
#include "quant_ops.h"

#include <type_traits>

namespace vfa {

constexpr int LD_WAVES = 8;
constexpr int LD_ROWS = 16;   // rows of x per workgroup
constexpr int LD_RANKS = 16;  // adapter rows per workgroup
constexpr int LD_PREFETCH = 8;  // K steps whose loads are in flight together

template <bool QUANT>
__global__ void __launch_bounds__(64 * LD_WAVES) lora_down_blocks(
    const uint16_t* __restrict__ x, int64_t m, int64_t k, int64_t ldx,
    const uint16_t* __restrict__ a, int rank, uint16_t* __restrict__ t, int64_t ldt,
    uint8_t* __restrict__ codes, float* __restrict__ scales, int64_t m_pad) {
  __shared__ float part[LD_WAVES][4][64];
  __shared__ uint32_t row_max[LD_WAVES][LD_ROWS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * LD_ROWS;
  const int rb = (int)blockIdx.y;
  if (m0 >= m && !(QUANT && rb == 0)) return;  // padding rows only: rank block 0 writes them

  const int fr = lane & 15, fq = lane >> 4;
  const int64_t row = m0 + fr;
  const bool rok = row < m;
  // Lane (fr, fq) of K step s supplies elements 32 s + 8 fq .. +7 of x row
  // m0 + fr and of adapter row 16 rb + fr (the same K positions for both).
  const v4i* xr = reinterpret_cast<const v4i*>(x + (rok ? row : 0) * ldx);
  const bool aok = rb * LD_RANKS + fr < rank;  // adapter rows past the rank read as zero
  const v4i* ar = reinterpret_cast<const v4i*>(a + (int64_t)(aok ? rb * LD_RANKS + fr : 0) * k);
  const int64_t steps = (k + 31) / 32;
  const int64_t s0 = steps * wave / LD_WAVES, s1 = steps * (wave + 1) / LD_WAVES;

  v4f acc = v4f{};
  uint32_t amax_pk = 0u;  // two |bf16| patterns (abs_max_pk) of this lane's row
  for (int64_t c0 = s0; c0 < s1; c0 += LD_PREFETCH) {
    v4i xv[LD_PREFETCH], av[LD_PREFETCH];
#pragma unroll
    for (int i = 0; i < LD_PREFETCH; ++i) {
      const int64_t s = c0 + i;
      const bool ok = s < s1 && s * 32 + fq * 8 < k;
      xv[i] = (ok && rok) ? xr[s * 4 + fq] : v4i{};
      av[i] = (ok && aok) ? ar[s * 4 + fq] : v4i{};
    }
#pragma unroll
    for (int i = 0; i < LD_PREFETCH; ++i) {
      if (c0 + i < s1) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av[i]),
                                                      __builtin_bit_cast(v8bf, xv[i]), acc, 0,
                                                      0, 0);
        if constexpr (QUANT) {
#pragma unroll
          for (int j = 0; j < 4; ++j) amax_pk = abs_max_pk(amax_pk, (uint32_t)xv[i][j]);
        }
      }
    }
  }

  // Lane (fr, fq) holds t[m0 + fr, 16 rb + 4 fq + i] in acc[i].
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave][i][lane] = acc[i];
  if constexpr (QUANT) {
    // The four lanes of a row cover its K positions of this wave's chunk.
    uint32_t u = __float_as_uint(abs_max_value(amax_pk));
    u = max(u, (uint32_t)__shfl_xor((int)u, 16, 64));
    u = max(u, (uint32_t)__shfl_xor((int)u, 32, 64));
    if (fq == 0) row_max[wave][fr] = u;
  }
  __syncthreads();
  if (wave == 0 && rok) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = part[0][i][lane];
#pragma unroll
      for (int w = 1; w < LD_WAVES; ++w) v += part[w][i][lane];
      o[i] = f32_to_bf16(v);
    }
    *reinterpret_cast<uint2*>(t + row * ldt + rb * LD_RANKS + 4 * fq) =
        make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  }
  if constexpr (!QUANT) return;

  // Codes of rows m0 + 2 wave and m0 + 2 wave + 1, vectors [v0, v1) (rank block
  // 0 also: the scales, and zero codes and scale 1 for the GEMM padding rows
  // [m, m_pad)).
  const int64_t nvec = k >> 3;
  const int64_t v0 = nvec * rb / gridDim.y, v1 = nvec * (rb + 1) / gridDim.y;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int lr = wave * 2 + j;
    const int64_t grow = m0 + lr;
    if (grow >= m_pad) break;
    if (grow >= m) {
      if (rb == 0) pad_row(codes, scales, grow, k, lane);
      continue;
    }
    uint32_t u = row_max[0][lr];
#pragma unroll
    for (int w = 1; w < LD_WAVES; ++w) u = max(u, row_max[w][lr]);
    const float amax = __uint_as_float(u);
    const float scale = row_scale(amax);
    const RowDivisor d = row_divisor(scale, amax);
    const v4i* src = reinterpret_cast<const v4i*>(x + grow * ldx);
    uint2* dst = reinterpret_cast<uint2*>(codes + grow * k);
    auto codes_of = [&](auto fast) {
      // Four vectors per lane in flight.
      for (int64_t v = v0 + lane; v < v1; v += 256) {
        v4i in[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) in[i] = v + 64 * i < v1 ? src[v + 64 * i] : v4i{};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (v + 64 * i < v1) dst[v + 64 * i] = quant8<fast>(in[i], d);
      }
    };
    if (d.fast)
      codes_of(std::true_type{});
    else
      codes_of(std::false_type{});
    if (rb == 0 && lane == 0) scales[grow] = scale;
  }
}

// t is [m, ldt] with ldt >= ceil16(rank): every rank block writes its 16 columns.
hipError_t launch_lora_down(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                            const uint16_t* a, int rank, uint16_t* t, int64_t ldt,
                            hipStream_t s) {
  const int blocks = (rank + LD_RANKS - 1) / LD_RANKS;
  if (rank < 1 || ldt < (int64_t)blocks * LD_RANKS) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((m + LD_ROWS - 1) / LD_ROWS), (unsigned)blocks);
  lora_down_blocks<false><<<grid, 64 * LD_WAVES, 0, s>>>(x, m, k, ldx, a, rank, t, ldt, nullptr,
                                                         nullptr, m);
  return hipGetLastError();
}

hipError_t launch_quant_lora(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                             const uint16_t* a, int rank, uint16_t* t, int64_t ldt,
                             uint8_t* codes, float* scales, int64_t m_pad, hipStream_t s) {
  const int blocks = (rank + LD_RANKS - 1) / LD_RANKS;
  if (rank < 1 || ldt < (int64_t)blocks * LD_RANKS || m_pad < m) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((m_pad + LD_ROWS - 1) / LD_ROWS), (unsigned)blocks);
  lora_down_blocks<true><<<grid, 64 * LD_WAVES, 0, s>>>(x, m, k, ldx, a, rank, t, ldt, codes,
                                                        scales, m_pad);
  return hipGetLastError();
}

}  // namespace vfa
