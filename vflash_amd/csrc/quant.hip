// Per-token (per-row) E4M3 activation quantization for gfx950.
//
// Arithmetic (reference: src/vflash/native/h3_fp8_activation.py:12-28 and its
// portable twin src/vflash/native/h3_fp8_linear.py:18-31):
//   amax  = max_k |x[row, k]|, NaN if any x is NaN  (binary32, torch's amax)
//   scale = amax > 0 ? max(amax / 448, FLT_MIN) : 1 (IEEE division)
//   code  = E4M3(clamp(x / scale, -448, 448))       (IEEE division, RNE)
// Rows in [m, m_pad) are the GEMM padding rows: codes 0, scale 1.
//
// Layout: one 64-lane wave owns one row; a 256-thread workgroup owns 4 rows.
// The aligned kernel keeps the whole row in VGPRs (16-byte loads, one HBM
// read per element), reduces the maximum across the wave with XOR shuffles and
// writes 8 codes per 16-byte input vector.
#include "quant_ops.h"

namespace vfa {

// Aligned path: k % 8 == 0, ldx % 8 == 0, x 16-byte aligned, k <= 512 * VPL.
template <int VPL>
__global__ void __launch_bounds__(256) quant_rows_vec(const uint16_t* __restrict__ x,
                                                      int64_t m, int64_t k, int64_t ldx,
                                                      uint8_t* __restrict__ codes,
                                                      float* __restrict__ scales,
                                                      int64_t m_pad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m_pad) return;
  if (row >= m) {
    pad_row(codes, scales, row, k, lane);
    return;
  }
  // Widen the row index before the multiply: row * ldx may exceed 2^31.
  const v4i* xr = reinterpret_cast<const v4i*>(x + row * ldx);
  const int nvec = (int)(k >> 3);
  v4i v[VPL];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    int j = lane + 64 * i;
    if (j < nvec) {
      v[i] = __builtin_nontemporal_load(xr + j);
      amax = nan_max(amax, absmax8(v[i]));
    }
  }
  amax = wave_nan_max(amax);
  const float scale = row_scale(amax);
  quant_row_regs<VPL>(reinterpret_cast<uint2*>(codes + row * k), v, lane, nvec, scale, amax);
  if (lane == 0) scales[row] = scale;
}

// Any k, any row stride: two passes over the row with scalar bf16 loads.
__global__ void __launch_bounds__(256) quant_rows_generic(const uint16_t* __restrict__ x,
                                                          int64_t m, int64_t k, int64_t ldx,
                                                          uint8_t* __restrict__ codes,
                                                          float* __restrict__ scales,
                                                          int64_t m_pad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m_pad) return;
  if (row >= m) {
    pad_row(codes, scales, row, k, lane);
    return;
  }
  const uint16_t* xr = x + row * ldx;
  float amax = 0.0f;
  for (int64_t j = lane; j < k; j += 64) amax = nan_max(amax, bf16_to_f32(xr[j] & 0x7fffu));
  amax = wave_nan_max(amax);
  const float scale = row_scale(amax);
  uint8_t* cr = codes + row * k;
  for (int64_t j = lane; j < k; j += 64) cr[j] = (uint8_t)quant1(bf16_to_f32(xr[j]), scale);
  if (lane == 0) scales[row] = scale;
}

// Requantization of a GEMM output whose epilogue already reduced |g| per row
// over each of its `parts` column tiles (amax_part[row * parts + p]).  The
// arithmetic is exactly quant_rows_*: the maximum of the partial maxima is the
// row maximum.  Streaming: no row is held in registers.
__global__ void __launch_bounds__(256) requant_rows(const uint16_t* __restrict__ g, int64_t m,
                                                    int64_t k, int64_t ldg,
                                                    const float* __restrict__ amax_part,
                                                    int parts, uint8_t* __restrict__ codes,
                                                    float* __restrict__ scales, int64_t m_pad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m_pad) return;
  if (row >= m) {
    pad_row(codes, scales, row, k, lane);
    return;
  }
  float amax = 0.0f;
  for (int p = lane; p < parts; p += 64) amax = nan_max(amax, amax_part[row * parts + p]);
  amax = wave_nan_max(amax);
  const float scale = row_scale(amax);
  const v4i* gr = reinterpret_cast<const v4i*>(g + row * ldg);
  uint2* cr = reinterpret_cast<uint2*>(codes + row * k);
  const int nvec = (int)(k >> 3);
  const RowDivisor d = row_divisor(scale, amax);
  if (d.fast) {
    for (int j = lane; j < nvec; j += 64) cr[j] = quant8<true>(__builtin_nontemporal_load(gr + j), d);
  } else {
    for (int j = lane; j < nvec; j += 64) cr[j] = quant8<false>(__builtin_nontemporal_load(gr + j), d);
  }
  if (lane == 0) scales[row] = scale;
}

}  // namespace vfa

// ---------------------------------------------------------------------------
// Host launchers (called from capi.hip)
// ---------------------------------------------------------------------------
namespace vfa {

hipError_t launch_quant_rows(const uint16_t* x, int64_t m, int64_t k, int64_t ldx,
                             uint8_t* codes, float* scales, int64_t m_pad, hipStream_t s) {
  const dim3 block(256), grid((unsigned)((m_pad + 3) / 4));
  const bool aligned = (k % 8 == 0) && (ldx % 8 == 0) &&
                       ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                       ((reinterpret_cast<uintptr_t>(codes) & 7) == 0);
  const int64_t nvec = k / 8;
  if (aligned && nvec <= 64 * 32) {
    if (nvec <= 64) quant_rows_vec<1><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
    else if (nvec <= 128) quant_rows_vec<2><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
    else if (nvec <= 256) quant_rows_vec<4><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
    else if (nvec <= 512) quant_rows_vec<8><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
    else if (nvec <= 1024) quant_rows_vec<16><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
    else quant_rows_vec<32><<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
  } else {
    quant_rows_generic<<<grid, block, 0, s>>>(x, m, k, ldx, codes, scales, m_pad);
  }
  return hipGetLastError();
}

hipError_t launch_requant_rows(const uint16_t* g, int64_t m, int64_t k, int64_t ldg,
                               const float* amax_part, int parts, uint8_t* codes,
                               float* scales, int64_t m_pad, hipStream_t s) {
  const dim3 block(256), grid((unsigned)((m_pad + 3) / 4));
  requant_rows<<<grid, block, 0, s>>>(g, m, k, ldg, amax_part, parts, codes, scales, m_pad);
  return hipGetLastError();
}

}  // namespace vfa
