// GELU-tanh of the FFN hidden rows fused with their per-token E4M3
// quantization, for gfx950.
//
// Replaces the activation between the FFN's two linears and the second
// linear's own activation quantization (the GELU-tanh form of
// src/vflash/native/h3_native_denoiser.py:369-382; quantization
// src/vflash/native/h3_fp8_activation.py:12-28):
//   g     = bf16(gelu_tanh(y))                    (per element)
//   amax  = max_k |g[row, k]|, NaN if any g is NaN
//   scale = amax > 0 ? max(amax / 448, FLT_MIN) : 1
//   code  = E4M3(clamp(g / scale, -448, 448))
//
// The input y is the bf16 output of the up projection, so GELU is a function of
// 16 bits: kGeluTanhTable (generated at build time, activation_tables.h) holds
// its value for every bf16 pattern, the real function rounded to binary32 and
// then to bf16.  Each workgroup copies the 128 KB table into LDS once and looks
// every element up with one LDS read; the kernel's work is then HBM-bound.
//
// Layout: one workgroup per CU (the table takes 128 KB of the 160 KB LDS), 12
// waves (three per SIMD), one row per wave at a time with the whole row in
// VGPRs (one HBM read per element); rows are dealt round-robin to the waves of
// the grid.  Row loads and stores go through buffer resources spanning exactly
// the row, so no lane needs a bounds branch and the loads issue back to back.
#include "_gen/activation_tables.h"
#include "quant_ops.h"

namespace vfa {

constexpr int GQ_WAVES = 12;
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// Byte offset of vector i (lanes 64 apart) of `bytes` bytes for this lane, as a
// lane base per group of 4096 bytes plus a constant below 4096 that the buffer
// instruction's immediate field carries (and its range check covers).
// The group base is made opaque so that the compiler cannot merge the two
// constants into one offset register per vector.
__device__ __forceinline__ uint32_t vec_off(int lane, int i, int bytes) {
  const int per_group = 4096 / (64 * bytes);
  uint32_t base = (uint32_t)lane * bytes + (uint32_t)(i / per_group) * 4096u;
  asm volatile("" : "+v"(base));
  return base + (uint32_t)(i % per_group) * 64u * bytes;
}

// y: bf16 [m, k] (row stride ldy); g (optional): bf16 [m, k] (row stride ldg);
// codes: [m_pad, k]; scales: [m_pad].  k % 8 == 0, k <= 512 * VPL.
template <int VPL>
__global__ void __launch_bounds__(64 * GQ_WAVES) gelu_quant_rows(
    const uint16_t* __restrict__ y, int64_t m, int64_t k, int64_t ldy, uint16_t* __restrict__ g,
    int64_t ldg, uint8_t* __restrict__ codes, float* __restrict__ scales, int64_t m_pad) {
  __shared__ __attribute__((aligned(16))) uint16_t table[65536];
  {
    const v4i* src = reinterpret_cast<const v4i*>(kGeluTanhTable);
    v4i* dst = reinterpret_cast<v4i*>(table);
#pragma unroll 4
    for (int i = threadIdx.x; i < 65536 / 8; i += 64 * GQ_WAVES) dst[i] = src[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  // The wave index as a scalar: rows, and the buffer resources built from them,
  // are then wave-uniform in the compiler's analysis.
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * GQ_WAVES;
  for (int64_t row = (int64_t)blockIdx.x * GQ_WAVES + wave; row < m_pad; row += stride) {
    if (row >= m) {
      pad_row(codes, scales, row, k, lane);
      continue;
    }
    // Branch-free row access: buffer resources over exactly this row, so lanes
    // past the end read zeros (T[0] = 0 leaves the maximum alone) and their
    // stores are dropped, and the loads issue back to back.
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + row * ldy, (uint32_t)(k * 2));
    v4i v[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(ry, vec_off(lane, i, 16), 0, 0);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t yw = (uint32_t)v[i][w];
        uint32_t gw = (uint32_t)table[yw & 0xffffu] | ((uint32_t)table[yw >> 16] << 16);
        // Only the packed pair stays live: left visible, the compiler keeps the
        // two looked-up halves apart for the later unpacking and runs out of
        // registers.
        asm volatile("" : "+v"(gw));
        v[i][w] = (int)gw;
      }
      amax = nan_max(amax, absmax8(v[i]));
      // At most two vectors' lookups (16 LDS reads) in flight: the compiler
      // would otherwise issue every lookup of the row first, holding one
      // register per half-word.
      if (i % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
    if (g) {
      const __amdgpu_buffer_rsrc_t rg = make_rsrc(g + row * ldg, (uint32_t)(k * 2));
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(v[i], rg, vec_off(lane, i, 16), 0, 0);
    }
    amax = wave_nan_max(amax);
    const float scale = row_scale(amax);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(codes + row * k, (uint32_t)k);
    const RowDivisor d = row_divisor(scale, amax);
    if (d.fast) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const uint2 c = quant8<true>(v[i], d);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, c), rc, vec_off(lane, i, 8), 0, 0);
        if (i % 2 == 1) __builtin_amdgcn_sched_barrier(0);  // bounded live temporaries
      }
    } else {
      // Rows with a NaN or infinite activation (or a scale out of the fast
      // range): the exact path, one vector at a time from a second read of y.
#pragma unroll 1
      for (int i = 0; i < VPL; ++i) {
        v4i yv = __builtin_amdgcn_raw_buffer_load_b128(ry, vec_off(lane, i, 16), 0, 0);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t yw = (uint32_t)yv[w];
          yv[w] = (int)((uint32_t)table[yw & 0xffffu] | ((uint32_t)table[yw >> 16] << 16));
        }
        const uint2 c = quant8<false>(yv, d);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, c), rc, vec_off(lane, i, 8), 0, 0);
      }
    }
    if (lane == 0) scales[row] = scale;
  }
}

int compute_units();

template <int VPL>
static void launch_gq(dim3 grid, hipStream_t s, const uint16_t* y, int64_t m, int64_t k,
                      int64_t ldy, uint16_t* g, int64_t ldg, uint8_t* codes, float* scales,
                      int64_t m_pad) {
  gelu_quant_rows<VPL><<<grid, dim3(64 * GQ_WAVES), 0, s>>>(y, m, k, ldy, g, ldg, codes, scales,
                                                            m_pad);
}

// Requires k % 8 == 0, 8 <= k <= 16384, ldy and ldg multiples of 8, y and g
// 16-byte aligned, codes 8-byte aligned (checked by the caller).
hipError_t launch_gelu_quant_rows(const uint16_t* y, int64_t m, int64_t k, int64_t ldy,
                                  uint16_t* g, int64_t ldg, uint8_t* codes, float* scales,
                                  int64_t m_pad, hipStream_t s) {
  const int64_t waves_needed = (m_pad + GQ_WAVES - 1) / GQ_WAVES;
  const int64_t cus = compute_units();
  const dim3 grid((unsigned)(waves_needed < cus ? waves_needed : cus));
  const int64_t nvec = k / 8;
  if (nvec <= 64) launch_gq<1>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 128) launch_gq<2>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 256) launch_gq<4>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 512) launch_gq<8>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 1024) launch_gq<16>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 1536) launch_gq<24>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else if (nvec <= 1792) launch_gq<28>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  else launch_gq<32>(grid, s, y, m, k, ldy, g, ldg, codes, scales, m_pad);
  return hipGetLastError();
}

}  // namespace vfa
