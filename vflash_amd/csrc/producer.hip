// The producer of a linear's input, fused with that linear's activation
// quantization: RMSNorm, adaLN modulation and per-token E4M3 quantization in
// one pass over the activation.
//
// Arithmetic, per row r of x [m, k] (bf16), in binary32 with the eager bf16
// rounding boundaries of the reference:
//   rstd  = 1 / sqrt(sum_k x^2 / k + eps)
//   n     = bf16(x * rstd * w)                 torch.nn.functional.rms_norm
//                                              (src/vflash/native/h3_native_denoiser.py:231-243)
//   y     = bf16(bf16(n * bf16(1 + scale)) + shift)
//                                              (h3_native_denoiser.py:363-364,
//                                               src/vflash/native/h3_fused_ops.py:52-122)
//   codes, row scale = the per-token E4M3 quantization of y
//                                              (src/vflash/native/h3_fp8_activation.py:12-28)
// The modulation row of x's row r is t = r % tokens (the [S, H] scale/shift
// broadcast over the batch), or index[t] when an index is given: the gather
// table[:, j, :].index_select(0, adaln_indices) of h3_native_denoiser.py:527-532
// read in place from the table, with no gathered copy.
//
// Layout: one 64-lane wave owns one row (the whole row in VGPRs: one HBM read of
// x), a 256-thread workgroup owns 4 rows.  The norm weight and the modulation
// rows are shared by many rows and stay in L2.
#include "gemm_params.h"
#include "quant_ops.h"

namespace vfa {

// Norm and modulation of the two bf16 of one 32-bit word (low element first);
// returns y as a packed bf16 pair.  A bf16 rounding whose result is used again
// is one conversion that leaves bf16(v) widened in the register
// (round_bf16_wide); the last one packs the pair.
template <bool HAS_W>
__device__ __forceinline__ uint32_t modulate2(float xl, float xh, uint32_t wv, uint32_t sv,
                                              uint32_t hv, float rstd) {
  float nl = xl * rstd, nh = xh * rstd;
  if constexpr (HAS_W) {
    nl *= bf16_lo(wv);
    nh *= bf16_hi(wv);
  }
  const float al = round_bf16_wide(round_bf16_wide(nl) * round_bf16_wide(1.0f + bf16_lo(sv)));
  const float ah = round_bf16_wide(round_bf16_wide(nh) * round_bf16_wide(1.0f + bf16_hi(sv)));
  return pack_bf16x2(al + bf16_lo(hv), ah + bf16_hi(hv));
}

// k % 8 == 0; x, norm_w, scale, shift, values 16-byte aligned with row strides
// that are multiples of 8 elements; k <= 512 * VPL.  The unrolled loops read
// vector min(j, nvec - 1) so that no load sits behind a branch (the compiler
// can then issue every load of a row early); only the stores are guarded.
template <int VPL, bool HAS_W>
__global__ void __launch_bounds__(256) norm_mod_quant_rows(NormModParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.m_pad) return;
  const int nvec = (int)(p.k >> 3);
  uint2* cr = reinterpret_cast<uint2*>(p.codes + row * p.k);
  if (row >= p.m) {
    for (int j = lane; j < nvec; j += 64) cr[j] = make_uint2(0u, 0u);
    if (lane == 0) p.scales[row] = 1.0f;
    return;
  }
  const int64_t token = row % p.tokens;
  int64_t mrow = token;
  if (p.index) {
    mrow = p.index[token];
    if ((uint64_t)mrow >= (uint64_t)p.mod_rows) {
      // An index outside the table: the row's codes are 0 and its scale NaN,
      // so every output of the consuming linear for this row is NaN.
      for (int j = lane; j < nvec; j += 64) cr[j] = make_uint2(0u, 0u);
      if (lane == 0) p.scales[row] = __builtin_nanf("");
      return;
    }
  }
  const v4i* xr = reinterpret_cast<const v4i*>(p.x + row * p.ldx);
  const v4i* sr = reinterpret_cast<const v4i*>(p.scale + mrow * p.ld_scale);
  const v4i* hr = reinterpret_cast<const v4i*>(p.shift + mrow * p.ld_shift);
  const v4i* wr = reinterpret_cast<const v4i*>(p.norm_w);
  // x is widened to binary32 once (the second pass reuses it); v[] later holds y.
  v4i v[VPL];
  float xf[VPL][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    const v4i xv = __builtin_nontemporal_load(xr + (j < nvec ? j : nvec - 1));
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xf[i][2 * e] = bf16_lo((uint32_t)xv[e]);
      xf[i][2 * e + 1] = bf16_hi((uint32_t)xv[e]);
      part += xf[i][2 * e] * xf[i][2 * e];  // exact squares (16 significant bits)
      part += xf[i][2 * e + 1] * xf[i][2 * e + 1];
    }
    ss += j < nvec ? part : 0.0f;
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)p.k + p.eps);

  uint32_t amax_pk = 0u;  // |y| maxima of the two halves, NaN propagated
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    const int jj = j < nvec ? j : nvec - 1;
    const v4i s = sr[jj], h = hr[jj];
    v4i w = s;
    if constexpr (HAS_W) w = wr[jj];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t y = modulate2<HAS_W>(xf[i][2 * e], xf[i][2 * e + 1], (uint32_t)w[e],
                                          (uint32_t)s[e], (uint32_t)h[e], rstd);
      amax_pk = abs_max_pk(amax_pk, y);
      v[i][e] = (int)y;
    }
  }
  const float amax = wave_nan_max(abs_max_value(amax_pk));
  const float scale = row_scale(amax);
  if (p.values) {
    v4i* vr = reinterpret_cast<v4i*>(p.values + row * p.ldv);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < nvec) vr[j] = v[i];
    }
  }
  quant_row_regs<VPL>(cr, v, lane, nvec, scale, amax);
  if (lane == 0) p.scales[row] = scale;
}

template <int VPL>
void launch_vpl(const NormModParams& p, dim3 grid, hipStream_t s) {
  if (p.norm_w) norm_mod_quant_rows<VPL, true><<<grid, 256, 0, s>>>(p);
  else norm_mod_quant_rows<VPL, false><<<grid, 256, 0, s>>>(p);
}

hipError_t launch_norm_mod_quant(const NormModParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.m_pad + 3) / 4));
  const int64_t nvec = p.k / 8;
  if (nvec <= 64) launch_vpl<1>(p, grid, s);
  else if (nvec <= 128) launch_vpl<2>(p, grid, s);
  else if (nvec <= 256) launch_vpl<4>(p, grid, s);
  else if (nvec <= 512) launch_vpl<8>(p, grid, s);
  else if (nvec <= 640) launch_vpl<10>(p, grid, s);
  else if (nvec <= 768) launch_vpl<12>(p, grid, s);
  else if (nvec <= 1024) launch_vpl<16>(p, grid, s);
  else launch_vpl<32>(p, grid, s);
  return hipGetLastError();
}

}  // namespace vfa
