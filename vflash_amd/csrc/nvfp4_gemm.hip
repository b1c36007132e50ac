// NVFP4-weight linear (W4A8) for gfx950.
//
//   acc[m, n] = sum_k e4m3(a[m, k]) * e2m1(w[n, k]) * e4m3(s[n, k / 16])
//   out       = bf16(bf16(acc * sa[m] * alpha) + bias[n])
//
// Replaces mm_fp4 in NVFP4Execution.linear (reference
// src/vflash/native/h3_nvfp4_linear.py:118-139); the activation side is the
// per-token E4M3 code of the W8A8 path instead of an NVFP4 activation.
//
// Every product e2m1 * e4m3 has at most 6 significant bits, so it is exact in
// bfloat16, and every E4M3 code is exact in bfloat16: the contraction runs on
// v_mfma_f32_32x32x16_bf16 with no rounding before the binary32 accumulator.
// Weights stay packed (0.5 byte/element) in HBM and are dequantized while
// being staged into LDS, once per workgroup tile, so the four waves read ready
// bf16 fragments.  Scales use the 128x4 tiled order of NVFP4Weight
// (h3_nvfp4_linear.py:22-33): for row n and K block j (16 elements),
//   off = (n/128)*(K/64)*512 + (j/4)*512 + (n%32)*16 + ((n%128)/32)*4 + j%4.
#include "common.h"

namespace vfa {

struct Fp4Params {
  const uint8_t* a;
  const float* sa;
  int64_t lda;
  const uint8_t* w;   // [n, k/2]
  const uint8_t* ws;  // 128x4 tiled e4m3 block scales
  const float* alpha; // device scalar output multiplier
  int64_t m, n, k;
  const uint16_t* bias;
  uint16_t* out;
  int64_t ldo;
  int group_m;
};

__device__ __forceinline__ int64_t scale_offset(int64_t n, int64_t j, int64_t k_tiles) {
  return (n >> 7) * k_tiles * 512 + (j >> 2) * 512 + (n & 31) * 16 + ((n & 127) >> 5) * 4 + (j & 3);
}

// Two binary32 values that are exact in bf16 -> one packed bf16 pair.
__device__ __forceinline__ uint32_t pack_exact_bf16(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

__device__ __forceinline__ void tile_coords_fp4(int tiles_m, int tiles_n, int group_m, int& tm,
                                                int& tn) {
  const int nwg = gridDim.x;
  const int b = blockIdx.x;
  const int q = nwg >> 3, r = nwg & 7;
  const int x = b & 7, i = b >> 3;
  const int logical = x * q + min(x, r) + i;
  const int per_group = group_m * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * group_m;
  const int gs = min(tiles_m - first_m, group_m);
  const int in_g = logical - group * per_group;
  tm = first_m + in_g % gs;
  tn = in_g / gs;
}

template <int BM, int BN>
__global__ void __launch_bounds__(256) nvfp4_gemm_kernel(const Fp4Params p) {
  constexpr int BK = 64;              // K elements per stage; 128 bytes of bf16 per LDS row
  constexpr int WM = BM / 2, WN = BN / 2, MB = WM / 32, NB = WN / 32;
  constexpr int ROWB = BK * 2;        // LDS row bytes
  constexpr int STAGE = (BM + BN) * ROWB;
  constexpr int ACH = BM * 4 / 256;   // 16-byte code chunks (16 codes) per thread
  constexpr int WCH = BN * 2 / 256;   // 16-byte packed chunks (32 values) per thread
  static_assert(ACH >= 1 && WCH >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tiles_m = (int)((p.m + BM - 1) / BM), tiles_n = (int)((p.n + BN - 1) / BN);
  int tm, tn;
  tile_coords_fp4(tiles_m, tiles_n, p.group_m, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  const int64_t rows_a = min((int64_t)BM, p.m - m0);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
  const int64_t ldw = p.k / 2;
  const int64_t k_tiles = p.k / 64;

  // A: chunk (row, c4) with c4 in 0..3 covering 16 codes each of the 64-element slice.
  const int ac = tid & 3, ar0 = tid >> 2;  // rows ar0 + 64 i
  // W: chunk (row, c2) with c2 in 0..1 covering 32 values each.
  const int wc = tid & 1, wr0 = tid >> 1;  // rows wr0 + 128 i

  v4i va[ACH], vw[WCH];
  uint32_t vs[WCH];
  auto gload = [&](int kt) {
    const uint32_t kb = (uint32_t)kt * BK;
#pragma unroll
    for (int i = 0; i < ACH; ++i)
      va[i] = __builtin_amdgcn_raw_buffer_load_b128(
          ra, (uint32_t)((ar0 + 64 * i) * p.lda) + kb + ac * 16, 0, 0);
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int64_t n = n0 + wr0 + 128 * i;
      if (n < p.n) {
        vw[i] = *reinterpret_cast<const v4i*>(p.w + n * ldw + (kb >> 1) + wc * 16);
        const int64_t j = (int64_t)kt * 4 + wc * 2;  // first of two K blocks
        vs[i] = *reinterpret_cast<const uint16_t*>(p.ws + scale_offset(n, j, k_tiles));
      } else {
        vw[i] = v4i{};
        vs[i] = 0;
      }
    }
  };
  // LDS rows hold 64 bf16 = 8 chunks of 16 bytes, slots swizzled by lds_swizzle(row).
  auto sstore = [&](int buf) {
    uint8_t* sa = smem + buf * STAGE;
    uint8_t* sw = sa + BM * ROWB;
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int row = ar0 + 64 * i;
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wd = (uint32_t)va[i][j];
        h[2 * j] = pack_exact_bf16(e4m3_to_f32(wd & 0xff), e4m3_to_f32((wd >> 8) & 0xff));
        h[2 * j + 1] = pack_exact_bf16(e4m3_to_f32((wd >> 16) & 0xff), e4m3_to_f32(wd >> 24));
      }
      const int c0 = ac * 2;  // two 16-byte chunks: 16 codes -> 16 bf16
      *reinterpret_cast<v4i*>(sa + row * ROWB + ((c0 ^ lds_swizzle(row)) << 4)) =
          v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
      *reinterpret_cast<v4i*>(sa + row * ROWB + (((c0 + 1) ^ lds_swizzle(row)) << 4)) =
          v4i{(int)h[4], (int)h[5], (int)h[6], (int)h[7]};
    }
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int row = wr0 + 128 * i;
#pragma unroll
      for (int half = 0; half < 2; ++half) {  // each half = one 16-element K block
        const float s = e4m3_to_f32((vs[i] >> (8 * half)) & 0xff);
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t wd = (uint32_t)vw[i][half * 2 + j];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t byte = (wd >> (8 * b)) & 0xff;
            h[j * 4 + b] = pack_exact_bf16(e2m1_to_f32(byte & 0xf) * s, e2m1_to_f32(byte >> 4) * s);
          }
        }
        const int c0 = wc * 4 + half * 2;
        *reinterpret_cast<v4i*>(sw + row * ROWB + ((c0 ^ lds_swizzle(row)) << 4)) =
            v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
        *reinterpret_cast<v4i*>(sw + row * ROWB + (((c0 + 1) ^ lds_swizzle(row)) << 4)) =
            v4i{(int)h[4], (int)h[5], (int)h[6], (int)h[7]};
      }
    }
  };

  v16f acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = v16f{};

  const int fr = lane & 31, fh = lane >> 5, sw7 = lds_swizzle(fr);
  auto compute = [&](int buf) {
    const uint8_t* sa = smem + buf * STAGE + (wm * WM + fr) * ROWB;
    const uint8_t* sw = smem + buf * STAGE + BM * ROWB + (wn * WN + fr) * ROWB;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {  // 16 K elements per MFMA
      const int o = ((ks * 2 + fh) ^ sw7) << 4;
      v8bf xf[MB], wf[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xf[mb] = *reinterpret_cast<const v8bf*>(sa + mb * 32 * ROWB + o);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        wf[nb] = *reinterpret_cast<const v8bf*>(sw + nb * 32 * ROWB + o);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[nb], xf[mb], acc[nb][mb], 0, 0, 0);
    }
  };

  const int KT = (int)(p.k / BK);
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    compute(kt & 1);
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

  const float alpha = *p.alpha;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t m = m0 + wm * WM + mb * 32 + fr;
    if (m >= p.m) continue;
    const float sam = p.sa[m] * alpha;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = n0 + wn * WN + nb * 32 + g * 8 + fh * 4;
        if (n >= p.n) continue;
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float y = round_bf16(acc[nb][mb][g * 4 + i] * sam);
          if (p.bias) y = round_bf16(y + bf16_to_f32(p.bias[n + i]));
          o[i] = f32_to_bf16(y);
        }
        *reinterpret_cast<uint2*>(p.out + m * p.ldo + n) =
            make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
      }
    }
  }
}

hipError_t launch_nvfp4_gemm(const Fp4Params& p, int tile, hipStream_t s) {
  auto go = [&](auto bm, auto bn) {
    constexpr int BM = decltype(bm)::value, BN = decltype(bn)::value;
    const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
    nvfp4_gemm_kernel<BM, BN><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(p);
    return hipGetLastError();
  };
  using I64 = std::integral_constant<int, 64>;
  using I128 = std::integral_constant<int, 128>;
  using I256 = std::integral_constant<int, 256>;
  if (tile == 0) {
    const int64_t big = ((p.m + 255) / 256) * ((p.n + 255) / 256);
    const int64_t mid = ((p.m + 127) / 128) * ((p.n + 127) / 128);
    tile = big >= 512 ? 1 : (mid >= 256 ? 2 : 3);
  }
  switch (tile) {
    case 1: return go(I256{}, I256{});
    case 2: return go(I128{}, I128{});
    case 3: return go(I64{}, I128{});
    default: return go(I128{}, I128{});
  }
}

hipError_t launch_nvfp4(const uint8_t* a, const float* sa, int64_t lda, const uint8_t* w,
                        const uint8_t* ws, const float* alpha, int64_t m, int64_t n, int64_t k,
                        const uint16_t* bias, uint16_t* out, int64_t ldo, int tile, int group_m,
                        hipStream_t s) {
  Fp4Params p{a, sa, lda, w, ws, alpha, m, n, k, bias, out, ldo, group_m};
  return launch_nvfp4_gemm(p, tile, s);
}

}  // namespace vfa
