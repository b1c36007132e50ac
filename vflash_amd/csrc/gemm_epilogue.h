// Tile ordering and the two-phase epilogue shared by the GEMM kernels of this
// path (E4M3 W8A8 and E2M1-weight W4A8).  Kernel-side only; not part of the C-ABI.
#pragma once
#include "common.h"
#include "gemm_params.h"

namespace vfa {

// Logical tile index for this workgroup.  Workgroup b is dispatched to XCD
// b % 8; renumbering gives each XCD a contiguous run of logical tiles, and a
// grouped (GROUP_M tall) column sweep keeps the tiles that are resident on one
// XCD at the same time sharing A rows and W rows in that XCD's L2.
__device__ __forceinline__ void grouped_tile(int logical, int tiles_m, int tiles_n, int group_m,
                                             int& tm, int& tn) {
  const int per_group = group_m * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * group_m;
  const int gs = min(tiles_m - first_m, group_m);
  const int in_g = logical - group * per_group;
  tm = first_m + in_g % gs;
  tn = in_g / gs;
}

__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group_m, int& tm,
                                            int& tn) {
  const int nwg = gridDim.x;
  const int b = blockIdx.x;
  const int q = nwg >> 3, r = nwg & 7;
  const int x = b & 7, i = b >> 3;
  grouped_tile(x * q + min(x, r) + i, tiles_m, tiles_n, group_m, tm, tn);
}

// Epilogue shared by every tiling, in two phases through LDS.
//
// Phase 1 (per wave, from the accumulators): a lane holds, for 32x32 block
// (nb, mb) and register r, tile row mb*32 + (lane & 31) and tile column
// nb*32 + 8*(r/4) + 4*(lane/32) + r%4 of its wave's sub-tile.  It applies the
// scales, bias and the register-level epilogue (GELU, LoRA merge), rounds to
// bf16 and writes the values into a BM x BN bf16 staging tile in LDS (16-byte
// chunk c of row r stored in slot c ^ (r % chunks-per-row)).  Scale and bias
// vectors are loaded once, before any store.
// Phase 2 (whole workgroup): each thread moves 16-byte row chunks from LDS to
// global memory with coalesced 16-byte stores, applying the gate-residual
// epilogue there with coalesced residual loads.
template <int BM, int BN, int WGM, int WGN, int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p,
                                              v16f (&acc)[BN / WGN / 32][BM / WGM / 32],
                                              int64_t m0, int64_t n0, int wm, int wn, int tid,
                                              uint8_t* stage) {
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr int NT = 64 * WGM * WGN;
  constexpr int CH = BN / 8;  // 16-byte chunks per staged row
  constexpr int PITCH = BN * 2;
  const int lane = tid & 63, fr = lane & 31, fh = lane >> 5;
  const float* __restrict__ sa_p = p.sa;
  const float* __restrict__ sw_p = p.sw;
  const uint16_t* __restrict__ bias_p = p.bias;

  constexpr int NG = NB / 2 > 0 ? NB / 2 : 1;  // 64-column groups per wave (GELU maxima)
  float rmax[MB][NG];
  static_for<MB>([&](auto i) { static_for<NG>([&](auto j) { rmax[i][j] = 0.0f; }); });
  float sam[MB];
  static_for<MB>([&](auto mb) {
    const int64_t m = m0 + wm * WM + mb * 32 + fr;
    sam[mb] = m < p.m ? sa_p[m] : 0.0f;
  });

  // Column-block major: the scale and bias of one 32-column block (4 columns
  // per g for this lane) are live while its MB row blocks are written.  All
  // phase-1 stores go to LDS, so these global loads never wait on them.
  static_for<NB>([&](auto nb) {
    float sv[4][4], bv[4][4];
    static_for<4>([&](auto g) {
      const int64_t n = n0 + wn * WN + nb * 32 + g * 8 + fh * 4;
      const bool ok = n < p.n;
      static_for<4>([&](auto i) {
        sv[g][i] = ok ? sw_p[(n + i) * p.sw_step] : 0.0f;
        bv[g][i] = (ok && bias_p) ? bf16_to_f32(bias_p[n + i]) : 0.0f;
      });
    });
    static_for<MB>([&](auto mb) {
      const int row = wm * WM + mb * 32 + fr;  // tile row
      const int64_t m = m0 + row;
      const bool mvalid = m < p.m;
      v16f d = v16f{};
      if constexpr (EPI == EPI_LORA) {
        // delta block = B[n, :] . t[m, :] on bf16 MFMA, binary32 accumulate.
        const int64_t nrow = n0 + wn * WN + nb * 32 + fr;
        const bool nok = nrow < p.n;
        for (int r = 0; r < p.rank; r += 16) {
          v8s bfr = v8s{}, tfr = v8s{};
          if (nok) bfr = *reinterpret_cast<const v8s*>(p.lora_b + nrow * p.ldb + r + fh * 8);
          if (mvalid) tfr = *reinterpret_cast<const v8s*>(p.lora_t + m * p.ldt + r + fh * 8);
          d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bfr),
                                                      __builtin_bit_cast(v8bf, tfr), d, 0, 0,
                                                      0);
        }
      }
      static_for<4>([&](auto g) {
        uint32_t w[2];
        // Output pairs: every bf16 rounding is one v_cvt_pk_bf16_f32 for two values.
        static_for<2>([&](auto h) {
          constexpr int i0 = 2 * h, i1 = 2 * h + 1;
          uint32_t pw = pack_bf16x2(acc[nb][mb][g * 4 + i0] * sam[mb] * sv[g][i0],
                                    acc[nb][mb][g * 4 + i1] * sam[mb] * sv[g][i1]);
          if (bias_p) pw = pack_bf16x2(bf16_lo(pw) + bv[g][i0], bf16_hi(pw) + bv[g][i1]);
          if constexpr (EPI == EPI_GELU) {
            pw = pack_bf16x2(gelu_tanh(bf16_lo(pw)), gelu_tanh(bf16_hi(pw)));
            rmax[mb][nb / 2] =
                fmaxf(rmax[mb][nb / 2], fmaxf(fabsf(bf16_lo(pw)), fabsf(bf16_hi(pw))));
          } else if constexpr (EPI == EPI_LORA) {
            uint32_t dp = pack_bf16x2(d[g * 4 + i0], d[g * 4 + i1]);
            if (p.lora_scale != 1.0f)
              dp = pack_bf16x2(bf16_lo(dp) * p.lora_scale, bf16_hi(dp) * p.lora_scale);
            if (p.lora_strength != 1.0f)
              dp = pack_bf16x2(bf16_lo(dp) * p.lora_strength, bf16_hi(dp) * p.lora_strength);
            pw = pack_bf16x2(bf16_lo(pw) + bf16_lo(dp), bf16_hi(pw) + bf16_hi(dp));
          }
          w[h] = pw;
        });
        const int c = (wn * WN + nb * 32 + g * 8) / 8;  // 16-byte chunk of the row
        *reinterpret_cast<uint2*>(stage + row * PITCH + ((c ^ (row % CH)) << 4) + fh * 8) =
            make_uint2(w[0], w[1]);
      });
    });
  });

  if constexpr (EPI == EPI_GELU) {
    static_assert(NB % 2 == 0, "GELU epilogue needs 64-column wave groups");
    // Lanes l and l + 32 hold the same row; each pair of 32-column blocks is
    // one 64-column group.  One partial maximum per (row, group).
    const int parts = (int)((p.n + 63) / 64);
    static_for<MB>([&](auto mb) {
      const int64_t m = m0 + wm * WM + mb * 32 + fr;
      static_for<NB / 2>([&](auto gi) {
        const float v = fmaxf(rmax[mb][gi], __shfl_xor(rmax[mb][gi], 32, 64));
        const int64_t col = n0 + wn * WN + gi * 64;
        if (fh == 0 && m < p.m && col < p.n) p.amax_part[m * parts + col / 64] = v;
      });
    });
  }
  __syncthreads();

  // Phase 2: LDS rows -> global, 16 bytes per thread per step.
  const bool vec_out = ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) && (p.ldo % 8 == 0) &&
                       (p.plane_cols == 0 || p.plane_stride % 8 == 0);
  for (int q = tid; q < BM * CH; q += NT) {
    const int row = q / CH, c = q % CH;
    const int64_t m = m0 + row, n = n0 + c * 8;
    if (m >= p.m || n >= p.n) continue;
    v4i v = *reinterpret_cast<const v4i*>(stage + row * PITCH + ((c ^ (row % CH)) << 4));
    if constexpr (EPI == EPI_GATE) {
      const uint16_t* res = p.residual + m * p.ldr + n;
      const uint16_t* gt = p.gate + m * p.gate_ts + n * p.gate_hs;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t y = (uint32_t)v[j];
        const uint32_t gy = pack_bf16x2(bf16_to_f32(gt[(2 * j) * p.gate_hs]) * bf16_lo(y),
                                        bf16_to_f32(gt[(2 * j + 1) * p.gate_hs]) * bf16_hi(y));
        v[j] = (int)pack_bf16x2(bf16_to_f32(res[2 * j]) + bf16_lo(gy),
                                bf16_to_f32(res[2 * j + 1]) + bf16_hi(gy));
      }
    }
    uint16_t* dst;
    if (p.plane_cols > 0) {
      const int64_t plane = n / p.plane_cols;
      dst = p.out + plane * p.plane_stride + m * p.ldo + (n - plane * p.plane_cols);
    } else {
      dst = p.out + m * p.ldo + n;
    }
    if (vec_out) {
      *reinterpret_cast<v4i*>(dst) = v;
    } else {
      reinterpret_cast<uint2*>(dst)[0] = make_uint2((uint32_t)v[0], (uint32_t)v[1]);
      reinterpret_cast<uint2*>(dst)[1] = make_uint2((uint32_t)v[2], (uint32_t)v[3]);
    }
  }
}

}  // namespace vfa
