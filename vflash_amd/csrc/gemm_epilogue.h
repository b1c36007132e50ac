// Tile ordering and the two-phase epilogue shared by the GEMM kernels of this
// path (E4M3 W8A8 and E2M1-weight W4A8).  Kernel-side only; not part of the C-ABI.
#pragma once
#include "_gen/silu_table.h"
#include "common.h"
#include "gemm_params.h"

#include <type_traits>

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

// Adapter operands of the LoRA epilogues.  A rank step covers 16 rank
// positions; lane half fh supplies positions 16 st + 8 fh .. +7 of its row.
// Positions at or past the rank read as zero, so a rank that is not a multiple
// of 16 needs no padding of t or B.  A row is read only below the rank rounded
// up to 8, which the row strides (ldt, ldb >= that, multiples of 8) contain.
__device__ __forceinline__ v8s lora_frag(const uint16_t* row, int rank, int st, int fh, bool ok) {
  const int e0 = st * 16 + fh * 8;
  v8s v = (ok && e0 < rank) ? *reinterpret_cast<const v8s*>(row + e0) : v8s{};
  if (rank & 7) {  // uniform: only ranks that end inside an 8-element vector
    const int valid = rank - e0;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e >= valid) v[e] = 0;
  }
  return v;
}

// Global column (row of the adapter's B) of tile column c.  SwiGLU tiles hold
// value columns n0 .. in [0, BN/2) and the matching gate columns half_n + n0 ..
// in [BN/2, BN), as the GEMM tile maps them.
template <int BN, bool SWIGLU>
__device__ __forceinline__ int64_t tile_column(const GemmParams& p, int64_t n0, int c) {
  if constexpr (SWIGLU) return c < BN / 2 ? n0 + c : p.half_n + n0 + c - BN / 2;
  return n0 + c;
}

// The adapter branch of a wave's columns, from its first column `col`: the
// offset of its t columns and its scale.  A wave's columns lie in one branch
// (the launcher picks a tiling whose wave width divides lora_branch_cols).
struct LoraBranch {
  int64_t toff;
  float scale;
};
__device__ __forceinline__ LoraBranch lora_branch(const GemmParams& p, int64_t col) {
  // At most three branches: two comparisons instead of a 64-bit division.
  const int64_t bc = p.lora_branch_cols;
  const int b = bc > 0 && col < p.n ? (int)(col >= bc) + (int)(col >= 2 * bc) : 0;
  // The three scales pass through readfirstlane before the choice: a choice
  // between plain loads of them would be folded into one indexed load of the
  // kernel's parameter block, which then gets copied to private memory.
  auto arg = [](float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); };
  const float s0 = arg(p.lora_scale[0]), s1 = arg(p.lora_scale[1]), s2 = arg(p.lora_scale[2]);
  const float s = b == 0 ? s0 : (b == 1 ? s1 : s2);
  return LoraBranch{b * p.lora_t_branch, s};
}

// LoRA products of one wave's blocks, d[nb * MB + mb] = B[n, :] . t[m, :]
// (bf16 MFMA, binary32 accumulation), with all loads issued before the MFMAs.
// Computed ahead of the main loop so the epilogue does not wait on them.
template <int BM, int BN, int WGM, int WGN, bool SWIGLU = false>
__device__ __forceinline__ void lora_blocks(const GemmParams& p, int64_t m0, int64_t n0, int wm,
                                            int wn, int lane, v16f* d) {
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr int RS = 8;  // rank steps of 16: rank <= 128
  const int fr = lane & 31, fh = lane >> 5;
  const LoraBranch br = lora_branch(p, tile_column<BN, SWIGLU>(p, n0, wn * WN));
  v8s bf[NB][RS], tf[MB][RS];
  static_for<NB>([&](auto nb) {
    const int64_t nrow = tile_column<BN, SWIGLU>(p, n0, wn * WN + nb * 32) + fr;
    static_for<RS>([&](auto r) {
      bf[nb][r] = lora_frag(p.lora_b + nrow * p.ldb, p.rank, r, fh, nrow < p.n);
    });
  });
  static_for<MB>([&](auto mb) {
    const int64_t m = m0 + wm * WM + mb * 32 + fr;
    static_for<RS>([&](auto r) {
      tf[mb][r] = lora_frag(p.lora_t + m * p.ldt + br.toff, p.rank, r, fh, m < p.m);
    });
  });
  static_for<NB>([&](auto nb) {
    static_for<MB>([&](auto mb) {
      v16f acc = v16f{};
      static_for<RS>([&](auto r) {
        if (r * 16 < p.rank)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bf[nb][r]),
                                                        __builtin_bit_cast(v8bf, tf[mb][r]), acc,
                                                        0, 0, 0);
      });
      d[nb * MB + mb] = acc;
    });
  });
}

// LDS bytes of the staged tile vectors: weight scales (or the one scalar),
// activation row scales, bias.
constexpr int VEC_LDS = 3 * 1024;
// LDS bytes of the silu window table, which SwiGLU tiles stage after the vectors.
constexpr int SILU_LDS = 2 * (int)kSiluN * 4;

// bf16(silu(g)) as a binary32 value, for the bf16 pattern `bits` (low 16 bits)
// of g: looked up in the window table `tab` (LDS) for 2^-9 <= |g| < 2^7, else
// bf16(g / 2) below the window, g above it for g > 0 and g * 0 for g < 0 (-0,
// or NaN for -inf and NaN).  Every bf16 input gives the binary32 formula
// g / (1 + exp(-g)) of h3_fused_ops.py:205 with each step correctly rounded,
// then rounded to bf16 (the window table is generated to that definition).
__device__ __forceinline__ float silu_lookup(uint32_t bits, float g, const float* tab) {
  const uint32_t a = bits & 0x7fffu;
  const uint32_t i = a - kSiluLo;  // wraps around below the window
  const uint32_t idx = min(i, kSiluN - 1u) | ((bits >> 4) & kSiluN);
  const float t = tab[idx];
  const float factor = a < kSiluLo ? 0.5f : ((bits & 0x8000u) ? 0.0f : 1.0f);
  const float outside = g * factor;
  // One rounding for both cases (table values are bf16 already), so that the
  // choice stays a select rather than a branch around the conversion.
  return round_bf16_wide(i < kSiluN ? t : outside);
}

// Copy the scale and bias vectors of a BM x BN tile into LDS (vec_lds) with
// buffer-load-to-LDS DMA, one instruction each on waves 0, 1 and 2.  Issued
// with the tile's first K stage, so the caller's first DMA wait and barrier
// also cover these; entries past the matrix edge read as zero.
// SWIGLU: tile columns [0, BN/2) are value columns n0.. and [BN/2, BN) the
// matching gate columns half_n + n0.. (as the GEMM tile maps them).
template <int BM, int BN, bool SWIGLU = false>
__device__ __forceinline__ void stage_vectors(const GemmParams& p, int64_t m0, int64_t n0,
                                              int wave, int lane, uint32_t vec_lds) {
  static_assert(BM * 4 <= 1024 && BN * 4 <= 1024, "vector slots hold 256 entries");
  if constexpr (SWIGLU) {
    static_assert(BN == 256, "SwiGLU tiles pair 128 value and 128 gate columns");
    const int half = lane >> 5, l = lane & 31;
    if (wave == 0) {
      // Lane l of half h: scales of tile columns 128 h + 4 l .. +3.
      const int64_t col = (half ? p.half_n : 0) + n0 + 4 * l;
      lds_dma16(make_rsrc(p.sw, (uint32_t)(p.n * 4)), vec_lds, (uint32_t)(col * 4));
    } else if (wave == 1) {
      lds_dma16(make_rsrc(p.sa + m0, (uint32_t)(min((int64_t)BM, p.m - m0) * 4)),
                vec_lds + 1024, (uint32_t)lane * 16);
    } else if (wave == 2 && p.bias) {
      // Lanes 0-15: bias of value columns n0 + 8 l; lanes 16-31: gate columns.
      const int64_t col = (lane >= 16 ? p.half_n + n0 + 8 * (lane - 16) : n0 + 8 * lane);
      const uint32_t off = lane < 32 ? (uint32_t)(col * 2) : VFA_OOB;
      lds_dma16(make_rsrc(p.bias, (uint32_t)(p.n * 2)), vec_lds + 2048, off);
    }
    // The silu window table after the vectors: SILU_LDS / 4 KB blocks of 1 KB per wave.
    constexpr int BLOCKS = SILU_LDS / 4096;
    static_assert(SILU_LDS % 4096 == 0, "four waves share the table's 1 KB blocks");
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(kSiluTable, (uint32_t)SILU_LDS);
    static_for<BLOCKS>([&](auto j) {
      const uint32_t blk = (uint32_t)(wave * BLOCKS + j);
      lds_dma16(rt, vec_lds + VEC_LDS + blk * 1024u, blk * 1024u + (uint32_t)lane * 16u);
    });
    return;
  }
  if (wave == 0) {
    const uint32_t bytes = p.sw_step ? (uint32_t)(min((int64_t)BN, p.n - n0) * 4) : 4u;
    lds_dma16(make_rsrc(p.sw + (p.sw_step ? n0 : 0), bytes), vec_lds, (uint32_t)lane * 16);
  } else if (wave == 1 && p.sa) {
    lds_dma16(make_rsrc(p.sa + m0, (uint32_t)(min((int64_t)BM, p.m - m0) * 4)), vec_lds + 1024,
              (uint32_t)lane * 16);
  } else if (wave == 2 && p.bias) {
    lds_dma16(make_rsrc(p.bias + n0, (uint32_t)(min((int64_t)BN, p.n - n0) * 2)),
              vec_lds + 2048, (uint32_t)lane * 16);
  }
}

// Epilogue shared by every tiling, in two phases through LDS.
//
// Phase 1 (per wave, from the accumulators): a lane holds, for 32x32 block
// (nb, mb) and register r, tile row mb*32 + (lane & 31) and tile column
// nb*32 + 8*(r/4) + 4*(lane/32) + r%4 of its wave's sub-tile.  It applies the
// scales, bias and the register-level epilogue (LoRA merge), rounds to
// bf16 and writes the values into a BM x BN bf16 staging tile in LDS (16-byte
// chunk c of row r stored in slot c ^ (r % chunks-per-row)).  Scale and bias
// vectors are loaded once, before any store.
// Phase 2 (whole workgroup): each thread moves 16-byte row chunks from LDS to
// global memory with coalesced 16-byte stores, applying the gate-residual
// epilogue there with coalesced residual loads.
//
// VEC: read the scale and bias vectors from the LDS copy `vec` made by
// stage_vectors (true), or from global memory (false).
// lora_d: for the LoRA epilogues, the per-block LoRA products computed ahead of
// the main loop ([nb * MB + mb], same layout as acc), or null to compute them here.
// SW_SCALAR: one weight scale for every column (sw[0], the E2M1-weight GEMM's
// alpha) instead of one per column; a compile-time choice, so the per-value
// scale needs no select.
template <int BM, int BN, int WGM, int WGN, int EPI, bool VEC = false, bool SW_SCALAR = false>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p,
                                              v16f (&acc)[BN / WGN / 32][BM / WGM / 32],
                                              int64_t m0, int64_t n0, int wm, int wn, int tid,
                                              uint8_t* stage, const uint8_t* vec = nullptr,
                                              const v16f* lora_d = nullptr) {
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr int NT = 64 * WGM * WGN;
  constexpr int CH = BN / 8;  // 16-byte chunks per staged row
  // Chunk c of staged row r sits in slot c ^ (r % SWZ): every slot of a row
  // when CH is a power of two, else within its aligned group of 8 (CH = 24).
  constexpr int SWZ = (CH & (CH - 1)) == 0 ? CH : 8;
  static_assert(CH % SWZ == 0 && (SWZ & (SWZ - 1)) == 0, "swizzle stays inside the row");
  constexpr int PITCH = BN * 2;
  const int lane = tid & 63, fr = lane & 31, fh = lane >> 5;
  constexpr bool LORA = epi_lora(EPI), GATE = epi_gate(EPI), SWIGLU = epi_swiglu(EPI);
  const LoraBranch br =
      LORA ? lora_branch(p, tile_column<BN, SWIGLU>(p, n0, wn * WN)) : LoraBranch{0, 1.0f};
  const float* __restrict__ sa_p = p.sa;
  const float* __restrict__ sw_p = p.sw;
  const uint16_t* __restrict__ bias_p = p.bias;

  float sam[MB];
  static_for<MB>([&](auto mb) {
    const int row = wm * WM + mb * 32 + fr;
    // No row scales (sa null): a row factor of one, which changes nothing.
    if (!sa_p) {
      sam[mb] = 1.0f;
    } else if constexpr (VEC) {
      sam[mb] = reinterpret_cast<const float*>(vec + 1024)[row];
    } else {
      sam[mb] = m0 + row < p.m ? sa_p[m0 + row] : 0.0f;
    }
  });
  const float sw0 = VEC && SW_SCALAR ? reinterpret_cast<const float*>(vec)[0] : 0.0f;

  // Phase 1, column-block major: the scale and bias of one 32-column block (4
  // columns per g for this lane) are live while its MB row blocks are written.
  // Two copies (with and without bias) keep the bias test out of the loop.
  auto phase1 = [&](auto has_bias) {
    // Every column block's LDS vector reads come first.  As far as the
    // compiler knows the staging writes below may alias them, so a read placed
    // after a write waits for that write, and reads issued block by block would
    // each pay a full LDS round trip.
    v4f s4r[VEC ? NB : 1][4];
    uint2 b4r[VEC ? NB : 1][4];
    if constexpr (VEC) {
      static_for<NB>([&](auto nb) {
        static_for<4>([&](auto g) {
          const int col = wn * WN + nb * 32 + g * 8 + fh * 4;
          s4r[nb][g] = *reinterpret_cast<const v4f*>(vec + col * 4);
          b4r[nb][g] = has_bias ? *reinterpret_cast<const uint2*>(vec + 2048 + col * 2)
                                : make_uint2(0u, 0u);
        });
      });
    }
    static_for<NB>([&](auto nb) {
      float sv[4][4], bv[4][4];
      static_for<4>([&](auto g) {
        const int col = wn * WN + nb * 32 + g * 8 + fh * 4;  // tile column of value i = 0
        if constexpr (VEC) {
          const v4f s4 = s4r[nb][g];
          const uint2 b4 = b4r[nb][g];
          static_for<4>([&](auto i) {
            sv[g][i] = SW_SCALAR ? sw0 : s4[(int)i];
            const uint32_t bw = i < 2 ? b4.x : b4.y;
            bv[g][i] = i % 2 ? bf16_hi(bw) : bf16_lo(bw);
          });
        } else {
          const int64_t n = n0 + col;
          const bool ok = n < p.n;
          static_for<4>([&](auto i) {
            sv[g][i] = ok ? sw_p[(n + i) * p.sw_step] : 0.0f;
            bv[g][i] = (ok && has_bias) ? bf16_to_f32(bias_p[n + i]) : 0.0f;
          });
        }
      });
      static_for<MB>([&](auto mb) {
        const int row = wm * WM + mb * 32 + fr;  // tile row
        const int64_t m = m0 + row;
        const bool mvalid = m < p.m;
        v16f d = v16f{};
        if (LORA && lora_d) {
          d = lora_d[nb * MB + mb];
        } else if constexpr (LORA) {
          // delta block = B[n, :] . t[m, :] on bf16 MFMA, binary32 accumulate.  The
          // operands of every rank step (rank <= 128) are loaded before the first
          // MFMA, so a block waits for one memory round trip, not one per step.
          const int64_t nrow = tile_column<BN, SWIGLU>(p, n0, wn * WN + nb * 32) + fr;
          const bool nok = nrow < p.n;
          v8s bfr[8], tfr[8];
          static_for<8>([&](auto st) {
            bfr[st] = lora_frag(p.lora_b + nrow * p.ldb, p.rank, st, fh, nok);
            tfr[st] = lora_frag(p.lora_t + m * p.ldt + br.toff, p.rank, st, fh, mvalid);
          });
          static_for<8>([&](auto st) {
            if (st * 16 < p.rank)
              d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bfr[st]),
                                                          __builtin_bit_cast(v8bf, tfr[st]), d, 0,
                                                          0, 0);
          });
        }
        if constexpr (LORA) {
          // delta = bf16(t . B^T), then the optional bf16(delta * scale) and
          // bf16(delta * strength) steps, for the block's 16 values at once (two
          // uniform branches per block); d then holds bf16 values as binary32.
          auto round_pairs = [&](float f) {
            static_for<16>([&](auto i) { d[(int)i] = round_bf16_wide(d[(int)i] * f); });
          };
          round_pairs(1.0f);
          if (br.scale != 1.0f) round_pairs(br.scale);
          if (p.lora_strength != 1.0f) round_pairs(p.lora_strength);
        }
        static_for<4>([&](auto g) {
          uint32_t w[2];
          // Output pairs: a bf16 rounding whose result is used again is one
          // conversion per value (round_bf16_wide); the last one is one
          // v_cvt_pk_bf16_f32 for the pair.
          static_for<2>([&](auto h) {
            constexpr int i0 = 2 * h, i1 = 2 * h + 1;
            float y0 = acc[nb][mb][g * 4 + i0] * sam[mb] * sv[g][i0];
            float y1 = acc[nb][mb][g * 4 + i1] * sam[mb] * sv[g][i1];
            if constexpr (has_bias) {
              y0 = round_bf16_wide(y0) + bv[g][i0];
              y1 = round_bf16_wide(y1) + bv[g][i1];
            }
            if constexpr (LORA) {
              y0 = round_bf16_wide(y0) + d[g * 4 + i0];
              y1 = round_bf16_wide(y1) + d[g * 4 + i1];
            }
            w[h] = pack_bf16x2(y0, y1);
          });
          const int c = (wn * WN + nb * 32 + g * 8) / 8;  // 16-byte chunk of the row
          *reinterpret_cast<uint2*>(stage + row * PITCH + ((c ^ (row & (SWZ - 1))) << 4) + fh * 8) =
              make_uint2(w[0], w[1]);
        });
      });
    });
  };
  if (bias_p)
    phase1(std::true_type{});
  else
    phase1(std::false_type{});

  __syncthreads();

  if constexpr (SWIGLU) {
    // Phase 2 of the SwiGLU tile: value chunk c and gate chunk c + CH/2 of a
    // row give 8 outputs h = bf16(value * bf16(silu(gate))) (the eager bf16
    // order of h3_fused_ops.py:184-224); the 16 threads of a row also reduce
    // max |h| over the tile's 128 output columns for the requantization.
    constexpr int CHO = CH / 2;   // output chunks per row
    constexpr int RPO = NT / CHO; // rows per pass
    static_assert(CHO == 16 && BM % RPO == 0, "one 16-lane group per row");
    const int c = tid % CHO, r0 = tid / CHO;
    const int64_t n = n0 + c * 8;
    const int rows = (int)min((int64_t)BM, p.m - m0);
    const int parts = (int)((p.half_n + BN / 2 - 1) / (BN / 2));
    const int part = (int)(n0 / (BN / 2));
    static_assert(VEC, "the silu table is staged with the vectors");
    const float* const silu_tab = reinterpret_cast<const float*>(vec + VEC_LDS);
    // The swizzle of row r0 + it * RPO repeats every two passes: two LDS
    // offsets per half serve every pass.  The chunks of a batch of rows are
    // read before any is used, so the LDS latency is paid once per batch.
    static_assert((2 * RPO) % SWZ == 0, "the swizzle repeats every two passes");
    constexpr int PASSES = BM / RPO, BATCH = PASSES < 8 ? PASSES : 8;
    // Output row r0 + it * RPO: one row step per pass for h and for the maxima.
    uint16_t* const out0 = p.out + (m0 + r0) * p.ldo + n;
    const int64_t ostep = (int64_t)RPO * p.ldo;
    float* const amax0 = p.amax_part + (m0 + r0) * parts + part;
    const int64_t astep = (int64_t)RPO * parts;
    const bool full = rows == BM;
    int vofs[2], gofs[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int rs = (r0 + k * RPO) & (SWZ - 1);
      vofs[k] = r0 * PITCH + ((c ^ rs) << 4);
      gofs[k] = r0 * PITCH + (((c + CHO) ^ rs) << 4);
    }
#pragma unroll
    for (int it0 = 0; it0 < PASSES; it0 += BATCH) {
      v4i vv[BATCH], gg[BATCH];
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int it = it0 + j;
        vv[j] = *reinterpret_cast<const v4i*>(stage + vofs[it & 1] + it * RPO * PITCH);
        gg[j] = *reinterpret_cast<const v4i*>(stage + gofs[it & 1] + it * RPO * PITCH);
      }
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int row = r0 + (it0 + j) * RPO;
        v4i h;
        uint32_t amax_pk = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t vw = (uint32_t)vv[j][q], gw = (uint32_t)gg[j][q];
          const float s0 = silu_lookup(gw, bf16_lo(gw), silu_tab);
          const float s1 = silu_lookup(gw >> 16, bf16_hi(gw), silu_tab);
          const uint32_t hw = pack_bf16x2(bf16_lo(vw) * s0, bf16_hi(vw) * s1);
          amax_pk = abs_max_pk(amax_pk, hw);
          h[q] = (int)hw;
        }
        // Maximum over the 16 lanes of the 128-column group (one DPP row),
        // NaN propagated: the bit patterns of |h| compare as unsigned integers.
        const float amax = __uint_as_float(row16_max_u32(__float_as_uint(abs_max_value(amax_pk))));
        const int it = it0 + j;
        if (full || row < rows) {
          if (n < p.half_n) *reinterpret_cast<v4i*>(out0 + it * ostep) = h;
          if (c == 0) amax0[it * astep] = amax;
        }
      }
    }
    return;
  }

  // Phase 2: LDS rows -> global.  Thread tid owns the 16-byte column chunk
  // c = tid % CH of rows tid / CH + RPP * it, so its column, plane and
  // bounds are computed once.  When CH does not divide the thread count
  // (CH = 24), the last NT - RPP * CH threads have no chunk.
  constexpr int RPP = NT / CH;  // rows per pass
  constexpr int PASSES = (BM + RPP - 1) / RPP;
  static_assert(RPP >= 1, "one row per pass at least");
  if (tid >= RPP * CH) return;
  const int c = tid % CH, r0 = tid / CH;
  const int64_t n = n0 + c * 8;
  if (n >= p.n) return;
  const int rows = (int)min((int64_t)BM, p.m - m0);
  uint16_t* base = p.out + n;
  if (p.plane_cols > 0) {
    const int64_t plane = n / p.plane_cols;
    base = p.out + plane * p.plane_stride + (n - plane * p.plane_cols);
  }
  // Chunk c of staged row `row` (SWZ is a power of two).
  auto lds_chunk = [&](int row) {
    return *reinterpret_cast<const v4i*>(stage + row * PITCH + ((c ^ (row & (SWZ - 1))) << 4));
  };
  // Gate-residual epilogues: the residual chunk and the gate chunk of output row m0 + row,
  // whose gate row is that of token `tok` (m % gate_tokens), through the index
  // when one is given (the adaLN gather read in place).  An index outside
  // [0, gate_rows) makes the row's gate NaN (quiet-NaN bf16 pairs in place of
  // the gate chunk); nothing outside is read.  With unit gate stride and
  // 16-byte aligned rows (vec_in) each is one load.
  struct GateIn {
    v4i res, gate;
  };
  const bool vec_in = GATE && p.gate_hs == 1 &&
                      ((reinterpret_cast<uintptr_t>(p.gate) | reinterpret_cast<uintptr_t>(p.residual)) & 15) == 0 &&
                      p.gate_ts % 8 == 0 && p.ldr % 8 == 0;
  auto gate_in = [&](int row, int64_t tok, auto vec) {
    GateIn in;
    const int64_t m = m0 + row;
    int64_t g = tok;
    bool bad = false;
    if (p.gate_index) {
      g = p.gate_index[tok];
      if ((uint64_t)g >= (uint64_t)p.gate_rows) {
        g = 0;
        bad = true;
      }
    }
    const uint16_t* res = p.residual + m * p.ldr + n;
    const uint16_t* gt = p.gate + g * p.gate_ts + n * p.gate_hs;
    if constexpr (vec) {
      in.res = *reinterpret_cast<const v4i*>(res);
      in.gate = *reinterpret_cast<const v4i*>(gt);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        in.res[j] = (int)((uint32_t)res[2 * j] | ((uint32_t)res[2 * j + 1] << 16));
        in.gate[j] = (int)((uint32_t)gt[(2 * j) * p.gate_hs] |
                           ((uint32_t)gt[(2 * j + 1) * p.gate_hs] << 16));
      }
    }
    if (bad) in.gate = v4i{0x7fc07fc0, 0x7fc07fc0, 0x7fc07fc0, 0x7fc07fc0};
    return in;
  };
  // out = bf16(residual + bf16(gate * y)) for the 8 outputs of a chunk.
  auto gate_apply = [&](v4i v, const GateIn& in) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t y = (uint32_t)v[j], gw = (uint32_t)in.gate[j], rw = (uint32_t)in.res[j];
      const float gy0 = round_bf16_wide(bf16_lo(gw) * bf16_lo(y));
      const float gy1 = round_bf16_wide(bf16_hi(gw) * bf16_hi(y));
      v[j] = (int)pack_bf16x2(bf16_lo(rw) + gy0, bf16_hi(rw) + gy1);
    }
    return v;
  };
  auto store = [&](v4i v, uint16_t* dst, auto vec_out) {
    if constexpr (vec_out) {
      *reinterpret_cast<v4i*>(dst) = v;
    } else {
      reinterpret_cast<uint2*>(dst)[0] = make_uint2((uint32_t)v[0], (uint32_t)v[1]);
      reinterpret_cast<uint2*>(dst)[1] = make_uint2((uint32_t)v[2], (uint32_t)v[3]);
    }
  };
  // Token of row r0 (gate-residual epilogues), advanced by RPP rows per pass.
  const int64_t tokens = GATE ? p.gate_tokens : 1;
  int64_t tok = GATE ? (m0 + r0) % tokens : 0;
  const int64_t tok_step = GATE ? RPP % tokens : 0;
  auto next_tok = [&]() {
    tok += tok_step;
    if (tok >= tokens) tok -= tokens;
  };
  auto pass = [&](auto vec_out) {
    if (rows == BM && (!GATE || vec_in)) {
      // A whole tile (with vector residual and gate loads for the gate-residual): the
      // chunks of BATCH rows (and their residual and gate chunks) are loaded
      // before any is stored, so each latency is paid once
      // per batch, not once per row.  The swizzle of row r0 + it * RPP repeats
      // every four passes, so four LDS offsets and one output row step serve
      // every pass.  With CH = 24 (26 passes of 10 rows) the last pass reaches
      // rows up to 259: those past BM are read from LDS (at most 100 KB into the
      // 112 KB ring) but neither loaded from global memory nor stored; the
      // batch's passes past the last (26..31) read nothing.
      static_assert((4 * RPP) % SWZ == 0, "the swizzle repeats every four passes");
      constexpr int BATCH = PASSES < 8 ? PASSES : 8;
      int lofs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) lofs[k] = r0 * PITCH + ((c ^ ((r0 + k * RPP) & (SWZ - 1))) << 4);
      uint16_t* const dst0 = base + (m0 + r0) * p.ldo;
      const int64_t dstep = (int64_t)RPP * p.ldo;
#pragma unroll
      for (int it0 = 0; it0 < PASSES; it0 += BATCH) {
        v4i v[BATCH];
        GateIn in[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
          const int it = it0 + j;
          const int row = r0 + it * RPP;
          if (it < PASSES)  // a constant: the loop is unrolled
            v[j] = *reinterpret_cast<const v4i*>(stage + lofs[it & 3] + it * RPP * PITCH);
          if constexpr (GATE) {
            if (it < PASSES && (PASSES * RPP == BM || row < BM))
              in[j] = gate_in(row, tok, std::true_type{});
            next_tok();
          }
        }
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
          const int it = it0 + j;
          const int row = r0 + it * RPP;
          if (it < PASSES && (PASSES * RPP == BM || row < BM)) {
            v4i o = v[j];
            if constexpr (GATE) o = gate_apply(o, in[j]);
            store(o, dst0 + it * dstep, vec_out);
          }
        }
      }
    } else {
#pragma unroll 8
      for (int it = 0; it < PASSES; ++it) {
        const int row = r0 + it * RPP;
        if (row >= rows) break;
        v4i o = lds_chunk(row);
        if constexpr (GATE) {
          o = vec_in ? gate_apply(o, gate_in(row, tok, std::true_type{}))
                     : gate_apply(o, gate_in(row, tok, std::false_type{}));
          next_tok();
        }
        store(o, base + (m0 + row) * p.ldo, vec_out);
      }
    }
  };
  if (((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) && (p.ldo % 8 == 0) &&
      (p.plane_cols == 0 || p.plane_stride % 8 == 0))
    pass(std::true_type{});
  else
    pass(std::false_type{});
}

}  // namespace vfa
