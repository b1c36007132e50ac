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

// block_col(wn, nb) = wave_col(wn) + block_off(nb): the tile column of the
// first column of block nb of wave column wn (WN columns per wave, NB blocks
// of 32).  SwiGLU tiles pair each value block with its gate block inside one
// wave: block 2j is value block wn * NB/2 + j (tile columns [0, BN/2)) and
// block 2j + 1 the matching gate block (BN/2 + the same), so a lane holds the
// value and the gate of each of its outputs.
template <int BN, int WN, bool SWIGLU>
__device__ __forceinline__ int wave_col(int wn) {
  return SWIGLU ? wn * (WN / 2) : wn * WN;
}
template <int BN, int WN, bool SWIGLU>
constexpr int block_off(int nb) {
  static_assert(!SWIGLU || (WN / 32) % 2 == 0, "value and gate blocks pair up");
  return SWIGLU ? (nb & 1) * (BN / 2) + (nb / 2) * 32 : nb * 32;
}
template <int BN, int WN, bool SWIGLU>
__device__ __forceinline__ int block_col(int wn, int nb) {
  return wave_col<BN, WN, SWIGLU>(wn) + block_off<BN, WN, SWIGLU>(nb);
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
  const LoraBranch br = lora_branch(p, tile_column<BN, SWIGLU>(p, n0, block_col<BN, WN, SWIGLU>(wn, 0)));
  v8s bf[NB][RS], tf[MB][RS];
  static_for<NB>([&](auto nb) {
    const int64_t nrow = tile_column<BN, SWIGLU>(p, n0, block_col<BN, WN, SWIGLU>(wn, nb)) + fr;
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
// LDS bytes of the silu lookup table, which SwiGLU tiles stage after the vectors.
constexpr int SILU_LDS = 2 * (int)kSiluStride * 4;

// bf16(silu(g)) as a binary32 value is silu_apply(g, silu_entry(g, tab)), for g
// a bf16 value held as binary32 (low half zero) and `tab` the lookup table in
// LDS; two steps, so a caller can have many table reads in flight.  The entry
// is that of g's bf16 pattern for 2^-9 <= |g| <= 126.5, else the below- or
// above-window entry of g's sign.
// An entry holds T (high half) and a factor M (low half), both bf16, and the
// result is bf16(fma(g, M, T)): T in the window; bf16(g / 2) below it; g above
// it for g > 0 and g * 0 (-0, or NaN for -inf) for g < 0, T being a zero of g's
// sign.  Every bf16 input gives the binary32 formula g / (1 + exp(-g)) of
// h3_fused_ops.py:205 with each step correctly rounded, then rounded to bf16
// (the table is generated to that definition).
__device__ __forceinline__ uint32_t silu_entry(float g, const uint32_t* tab) {
  const uint32_t gw = __float_as_uint(g);
  const int a = (int)((gw >> 16) & 0x7fffu);
  // Clamped to one entry below and one above the window.
  const int c = min(max(a, (int)kSiluLo - 1), (int)(kSiluLo + kSiluN));
  return tab[(gw >> 31) * kSiluStride + (uint32_t)(c - ((int)kSiluLo - 1))];
}
__device__ __forceinline__ float silu_apply(float g, uint32_t e) {
  return round_bf16_wide(__builtin_fmaf(g, __uint_as_float(e << 16), __uint_as_float(e & 0xffff0000u)));
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

// The default `pre` of gemm_epilogue: no MFMA left to issue.
struct NoPre {
  template <class Q>
  __device__ __forceinline__ void operator()(Q) const {}
};

// Epilogue shared by every tiling, in two phases through LDS.
//
// Phase 1 (per wave, from the accumulators): a lane holds, for 32x32 block
// (nb, mb) and register r, tile row mb*32 + (lane & 31) and tile column
// block_col(wn, nb) + 8*(r/4) + 4*(lane/32) + r%4.  It applies the scales,
// bias and the register-level epilogue (LoRA merge), rounds to bf16 and
// writes the values into a BM x BN bf16 staging tile in LDS (16-byte chunk c
// of row r stored in slot c ^ (r % chunks-per-row)).  Scale and bias vectors
// are loaded once, before any store.  SwiGLU tiles hold each output's value
// and gate in one lane, so phase 1 forms h = bf16(value * bf16(silu(gate)))
// there and stages the BM x BN/2 tile of h.
// Phase 2 (whole workgroup): each thread moves 16-byte row chunks from LDS to
// global memory with coalesced 16-byte stores, applying the gate-residual
// epilogue there with coalesced residual loads (SwiGLU: and reducing the row
// maxima of h).
//
// VEC: read the scale and bias vectors from the LDS copy `vec` made by
// stage_vectors (true), or from global memory (false).
// lora_d: for the LoRA epilogues, the per-block LoRA products computed ahead of
// the main loop ([nb * MB + mb], same layout as acc), or null to compute them here.
// SW_SCALAR: one weight scale for every column (sw[0], the E2M1-weight GEMM's
// alpha) instead of one per column; a compile-time choice, so the per-value
// scale needs no select.
// pre(q): issues the last MFMA of block q = nb * MB + mb (the caller's last
// K substep), called LAG blocks ahead of phase 1's work on block q, so the
// MFMA pipe runs those MFMAs under phase 1's VALU work.
template <int BM, int BN, int WGM, int WGN, int EPI, bool VEC = false, bool SW_SCALAR = false,
          class Pre = NoPre>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p,
                                              v16f (&acc)[BN / WGN / 32][BM / WGM / 32],
                                              int64_t m0, int64_t n0, int wm, int wn, int tid,
                                              uint8_t* stage, const uint8_t* vec = nullptr,
                                              const v16f* lora_d = nullptr, Pre pre = Pre{}) {
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr int NT = 64 * WGM * WGN;
  constexpr bool LORA = epi_lora(EPI), GATE = epi_gate(EPI), SWIGLU = epi_swiglu(EPI);
  // Staged columns: the tile's, or the BN/2 outputs of a SwiGLU tile.
  constexpr int SBN = SWIGLU ? BN / 2 : BN;
  constexpr int CH = SBN / 8;  // 16-byte chunks per staged row
  // Chunk c of staged row r sits in slot c ^ (r % SWZ): every slot of a row
  // when CH is a power of two, else within its aligned group of 8 (CH = 24).
  constexpr int SWZ = (CH & (CH - 1)) == 0 ? CH : 8;
  static_assert(CH % SWZ == 0 && (SWZ & (SWZ - 1)) == 0, "swizzle stays inside the row");
  constexpr int PITCH = SBN * 2;
  const int lane = tid & 63, fr = lane & 31, fh = lane >> 5;
  const LoraBranch br =
      LORA ? lora_branch(p, tile_column<BN, SWIGLU>(p, n0, block_col<BN, WN, SWIGLU>(wn, 0)))
           : LoraBranch{0, 1.0f};
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

  // The LoRA delta of block (nb, mb) as bf16 values held in binary32: the
  // products computed ahead of the main loop, or B[n, :] . t[m, :] on bf16
  // MFMA (binary32 accumulation) with the operands of every rank step (rank <=
  // 128) loaded before the first MFMA, so a block waits for one memory round
  // trip, not one per step; then bf16(t . B^T) and the optional bf16(delta *
  // scale) and bf16(delta * strength) steps, for the block's 16 values at once
  // (two uniform branches per block).
  auto lora_delta = [&](auto nb, auto mb) {
    v16f d = v16f{};
    if constexpr (LORA) {
      if (lora_d) {
        d = lora_d[nb * MB + mb];
      } else {
        const int64_t m = m0 + wm * WM + mb * 32 + fr;
        const int64_t nrow = tile_column<BN, SWIGLU>(p, n0, block_col<BN, WN, SWIGLU>(wn, nb)) + fr;
        const bool nok = nrow < p.n, mvalid = m < p.m;
        v8s bfr[8], tfr[8];
        static_for<8>([&](auto st) {
          bfr[st] = lora_frag(p.lora_b + nrow * p.ldb, p.rank, st, fh, nok);
          tfr[st] = lora_frag(p.lora_t + m * p.ldt + br.toff, p.rank, st, fh, mvalid);
        });
        static_for<8>([&](auto st) {
          if (st * 16 < p.rank)
            d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bfr[st]),
                                                        __builtin_bit_cast(v8bf, tfr[st]), d, 0, 0,
                                                        0);
        });
      }
      auto round_pairs = [&](float f) {
        static_for<16>([&](auto i) { d[(int)i] = round_bf16_wide(d[(int)i] * f); });
      };
      round_pairs(1.0f);
      if (br.scale != 1.0f) round_pairs(br.scale);
      if (p.lora_strength != 1.0f) round_pairs(p.lora_strength);
    }
    return d;
  };

  // Phase 1, column-block major: the scale and bias of one 32-column block (4
  // columns per g for this lane) are live while its MB row blocks are written.
  // Two copies (with and without bias) keep the bias test out of the loop.
  auto phase1 = [&](auto has_bias) {
    // Every column block's LDS vector reads come first.  As far as the
    // compiler knows the staging writes below may alias them, so a read placed
    // after a write waits for that write, and reads issued block by block would
    // each pay a full LDS round trip.
    // (SwiGLU tiles, whose phase 1 holds more registers, read them block by
    // block instead, for one value/gate pair of blocks at a time.)
    constexpr int PRE_NB = VEC && !SWIGLU ? NB : 1;
    v4f s4r[PRE_NB][4];
    uint2 b4r[PRE_NB][4];
    if constexpr (VEC && !SWIGLU) {
      static_for<NB>([&](auto nb) {
        static_for<4>([&](auto g) {
          const int col = block_col<BN, WN, SWIGLU>(wn, nb) + g * 8 + fh * 4;
          s4r[nb][g] = *reinterpret_cast<const v4f*>(vec + col * 4);
          b4r[nb][g] = has_bias ? *reinterpret_cast<const uint2*>(vec + 2048 + col * 2)
                                : make_uint2(0u, 0u);
        });
      });
    }
    // Scale and bias of the 16 columns block nb holds in this lane.
    auto block_vectors = [&](auto nb, float (&sv)[4][4], float (&bv)[4][4]) {
      static_for<4>([&](auto g) {
        const int col = block_col<BN, WN, SWIGLU>(wn, nb) + g * 8 + fh * 4;  // value i = 0
        if constexpr (VEC) {
          v4f s4;
          uint2 b4;
          if constexpr (SWIGLU) {
            s4 = *reinterpret_cast<const v4f*>(vec + col * 4);
            b4 = has_bias ? *reinterpret_cast<const uint2*>(vec + 2048 + col * 2) : make_uint2(0u, 0u);
          } else {
            s4 = s4r[nb][g];
            b4 = b4r[nb][g];
          }
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
    };
    // The epilogue value of register i of a block before its last bf16
    // rounding: bf16(acc * sa * sw) + bias, then bf16(.) + delta where present
    // (the reference's roundings, in order).
    auto value = [&](float a, float sm, float sc, float b, float dl) {
      float y = a * sm * sc;
      if constexpr (has_bias) y = round_bf16_wide(y) + b;
      if constexpr (LORA) y = round_bf16_wide(y) + dl;
      return y;
    };
    constexpr int Q = NB * MB, LAG = 2;
    if constexpr (SWIGLU) {
      // Value block 2j and gate block 2j + 1 hold the same outputs: every
      // block's last MFMA first.
      static_for<Q>([&](auto q) { pre(q); });
      const uint32_t* const silu_tab = reinterpret_cast<const uint32_t*>(vec + VEC_LDS);
      static_for<NB / 2>([&](auto j) {
        constexpr int vb = 2 * j, gb = 2 * j + 1;
        float svv[4][4], bvv[4][4], svg[4][4], bvg[4][4];
        block_vectors(std::integral_constant<int, vb>{}, svv, bvv);
        block_vectors(std::integral_constant<int, gb>{}, svg, bvg);
        static_for<MB>([&](auto mb) {
          const int row = wm * WM + mb * 32 + fr;  // tile row
          const v16f dv = lora_delta(std::integral_constant<int, vb>{}, mb);
          const v16f dg = lora_delta(std::integral_constant<int, gb>{}, mb);
          // Eight outputs at a time: their gates and table reads first, then
          // the values while the reads are in flight (scheduling barriers
          // keep the groups apart).
          static_for<2>([&](auto half) {
            float gt[8], vl[8];
            uint32_t e[8];
            static_for<8>([&](auto t) {
              constexpr int i = 8 * half + t, g = i / 4, k = i % 4;
              gt[t] = round_bf16_wide(value(acc[gb][mb][i], sam[mb], svg[g][k], bvg[g][k], dg[i]));
            });
            static_for<8>([&](auto t) { e[t] = silu_entry(gt[t], silu_tab); });
            __builtin_amdgcn_sched_barrier(0);
            static_for<8>([&](auto t) {
              constexpr int i = 8 * half + t, g = i / 4, k = i % 4;
              vl[t] = round_bf16_wide(value(acc[vb][mb][i], sam[mb], svv[g][k], bvv[g][k], dv[i]));
            });
            __builtin_amdgcn_sched_barrier(0);
            static_for<2>([&](auto gg) {
              constexpr int g = 2 * half + gg;
              uint32_t w[2];
              static_for<2>([&](auto h) {
                constexpr int t0 = 4 * gg + 2 * h, t1 = t0 + 1;
                w[h] = pack_bf16x2(vl[t0] * silu_apply(gt[t0], e[t0]), vl[t1] * silu_apply(gt[t1], e[t1]));
              });
              // Output chunk of these 4 columns (the value block's tile column / 8).
              const int c = (block_col<BN, WN, SWIGLU>(wn, vb) + g * 8) / 8;
              *reinterpret_cast<uint2*>(stage + row * PITCH + ((c ^ (row & (SWZ - 1))) << 4) + fh * 8) =
                  make_uint2(w[0], w[1]);
            });
          });
        });
      });
      return;
    }
    static_for<(LAG < Q ? LAG : Q)>([&](auto q) { pre(q); });
    static_for<NB>([&](auto nb) {
      float sv[4][4], bv[4][4];
      block_vectors(nb, sv, bv);
      static_for<MB>([&](auto mb) {
        constexpr int q = nb * MB + mb;
        if constexpr (q + LAG < Q) pre(std::integral_constant<int, q + LAG>{});
        const int row = wm * WM + mb * 32 + fr;  // tile row
        const v16f d = lora_delta(nb, mb);
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
          const int c = (block_col<BN, WN, SWIGLU>(wn, nb) + g * 8) / 8;  // 16-byte chunk of the row
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
    // Phase 2 of the SwiGLU tile: 16 threads per row store its 128 outputs of
    // h (8 per thread) and reduce max |h| over them for the requantization.
    constexpr int RPO = NT / CH;  // rows per pass
    static_assert(CH == 16 && BM % RPO == 0, "one 16-lane group per row");
    const int c = tid % CH, r0 = tid / CH;
    const int64_t n = n0 + c * 8;
    const int rows = (int)min((int64_t)BM, p.m - m0);
    const int parts = (int)((p.half_n + BN / 2 - 1) / (BN / 2));
    const int part = (int)(n0 / (BN / 2));
    static_assert(VEC, "the silu table is staged with the vectors");
    // The swizzle of row r0 + it * RPO repeats every four passes: four LDS
    // offsets serve every pass.  The chunks of a batch of rows are read before
    // any is used, so the LDS latency is paid once per batch.
    static_assert((4 * RPO) % SWZ == 0, "the swizzle repeats every four passes");
    constexpr int PASSES = BM / RPO, BATCH = PASSES < 8 ? PASSES : 8;
    // Output row r0 + it * RPO: one row step per pass for h and for the maxima.
    uint16_t* const out0 = p.out + (m0 + r0) * p.ldo + n;
    const int64_t ostep = (int64_t)RPO * p.ldo;
    float* const amax0 = p.amax_part + (m0 + r0) * parts + part;
    const int64_t astep = (int64_t)RPO * parts;
    const bool full = rows == BM;
    int ofs[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) ofs[k] = r0 * PITCH + ((c ^ ((r0 + k * RPO) & (SWZ - 1))) << 4);
#pragma unroll
    for (int it0 = 0; it0 < PASSES; it0 += BATCH) {
      v4i hh[BATCH];
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int it = it0 + j;
        hh[j] = *reinterpret_cast<const v4i*>(stage + ofs[it & 3] + it * RPO * PITCH);
      }
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int it = it0 + j;
        const int row = r0 + it * RPO;
        uint32_t amax_pk = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) amax_pk = abs_max_pk(amax_pk, (uint32_t)hh[j][q]);
        // Maximum over the 16 lanes of the 128-column group (one DPP row),
        // NaN propagated: the bit patterns of |h| compare as unsigned integers.
        const float amax = __uint_as_float(row16_max_u32(__float_as_uint(abs_max_value(amax_pk))));
        if (full || row < rows) {
          if (n < p.half_n) *reinterpret_cast<v4i*>(out0 + it * ostep) = hh[j];
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
      // chunks of BATCH rows are read from LDS before any is stored, so each
      // latency is paid once per batch, not once per row.  The swizzle of row r0 + it * RPP repeats
      // every four passes, so four LDS offsets and one output row step serve
      // every pass.  With CH = 24 (26 passes of 10 rows) the last pass reaches
      // rows up to 259: those past BM are read from LDS (at most 100 KB into the
      // 136 KB ring, below the vectors at 112 KB) but neither loaded from global
      // memory nor stored; the batch's passes past the last (26..31) read nothing.
      static_assert((4 * RPP) % SWZ == 0, "the swizzle repeats every four passes");
      constexpr int BATCH = PASSES < 8 ? PASSES : 8;
      int lofs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) lofs[k] = r0 * PITCH + ((c ^ ((r0 + k * RPP) & (SWZ - 1))) << 4);
      uint16_t* const dst0 = base + (m0 + r0) * p.ldo;
      const int64_t dstep = (int64_t)RPP * p.ldo;
      if constexpr (GATE) {
        // Gate-residual: the residual and gate chunks of batch b + 1 are
        // loaded before batch b is combined and stored, so their latency
        // overlaps that work.  A gate of one row (no index) is loaded once.
        constexpr int NBATCH = (PASSES + BATCH - 1) / BATCH;
        auto run = [&](auto bcast) {
          v4i gate0 = v4i{};
          if constexpr (bcast) gate0 = *reinterpret_cast<const v4i*>(p.gate + n);
          GateIn in[2][BATCH];
          auto load = [&](auto b) {
            static_for<BATCH>([&](auto j) {
              constexpr int it = b * BATCH + j;
              const int row = r0 + it * RPP;
              if constexpr (it < PASSES) {
                if (PASSES * RPP == BM || row < BM) {
                  if constexpr (bcast) {
                    in[b & 1][j].res = *reinterpret_cast<const v4i*>(p.residual + (m0 + row) * p.ldr + n);
                    in[b & 1][j].gate = gate0;
                  } else {
                    in[b & 1][j] = gate_in(row, tok, std::true_type{});
                  }
                }
                if constexpr (!bcast) next_tok();
              }
            });
          };
          load(std::integral_constant<int, 0>{});
          static_for<NBATCH>([&](auto b) {
            v4i v[BATCH];
            static_for<BATCH>([&](auto j) {
              constexpr int it = b * BATCH + j;
              if constexpr (it < PASSES)
                v[j] = *reinterpret_cast<const v4i*>(stage + lofs[it & 3] + it * RPP * PITCH);
            });
            if constexpr (b + 1 < NBATCH) load(std::integral_constant<int, b + 1>{});
            static_for<BATCH>([&](auto j) {
              constexpr int it = b * BATCH + j;
              const int row = r0 + it * RPP;
              if constexpr (it < PASSES) {
                if (PASSES * RPP == BM || row < BM)
                  store(gate_apply(v[j], in[b & 1][j]), dst0 + it * dstep, vec_out);
              }
            });
          });
        };
        if (tokens == 1 && !p.gate_index)
          run(std::true_type{});
        else
          run(std::false_type{});
      } else {
#pragma unroll
        for (int it0 = 0; it0 < PASSES; it0 += BATCH) {
          v4i v[BATCH];
#pragma unroll
          for (int j = 0; j < BATCH; ++j) {
            const int it = it0 + j;
            if (it < PASSES)  // a constant: the loop is unrolled
              v[j] = *reinterpret_cast<const v4i*>(stage + lofs[it & 3] + it * RPP * PITCH);
          }
#pragma unroll
          for (int j = 0; j < BATCH; ++j) {
            const int it = it0 + j;
            const int row = r0 + it * RPP;
            if (it < PASSES && (PASSES * RPP == BM || row < BM)) store(v[j], dst0 + it * dstep, vec_out);
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
