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
// binary16, and so is every E4M3 code: the contraction has no rounding ahead of
// the binary32 accumulator.  One kernel serves every shape (nvfp4_gemm_pipe:
// packed operands staged in LDS by DMA and dequantized in registers into f16
// MFMA operands), so the sum order of an output never depends on M.
// Weights stay packed (0.5 byte/element) in HBM.  Scales use the 128x4 tiled order of NVFP4Weight
// (h3_nvfp4_linear.py:22-33): for row n and K block j (16 elements),
//   off = (n/128)*(K/64)*512 + (j/4)*512 + (n%32)*16 + ((n%128)/32)*4 + j%4.
#include "gemm_epilogue.h"

namespace vfa {

// ---------------------------------------------------------------------------
// Pipelined 256x256 W4A8 kernel: packed operands in LDS, dequantization in
// registers, f16 MFMA.
//
// Every E4M3 code and every product e2m1 * e4m3 (at most 6 significant bits,
// magnitude 2^-10 .. 2688) is exact in binary16, so the contraction runs on
// v_mfma_f32_32x32x16_f16 with no rounding ahead of the binary32 accumulator,
// the same sum as the bf16 form.  binary16 is used because its packed multiply
// (v_pk_mul_f16) applies the E4M3 block scale exactly in one instruction; the
// hardware-scaled converters take only the exponent of their scale operand.
//
// LDS holds each stage (128 K) as it sits in HBM: A codes (256 rows x 128 B),
// packed weights (256 rows x 64 B) and the stage's block scales (two 1 KB
// runs of the 128x4 order), filled by buffer-load-to-LDS DMA, two slots.  A
// lane dequantizes only the values it feeds to its MFMAs:
//   A: v_cvt_scalef32_pk_f16_fp8 (scale 1), two codes per instruction;
//   W: v_cvt_scalef32_pk_f16_fp4 (scale 1) then v_pk_mul_f16 by the block
//      scale, two values per two instructions.
// K is consumed in a lane-friendly order (the sum does not depend on it): for
// MFMA step v of a 64-K half u, lanes 0-31 supply K 64u + 8v .. +7 and lanes
// 32-63 supply K 64u + 32 + 8v .. +7, so each lane reads 32 contiguous codes
// and 16 contiguous packed bytes (one or two 16-element scale blocks) per half.
//
// W4A4 (A4 = true, the reference's mm_fp4 arithmetic): A is packed E2M1 with
// its own 128x4 block scales, staged and dequantized exactly as W; the slot is
// A 16 KB + W 16 KB + W scales 2 KB + A scales 2 KB, and the epilogue applies
// the one output scale alpha (no per-row scale).
constexpr int FP4_A = 256 * 128;
constexpr int FP4_W = 256 * 64;
constexpr int FP4_S = 2 * 1024;
constexpr int FP4_LDS = 256 * 256 * 2;  // also the epilogue's bf16 staging tile
template <bool A4>
constexpr int fp4_a_bytes() { return A4 ? FP4_W : FP4_A; }
template <bool A4>
constexpr int fp4_slot() { return fp4_a_bytes<A4>() + FP4_W + FP4_S + (A4 ? FP4_S : 0); }
static_assert(2 * fp4_slot<false>() <= FP4_LDS && 2 * fp4_slot<true>() <= FP4_LDS,
              "ring fits the staging buffer");

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <bool A4>
__global__ void __launch_bounds__(256) nvfp4_gemm_pipe(const GemmParams p) {
  constexpr int SA = fp4_a_bytes<A4>(), FP4_SLOT = fp4_slot<A4>();
  constexpr int OFF_W = SA, OFF_WS = SA + FP4_W, OFF_AS = SA + FP4_W + FP4_S;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[FP4_LDS];
  __shared__ __attribute__((aligned(1024))) uint8_t vec[VEC_LDS];
  constexpr int MB = 4, NB = 4;
  const int tiles_m = (int)((p.m + 255) / 256), tiles_n = (int)((p.n + 255) / 256);
  int tm, tn;
  tile_coords(tiles_m, tiles_n, p.group_m, tm, tn);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = (int)threadIdx.x & 63;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t m0 = (int64_t)tm * 256, n0 = (int64_t)tn * 256;
  const int64_t k_tiles = p.k / 64;  // 128x4 scale tiles along K
  const int64_t rows_a = min((int64_t)256, p.m - m0);
  const int64_t rows_w = min((int64_t)256, p.n - n0);  // 128 or 256 (n % 128 == 0)
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w + n0 * p.ldw, (uint32_t)(rows_w * p.ldw));
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(p.wsb + (n0 / 128) * k_tiles * 512, (uint32_t)((rows_w / 128) * k_tiles * 512));
  // A4: the A scales' 128-row tiles of this block (the caller pads the rows to 128).
  const __amdgpu_buffer_rsrc_t ras =
      A4 ? make_rsrc(p.asb + (m0 / 128) * k_tiles * 512,
                     (uint32_t)(((rows_a + 127) / 128) * k_tiles * 512))
         : rs;

  // DMA lane maps.  A: 1 KB block i of a wave = rows wave*64 + 8i .. +7, lane l
  // fills row + l/8, slot l%8 with logical chunk (l%8) ^ lds_swizzle(row).
  const int drow = lane >> 3;
  const int ach0 = (lane & 7) ^ lds_swizzle(drow), ach1 = (lane & 7) ^ lds_swizzle(drow + 8);
  const uint32_t a_base0 = (uint32_t)((wave * 64 + drow) * p.lda + ach0 * 16);
  const uint32_t a_base1 = (uint32_t)((wave * 64 + drow + 8) * p.lda + ach1 * 16);
  const uint32_t a_step = (uint32_t)(16 * p.lda);
  // W: 64-byte rows; 1 KB block i of a wave = rows wave*64 + 16i .. +15, lane
  // l fills row + l/4, slot l%4 with logical chunk (l%4) ^ ((row >> 2) & 3).
  const int wch = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t w_base = (uint32_t)((wave * 64 + (lane >> 2)) * p.ldw + wch * 16);
  const uint32_t w_step = (uint32_t)(16 * p.ldw);
  // Scales: waves 0 and 1 copy the stage's 1 KB (K tiles 2s, 2s+1) of W row tile
  // wave & 1; with A4, waves 2 and 3 do the same for A.
  const uint32_t dst_a = ring_lds + wave * (A4 ? 4096 : 8192), dst_w = ring_lds + OFF_W + wave * 4096;
  const uint32_t dst_s = ring_lds + OFF_WS + (wave & 1) * 1024;
  const uint32_t dst_as = ring_lds + OFF_AS + (wave & 1) * 1024;
  const uint32_t s_base_any = (uint32_t)((wave & 1) * k_tiles * 512 + lane * 16);
  const int KT = (int)((p.k + 127) / 128);

  // Full tiles with K % 128 == 0 (FULL) advance K and the row blocks through the
  // scalar offset, and kill stages past the end by switching to an empty
  // resource, so a DMA instruction costs no vector instruction; other tiles keep
  // every offset in the lane offset, where the range check zeroes rows past the
  // end and chunks past K.
  const bool full = __builtin_amdgcn_readfirstlane(
                        (int)(rows_a == 256 && rows_w == 256 && p.k % 128 == 0)) != 0;
  const __amdgpu_buffer_rsrc_t none = make_rsrc(p.w, 0u);
  auto issue_s = [&](int j, int s) {
    const uint32_t slot = (uint32_t)j * FP4_SLOT;
    const bool live = s < KT;
    const __amdgpu_buffer_rsrc_t ra_s = live ? ra : none, rw_s = live ? rw : none;
    const __amdgpu_buffer_rsrc_t rs_s = live ? rs : none, ras_s = live ? ras : none;
    const uint32_t kb = live ? (uint32_t)s * 128u : 0u, kw = kb / 2;
    if constexpr (A4) {
      const uint32_t a4_base = (uint32_t)((wave * 64 + (lane >> 2)) * p.lda + wch * 16);
      static_for<4>([&](auto i) {
        lds_dma16_so(ra_s, dst_a + slot + i * 1024, a4_base, i * (uint32_t)(16 * p.lda) + kw);
      });
    } else {
      static_for<8>([&](auto i) {
        lds_dma16_so(ra_s, dst_a + slot + i * 1024, i % 2 ? a_base1 : a_base0, (i / 2) * a_step + kb);
      });
    }
    static_for<4>([&](auto i) {
      lds_dma16_so(rw_s, dst_w + slot + i * 1024, w_base, i * w_step + kw);
    });
    if (wave < 2) {
      lds_dma16_so(rs_s, dst_s + slot, s_base_any, live ? (uint32_t)s * 1024u : 0u);
    } else if constexpr (A4) {
      lds_dma16_so(ras_s, dst_as + slot, s_base_any, live ? (uint32_t)s * 1024u : 0u);
    }
  };
  auto issue_v = [&](int j, int s) {
    const uint32_t slot = (uint32_t)j * FP4_SLOT;
    const int64_t kb = (int64_t)s * 128;
    const int64_t kw = kb / 2;
    const uint32_t killw = kw + wch * 16 < p.k / 2 ? 0u : VFA_OOB;
    if constexpr (A4) {
      // 64-byte packed rows, the W map with A's row stride.
      const uint32_t a4_base = (uint32_t)((wave * 64 + (lane >> 2)) * p.lda + wch * 16);
      static_for<4>([&](auto i) {
        lds_dma16(ra, dst_a + slot + i * 1024,
                  (a4_base + i * (uint32_t)(16 * p.lda) + (uint32_t)kw) | killw);
      });
    } else {
      const uint32_t kill0 = kb + ach0 * 16 < p.k ? 0u : VFA_OOB;
      const uint32_t kill1 = kb + ach1 * 16 < p.k ? 0u : VFA_OOB;
      static_for<8>([&](auto i) {
        const uint32_t off = (i % 2 ? a_base1 : a_base0) + (i / 2) * a_step + (uint32_t)kb;
        lds_dma16(ra, dst_a + slot + i * 1024, off | (i % 2 ? kill1 : kill0));
      });
    }
    static_for<4>([&](auto i) {
      lds_dma16(rw, dst_w + slot + i * 1024, (w_base + i * w_step + (uint32_t)kw) | killw);
    });
    const uint32_t kills = 2 * (int64_t)s + (lane >> 5) < k_tiles ? 0u : VFA_OOB;
    if (wave < 2) {
      lds_dma16(rs, dst_s + slot, (s_base_any + (uint32_t)s * 1024) | kills);
    } else if constexpr (A4) {
      lds_dma16(ras, dst_as + slot, (s_base_any + (uint32_t)s * 1024) | kills);
    }
  };
  auto issue = [&](int j, int s, auto use_s) {
    if constexpr (use_s)
      issue_s(j, s);
    else
      issue_v(j, s);
  };

  const int fr = lane & 31, fh = lane >> 5;
  const int asw = lds_swizzle(fr), wsw = (fr >> 2) & 3;
  struct Raw {
    v4i a[MB][A4 ? 1 : 2];
    uint32_t as[A4 ? MB : 1];
    v4i w[NB];
    uint32_t s[NB];
  };
  // The packed operands of 64-K half u of the stage in slot j.
  auto read_raw = [&](Raw& r, int j, auto u) {
    const uint8_t* base = ring + j * FP4_SLOT;
    static_for<MB>([&](auto mb) {
      if constexpr (A4) {
        const uint8_t* row = base + (wm * 128 + mb * 32 + fr) * 64;
        r.a[mb][0] = *reinterpret_cast<const v4i*>(row + (((2 * u + fh) ^ wsw) << 4));
        r.as[mb] = *reinterpret_cast<const uint32_t*>(base + OFF_AS + wm * 1024 + u * 512 +
                                                      fr * 16 + mb * 4);
      } else {
        const uint8_t* row = base + (wm * 128 + mb * 32 + fr) * 128;
        r.a[mb][0] = *reinterpret_cast<const v4i*>(row + (((4 * u + 2 * fh) ^ asw) << 4));
        r.a[mb][1] = *reinterpret_cast<const v4i*>(row + (((4 * u + 2 * fh + 1) ^ asw) << 4));
      }
    });
    static_for<NB>([&](auto nb) {
      const uint8_t* row = base + OFF_W + (wn * 128 + nb * 32 + fr) * 64;
      r.w[nb] = *reinterpret_cast<const v4i*>(row + (((2 * u + fh) ^ wsw) << 4));
      r.s[nb] = *reinterpret_cast<const uint32_t*>(base + OFF_WS + wn * 1024 + u * 512 +
                                                   fr * 16 + nb * 4);
    });
  };

  v16f acc[NB][MB];
  static_for<NB>([&](auto i) { static_for<MB>([&](auto jj) { acc[i][jj] = v16f{}; }); });
  // Block scales of the current half as binary16: a lane's two 16-K blocks of
  // the half (bytes 2 fh and 2 fh + 1 of the row's scale word), converted by
  // one instruction at the half's first step; step v multiplies by element
  // v / 2, broadcast to both halves of the packed multiply.
  v2h scw[NB], sca[A4 ? MB : 1];
  // Binary16 operands of MFMA step v (0..3) of a half held in r.
  struct Ops {
    v8h xa[MB], xw[NB];
  };
  auto convert = [&](const Raw& r, auto v) {
    Ops o;
    // E4M3 block scales (bytes 2*fh, 2*fh + 1 of the row's scale word), exact in binary16.
    auto scale_pair = [&](uint32_t sword) {
      return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sword >> (16 * fh), 1.0f, false);
    };
    if constexpr (v == 0) {
      static_for<NB>([&](auto nb) { scw[nb] = scale_pair(r.s[nb]); });
      if constexpr (A4) static_for<MB>([&](auto mb) { sca[mb] = scale_pair(r.as[mb]); });
    }
    // Eight E2M1 values of packed word d times their block scale (element v / 2
    // of sc2), exact in binary16.
    auto fp4x8 = [&](uint32_t d, v2h sc2) {
      const v2h sc = v2h{sc2[v / 2], sc2[v / 2]};
      const v2h y0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 0) * sc;
      const v2h y1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 1) * sc;
      const v2h y2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 2) * sc;
      const v2h y3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.0f, 3) * sc;
      return v8h{y0[0], y0[1], y1[0], y1[1], y2[0], y2[1], y3[0], y3[1]};
    };
    static_for<MB>([&](auto mb) {
      if constexpr (A4) {
        o.xa[mb] = fp4x8((uint32_t)r.a[mb][0][(int)v], sca[mb]);
      } else {
        const uint32_t d0 = (uint32_t)r.a[mb][v / 2][(v % 2) * 2];
        const uint32_t d1 = (uint32_t)r.a[mb][v / 2][(v % 2) * 2 + 1];
        const v2h x0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false);
        const v2h x1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true);
        const v2h x2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false);
        const v2h x3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true);
        o.xa[mb] = v8h{x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], x3[0], x3[1]};
      }
    });
    static_for<NB>([&](auto nb) { o.xw[nb] = fp4x8((uint32_t)r.w[nb][(int)v], scw[nb]); });
    return o;
  };
  // The MFMAs of one step, with the dequantization of the next step (nxt, from
  // half r, step v) interleaved: one MFMA, then three VALU instructions (four
  // with E2M1 activations, whose dequantization is longer), so the VALU work
  // runs while the MFMA pipe is busy instead of between its bursts.
  auto pipelined = [&](const Ops& cur, const Raw& r, auto v) {
    const Ops nxt = convert(r, v);
    static_for<NB>([&](auto nb) {
      static_for<MB>([&](auto mb) {
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.xw[nb], cur.xa[mb], acc[nb][mb], 0, 0, 0);
      });
    });
    static_for<NB * MB>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, A4 ? 4 : 3, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
    return nxt;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  Raw r0, r1;
  stage_vectors<256, 256>(p, m0, n0, wave, lane, __builtin_amdgcn_readfirstlane(lds_addr(vec)));
  auto run = [&](auto use_s) {
    issue(0, 0, use_s);
    issue(1, 1, use_s);
    wait_vmcnt<0, true>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_raw(r0, 0, I0{});
    // Same pending LDS reads on both loop entries (see the W8A8 kernel).
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    // Software pipeline: cur holds the converted operands of the next MFMA step.
    Ops cur = convert(r0, I0{});
    // Stage kt in slot jc (a constant: the loop runs two stages per trip, so
    // every LDS read address is a loop-invariant register plus an immediate).
    auto stage = [&](int kt, auto jc) {
      constexpr int j = jc;
      read_raw(r1, j, I1{});
      cur = pipelined(cur, r0, I1{});
      cur = pipelined(cur, r0, I2{});
      cur = pipelined(cur, r0, I3{});
      cur = pipelined(cur, r1, I0{});
      cur = pipelined(cur, r1, I1{});
      // Stage kt+1 has landed for every wave and stage kt is fully read.
      wait_vmcnt<0, true>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      issue(j, kt + 2, use_s);
      read_raw(r0, 1 - j, I0{});
      cur = pipelined(cur, r1, I2{});
      cur = pipelined(cur, r1, I3{});
      // Half 0 of stage kt+1 (zeros past the last stage, never multiplied).
      cur = pipelined(cur, r0, I0{});
    };
    for (int kt = 0; kt < KT; kt += 2) {
      stage(kt, I0{});
      if (kt + 1 < KT) stage(kt + 1, I1{});
    }
  };
  if (full)
    run(std::true_type{});
  else
    run(std::false_type{});
  wait_vmcnt<0, true>();  // every DMA has landed before the ring becomes the staging tile
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  gemm_epilogue<256, 256, 2, 2, EPI_BIAS, true, true>(p, acc, m0, n0, wm, wn, (int)threadIdx.x, ring,
                                                    vec);
}

hipError_t launch_nvfp4_w4a4(const uint8_t* a, int64_t lda, const uint8_t* as, const uint8_t* w,
                             const uint8_t* ws, const float* alpha, int64_t m, int64_t n, int64_t k,
                             const uint16_t* bias, uint16_t* out, int64_t ldo, int group_m,
                             hipStream_t s) {
  GemmParams g{};
  g.a = a;
  g.sa = nullptr;  // no per-row scale: the epilogue's row factor is 1
  g.lda = lda;
  g.asb = as;
  g.w = w;
  g.ldw = k / 2;
  g.wsb = ws;
  g.sw = alpha;
  g.sw_step = 0;
  g.m = m;
  g.n = n;
  g.k = k;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.group_m = group_m;
  const int64_t tiles = ((m + 255) / 256) * ((n + 255) / 256);
  nvfp4_gemm_pipe<true><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(g);
  return hipGetLastError();
}

hipError_t launch_nvfp4(const uint8_t* a, const float* sa, int64_t lda, const uint8_t* w,
                        const uint8_t* ws, const float* alpha, int64_t m, int64_t n, int64_t k,
                        const uint16_t* bias, uint16_t* out, int64_t ldo, int group_m,
                        hipStream_t s) {
  GemmParams g{};
  g.a = a;
  g.sa = sa;
  g.lda = lda;
  g.w = w;
  g.ldw = k / 2;
  g.wsb = ws;
  g.sw = alpha;
  g.sw_step = 0;
  g.m = m;
  g.n = n;
  g.k = k;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.group_m = group_m;
  const int64_t tiles = ((m + 255) / 256) * ((n + 255) / 256);
  nvfp4_gemm_pipe<false><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(g);
  return hipGetLastError();
}

}  // namespace vfa
