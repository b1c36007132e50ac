// W8A8 E4M3 GEMM with fused epilogues for gfx950 (CDNA4).
//
//   acc[m, n] = sum_k A[m, k] * W[n, k]          (E4M3 x E4M3, binary32 accumulate)
//   base      = bf16(bf16(acc * sa[m] * sw[n]) + bias[n])
//
// This replaces torch._scaled_mm(codes, weight.t(), scale_a, scale_b, bf16)
// followed by the separate "+ bias" of RowFP8Execution.linear
// (reference src/vflash/native/h3_fp8_linear.py:109-121); the two bf16
// roundings are kept in that order.  Epilogue variants:
//   EPI_BIAS   out = base                                   (also merged QKV planes)
//   EPI_GATE   out = bf16(residual + bf16(gate * base))
//              (h3_fused_ops.py:124-170 strict_gate_residual_kernel)
//   EPI_LORA   out = bf16(base + delta), delta = bf16(t . B^T) with the optional
//              bf16(delta * scale), bf16(delta * strength) steps
//              (adapters/h3_reference_lora.py:75-90)
//   EPI_SWIGLU h = bf16(value * bf16(silu(gate))) with value = base[:, f] and
//              gate = base[:, half_n + f], plus per-row |h| maxima per 128
//              columns (h3_native_denoiser.py:369-376, h3_fused_ops.py:184-224)
//
// Tiling: a workgroup of WGM x WGN waves computes a BM x BN tile; each wave
// owns (BM/WGM) x (BN/WGN) as 32x32 blocks of v_mfma_f32_32x32x64_f8f6f4.
// The weight fragment is MFMA operand A and the activation fragment operand B,
// so a lane's accumulator holds 4 consecutive output columns of one row.
// K advances 128 bytes per stage; A/W tiles are double buffered in LDS with a
// 16-byte-chunk XOR swizzle (lds_swizzle) so that ds_read_b128 of consecutive
// rows touches distinct bank groups.
#include "gemm_epilogue.h"

namespace vfa {

template <int BM, int BN, int WGM, int WGN, int EPI>
__global__ void __launch_bounds__(64 * WGM * WGN) fp8_gemm_kernel(const GemmParams p) {
  constexpr int NT = 64 * WGM * WGN;         // threads per workgroup
  constexpr int BK = 128;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MB = WM / 32, NB = WN / 32;
  constexpr int ACH = BM * (BK / 16) / NT;  // 16-byte chunks per thread, A tile
  constexpr int WCH = BN * (BK / 16) / NT;  // 16-byte chunks per thread, W tile
  constexpr int RSTEP = NT / 8;             // rows between a thread's chunks
  constexpr int STAGE = (BM + BN) * BK;
  static_assert(ACH >= 1 && WCH >= 1 && MB >= 1 && NB >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tiles_m = (int)((p.m + BM - 1) / BM);
  const int tiles_n = (int)((p.n + BN - 1) / BN);
  int tm, tn;
  tile_coords(tiles_m, tiles_n, p.group_m, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;

  // Buffer resources span only this tile's rows: every offset fits 31 bits,
  // and rows past the matrix edge read as zero.
  const int64_t rows_a = min((int64_t)BM, p.m - m0);
  const int64_t rows_w = min((int64_t)BN, p.n - n0);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w + n0 * p.ldw, (uint32_t)(rows_w * p.ldw));

  const int c = tid & 7;        // 16-byte chunk of the 128-byte K slice
  const int r0 = tid >> 3;      // rows r0 + RSTEP i of the tile
  const int pc = c ^ lds_swizzle(r0);  // swizzled chunk slot (RSTEP % 16 == 0)
  const uint32_t a_off0 = (uint32_t)(r0 * p.lda + c * 16);
  const uint32_t w_off0 = (uint32_t)(r0 * p.ldw + c * 16);
  const uint32_t a_step = (uint32_t)(RSTEP * p.lda), w_step = (uint32_t)(RSTEP * p.ldw);
  const int KT = (int)((p.k + BK - 1) / BK);
  const int k_full = (int)(p.k / BK);  // stages with no K tail

  v4i va[ACH], vw[WCH];
  // Stage kt -> registers.  Only the tail stage (uniform branch) masks chunks
  // past K, by pointing them beyond the buffer range so they read as zero.
  auto gload = [&](int kt) {
    const uint32_t kb = (uint32_t)kt * BK;
    if (kt < k_full) {
      static_for<ACH>([&](auto i) {
        va[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off0 + i * a_step + kb, 0, 0);
      });
      static_for<WCH>([&](auto i) {
        vw[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_off0 + i * w_step + kb, 0, 0);
      });
    } else {
      const uint32_t kill = ((int64_t)kb + c * 16 < p.k) ? 0u : VFA_OOB;
      static_for<ACH>([&](auto i) {
        va[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, (a_off0 + i * a_step + kb) | kill, 0, 0);
      });
      static_for<WCH>([&](auto i) {
        vw[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, (w_off0 + i * w_step + kb) | kill, 0, 0);
      });
    }
  };
  auto sstore = [&](int buf) {
    uint8_t* sa = smem + buf * STAGE;
    uint8_t* sw = sa + BM * BK;
    static_for<ACH>([&](auto i) {
      *reinterpret_cast<v4i*>(sa + (r0 + RSTEP * i) * BK + pc * 16) = va[i];
    });
    static_for<WCH>([&](auto i) {
      *reinterpret_cast<v4i*>(sw + (r0 + RSTEP * i) * BK + pc * 16) = vw[i];
    });
  };

  v16f acc[NB][MB];
  static_for<NB>([&](auto i) { static_for<MB>([&](auto j) { acc[i][j] = v16f{}; }); });

  const int fr = lane & 31;  // fragment row within a 32-row block
  const int fh = lane >> 5;  // which 32-byte half of the 64-byte K step
  const int sw7 = lds_swizzle(fr);  // block rows start at multiples of 32
  auto compute = [&](int buf) {
    const uint8_t* sa = smem + buf * STAGE + (wm * WM + fr) * BK;
    const uint8_t* sw = smem + buf * STAGE + BM * BK + (wn * WN + fr) * BK;
    static_for<2>([&](auto ks) {
      const int cc = ks * 4 + fh * 2;
      const int o0 = ((cc ^ sw7) << 4), o1 = (((cc + 1) ^ sw7) << 4);
      v8i xf[MB], wf[NB];
      static_for<MB>([&](auto mb) {
        v4i lo = *reinterpret_cast<const v4i*>(sa + mb * 32 * BK + o0);
        v4i hi = *reinterpret_cast<const v4i*>(sa + mb * 32 * BK + o1);
        xf[mb] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      });
      static_for<NB>([&](auto nb) {
        v4i lo = *reinterpret_cast<const v4i*>(sw + nb * 32 * BK + o0);
        v4i hi = *reinterpret_cast<const v4i*>(sw + nb * 32 * BK + o1);
        wf[nb] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      });
      static_for<NB>([&](auto nb) {
        static_for<MB>([&](auto mb) {
          acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              wf[nb], xf[mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
        });
      });
    });
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    compute(kt & 1);
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

  gemm_epilogue<BM, BN, WGM, WGN, EPI>(p, acc, m0, n0, wm, wn, tid, smem);
}

// ---------------------------------------------------------------------------
// Two-slot pipelined 256x256 main loop with 128-byte K stages.
//
// Each stage holds 128 bytes of K for all 256 A rows and 256 W rows (64 KB);
// two LDS slots alternate.  The DMA reads whole 128-byte row segments (eight
// lanes per row), which moves L2 data into LDS markedly faster than 64-byte
// segments.  Per stage kt, per wave (2x2 waves, 128x128 each):
//   16 MFMAs of K-substep 0, interleaved with the LDS reads of substep 1;
//   8 MFMAs of substep 1;
//   wait for this wave's DMA of stage kt+1 and its own LDS reads, s_barrier;
//   issue the DMA of stage kt+2 into the slot of stage kt (fully read now);
//   8 MFMAs of substep 1, interleaved with the reads of stage kt+1 substep 0.
// The DMA of a stage is issued about one stage of MFMA work before it is
// needed; rows are stored with the lds_swizzle chunk permutation.
// Ring bytes of the two-slot pipeline for a BT x BT tile (BT = 256 or 128).
constexpr int pipe2_lds(int bt, int ns = 2) { return ns * 2 * bt * 128; }
constexpr int PIPE2_LDS = pipe2_lds(256);  // two 64 KB stage slots

// NS stage slots: the DMA of stage kt + NS is issued once stage kt is read,
// so NS - 1 stages are in flight while one is multiplied.
// PRE: MFMAs of K-substep 1 issued before the stage barrier (-1: half of them);
// the DMA of the next stage is spread over the remaining ones.
// SDMA: K % 128 == 0; in full tiles the DMA advances K through the scalar
// offset and kills stages past the end by switching to an empty buffer
// resource, so issuing a DMA instruction costs no vector instruction.
template <int EPI, int BT = 256, int NS = 2, int PRE = -1, bool SDMA = false>
__device__ __forceinline__ void pipe2_tile(const GemmParams& p, int tm, int tn, uint8_t* ring,
                                           uint32_t ring_lds, uint8_t* vec, uint32_t vec_lds,
                                           int wave) {
  constexpr int BM = BT, BN = BT, BK = 128, WGM = 2, WGN = 2;
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr int HALF = BM * BK;            // one operand of one stage (32 KB at BT = 256)
  constexpr int SLOT = 2 * HALF;
  constexpr int DMA_A = HALF / 1024 / 4;   // one-KB DMA instructions per wave per operand
  constexpr int DMA = 2 * DMA_A;           // per wave per stage
  static_assert(NS * SLOT == pipe2_lds(BT, NS), "slot layout");
  static_assert(NS >= 2 && (NS - 1) * DMA < 64, "vmcnt range");
  static_assert(DMA_A % 2 == 0, "A blocks alternate between the two swizzle parities");

  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (EPI == EPI_SWIGLU ? BN / 2 : BN);
  // The lane index comes from mbcnt and the wave index arrives as a scalar.
  const int lane = (int)__builtin_amdgcn_mbcnt_hi(-1, __builtin_amdgcn_mbcnt_lo(-1, 0));
  const int tid_v = wave * 64 + lane;
  const int wm = wave % WGM, wn = wave / WGM;

  const int64_t rows_a = min((int64_t)BM, p.m - m0);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
  __amdgpu_buffer_rsrc_t rw;
  // A tile whose A and W rows all lie inside the operands.  Only such tiles use
  // the scalar-offset DMA: it puts the 16-row block step in soffset, which the
  // buffer range check does not cover, so in a partial tile it would read rows
  // past the operand's end.  Partial tiles keep every row step in the lane
  // offset, where the range check turns rows past the end into zeros.
  bool full = rows_a == BM;
  if constexpr (EPI == EPI_SWIGLU) {
    // Waves 0-1 load tile rows 0..BN/2-1 = value rows n0.., waves 2-3 load tile
    // rows BN/2.. = gate rows half_n + n0.. (the resource is based BN/2 rows
    // earlier, so tile row r maps to half_n + n0 + r - BN/2).
    static_assert(DMA_A * 8 * 2 == BN / 2, "each wave loads rows of one half");
    const int64_t rows_h = min((int64_t)(BN / 2), p.half_n - n0);
    full = full && rows_h == BN / 2;
    if (wave < 2)
      rw = make_rsrc(p.w + n0 * p.ldw, (uint32_t)(rows_h * p.ldw));
    else
      rw = make_rsrc(p.w + (p.half_n + n0 - BN / 2) * p.ldw, (uint32_t)((BN / 2 + rows_h) * p.ldw));
  } else {
    const int64_t rows_w = min((int64_t)BN, p.n - n0);
    full = full && rows_w == BN;
    rw = make_rsrc(p.w + n0 * p.ldw, (uint32_t)(rows_w * p.ldw));
  }
  // Wave-uniform in the compiler's analysis (the tile coordinates are).
  full = __builtin_amdgcn_readfirstlane((int)full) != 0;

  // DMA lane map: 1 KB block b of an operand holds rows 8b..8b+7; lane l fills
  // row 8b + l/8, slot l%8, from logical chunk (l%8) ^ lds_swizzle(row).  The
  // swizzle depends on row % 16, i.e. on the parity of b, so two chunk values
  // and two base offsets per operand cover all of a wave's blocks.
  const int drow = lane >> 3;
  const int dch0 = (lane & 7) ^ lds_swizzle(drow), dch1 = (lane & 7) ^ lds_swizzle(drow + 8);
  const int row0 = wave * DMA_A * 8 + drow;
  const uint32_t a_base0 = (uint32_t)(row0 * p.lda + dch0 * 16);
  const uint32_t a_base1 = (uint32_t)((row0 + 8) * p.lda + dch1 * 16);
  const uint32_t w_base0 = (uint32_t)(row0 * p.ldw + dch0 * 16);
  const uint32_t w_base1 = (uint32_t)((row0 + 8) * p.ldw + dch1 * 16);
  const uint32_t a_step = (uint32_t)(16 * p.lda), w_step = (uint32_t)(16 * p.ldw);
  const int KT = (int)((p.k + BK - 1) / BK);
  const uint32_t wave_lds = ring_lds + wave * DMA_A * 1024;

  // DMA of stage s into slot j: instruction i < DMA_A is A block i, the rest W
  // blocks; chunks past K (and whole stages past the end) read as zeros.
  struct Dma {
    uint32_t base, kb, kill0, kill1;
  };
  auto dma_setup = [&](int j, int s) {
    const uint32_t kb = (uint32_t)s * BK;
    return Dma{wave_lds + j * SLOT, kb, ((int64_t)kb + dch0 * 16 < p.k) ? 0u : VFA_OOB,
               ((int64_t)kb + dch1 * 16 < p.k) ? 0u : VFA_OOB};
  };
  auto dma_one = [&](const Dma& d, auto i) {
    if constexpr (i < DMA_A) {
      const uint32_t off = (i % 2 ? a_base1 : a_base0) + (i / 2) * a_step + d.kb;
      lds_dma16(ra, d.base + i * 1024, off | (i % 2 ? d.kill1 : d.kill0));
    } else {
      constexpr int w = i - DMA_A;
      const uint32_t off = (w % 2 ? w_base1 : w_base0) + (w / 2) * w_step + d.kb;
      lds_dma16(rw, d.base + HALF + w * 1024, off | (w % 2 ? d.kill1 : d.kill0));
    }
  };
  // Scalar-offset form (SDMA): resources are selected per stage.
  const __amdgpu_buffer_rsrc_t ra_none = make_rsrc(p.a, 0u), rw_none = make_rsrc(p.w, 0u);
  struct SDma {
    __amdgpu_buffer_rsrc_t ra, rw;
    uint32_t base, kb;
  };
  auto sdma_setup = [&](int j, int s) {
    const bool live = s < KT;
    return SDma{live ? ra : ra_none, live ? rw : rw_none, wave_lds + j * SLOT,
                live ? (uint32_t)s * BK : 0u};
  };
  auto sdma_one = [&](const SDma& d, auto i) {
    if constexpr (i < DMA_A) {
      lds_dma16_so(d.ra, d.base + i * 1024, i % 2 ? a_base1 : a_base0, d.kb + (i / 2) * a_step);
    } else {
      constexpr int w = i - DMA_A;
      lds_dma16_so(d.rw, d.base + HALF + w * 1024, w % 2 ? w_base1 : w_base0,
                   d.kb + (w / 2) * w_step);
    }
  };
  auto issue = [&](int j, int s, auto use_sdma) {
    if constexpr (use_sdma) {
      const SDma d = sdma_setup(j, s);
      static_for<DMA>([&](auto i) { sdma_one(d, i); });
    } else {
      const Dma d = dma_setup(j, s);
      static_for<DMA>([&](auto i) { dma_one(d, i); });
    }
  };

  const int fr = lane & 31, fh = lane >> 5;
  const int fsw = lds_swizzle(fr);
  v8i F[2][MB + NB];  // [K-substep][activation blocks, then weight blocks]
  // Fragments of K-substep ks of the stage in slot j into register set ks.
  auto read_one = [&](int j, auto ks, auto f) {
    const int cc = ks * 4 + fh * 2;
    const int o0 = (cc ^ fsw) << 4, o1 = ((cc + 1) ^ fsw) << 4;
    const uint8_t* src = f < MB ? ring + j * SLOT + (wm * WM + fr) * BK + f * 32 * BK
                                : ring + j * SLOT + HALF + (wn * WN + fr) * BK + (f - MB) * 32 * BK;
    const v4i lo = *reinterpret_cast<const v4i*>(src + o0);
    const v4i hi = *reinterpret_cast<const v4i*>(src + o1);
    F[ks][f] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto read = [&](int j, auto ks) { static_for<MB + NB>([&](auto f) { read_one(j, ks, f); }); };
  v16f acc[NB][MB];
  static_for<NB>([&](auto i) { static_for<MB>([&](auto jj) { acc[i][jj] = v16f{}; }); });
  // MFMAs number q0..q1-1 of K-substep ks (q = nb * MB + mb).
  auto mfmas = [&](auto ks, auto q0, auto q1) {
    static_for<q1 - q0>([&](auto qq) {
      constexpr int q = q0 + qq, nb = q / MB, mb = q % MB;
      acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          F[ks][MB + nb], F[ks][mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
    });
  };
  auto interleave = [&](auto n) {  // pair each of n MFMAs with one LDS read
    static_for<n>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    });
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  constexpr int Q = MB * NB, QB = PRE < 0 ? Q / 2 : PRE, QA = Q - QB;
  constexpr int RD = 2 * (MB + NB);  // ds_read_b128 per K-substep
  static_assert(QA > 0 && DMA % QA == 0, "DMA instructions spread evenly after the barrier");

  // 128x128 LoRA tiles compute their adapter products before the K loop (64
  // registers); the 256x256 tiles, whose registers hold the main loop, compute
  // them in the epilogue.
  constexpr bool LORA_PRE = EPI == EPI_LORA && BT == 128;
  v16f lora_d[LORA_PRE ? MB * NB : 1];
  if constexpr (LORA_PRE) lora_blocks<BM, BN, WGM, WGN>(p, m0, n0, wm, wn, lane, lora_d);
  // Prologue and K loop; use_sdma selects the scalar-offset DMA (full tiles).
  auto main_loop = [&](auto use_sdma) {
    stage_vectors<BM, BN, EPI == EPI_SWIGLU>(p, m0, n0, wave, lane, vec_lds);
    static_for<NS>([&](auto s) { issue((int)s, (int)s, use_sdma); });
    wait_vmcnt<(NS - 1) * DMA, true>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read(I0{}, I0{});
    // The first fragments have landed before the loop: the compiler's wait
    // tracking then sees the same pending LDS reads on both loop entries and
    // waits only for the fragments each MFMA needs.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt untouched
    int j = 0;  // slot of stage kt
    for (int kt = 0; kt < KT; ++kt) {
      const int jn = j + 1 == NS ? 0 : j + 1;  // slot of stage kt + 1
      // Substep 0 of stage kt, while reading substep 1 of the same stage.
      mfmas(I0{}, I0{}, std::integral_constant<int, Q>{});
      read(j, I1{});
      interleave(std::integral_constant<int, (RD < Q ? RD : Q)>{});
      mfmas(I1{}, I0{}, std::integral_constant<int, QB>{});
      // The MFMAs above stay above the wait (they keep the MFMA pipe busy while
      // the wave waits); scheduling barriers pin the order.
      __builtin_amdgcn_sched_barrier(0);
      // Stage kt+1 has landed for every wave (the DMAs of stages kt+2 ..
      // kt+NS-1 may still be in flight); stage kt is fully read.
      wait_vmcnt<(NS - 2) * DMA, true>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // Second half: each remaining MFMA is followed by DMA / QH of the DMA
      // instructions of stage kt+2 and by the reads of one fragment of stage kt+1
      // (unused after the last stage), so DMA issue and reads overlap the MFMA pipe.
      const Dma d = dma_setup(j, kt + NS);
      const SDma sd = sdma_setup(j, kt + NS);
      static_for<QA>([&](auto i) {
        constexpr int q = QB + i, nb = q / MB, mb = q % MB;
        acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            F[1][MB + nb], F[1][mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
        static_for<DMA / QA>([&](auto t) {
          constexpr int di = i * (DMA / QA) + t;
          if constexpr (use_sdma)
            sdma_one(sd, std::integral_constant<int, di>{});
          else
            dma_one(d, std::integral_constant<int, di>{});
        });
        if constexpr (i < MB + NB) read_one(jn, I0{}, i);
        __builtin_amdgcn_sched_barrier(0);
      });
      // Fragments not covered above (smaller tiles have fewer MFMAs than fragments).
      static_for<(MB + NB > QA ? MB + NB - QA : 0)>([&](auto i) {
        read_one(jn, I0{}, std::integral_constant<int, QA + i>{});
      });
      j = jn;
    }
  };
  if constexpr (SDMA) {
    if (full)
      main_loop(std::true_type{});
    else
      main_loop(std::false_type{});
  } else {
    main_loop(std::false_type{});
  }
  wait_vmcnt<0, true>();  // every DMA has landed before the ring is reused
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  gemm_epilogue<BM, BN, WGM, WGN, EPI, true>(p, acc, m0, n0, wm, wn, tid_v, ring, vec,
                                             LORA_PRE ? lora_d : nullptr);
}

template <int EPI, int PRE = -1, bool SDMA = false>
__global__ void __launch_bounds__(256) fp8_gemm_pipe2(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[PIPE2_LDS];
  __shared__ __attribute__((aligned(1024))) uint8_t vec[VEC_LDS];
  int tm, tn;
  // SwiGLU tiles cover 128 value columns and their 128 gate columns.
  const int64_t tile_cols = EPI == EPI_SWIGLU ? (p.half_n + 127) / 128 : (p.n + 255) / 256;
  tile_coords((int)((p.m + 255) / 256), (int)tile_cols, p.group_m, tm, tn);
  pipe2_tile<EPI, 256, 2, PRE, SDMA>(p, tm, tn, ring,
                                     __builtin_amdgcn_readfirstlane(lds_addr(ring)), vec,
                                     __builtin_amdgcn_readfirstlane(lds_addr(vec)),
                                     __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6));
}

// 128 x 128 form for shapes with too few 256 x 256 tiles to fill the GPU: the
// same pipeline with 64 x 64 per wave (64 accumulator registers), so that two
// workgroups share a CU and each hides the other's DMA latency and epilogue.
template <int EPI, int NS, int PRE = -1, bool SDMA = false>
__global__ void __launch_bounds__(256, NS == 2 ? 2 : 1) fp8_gemm_pipe2s(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[pipe2_lds(128, NS)];
  __shared__ __attribute__((aligned(1024))) uint8_t vec[VEC_LDS];
  int tm, tn;
  tile_coords((int)((p.m + 127) / 128), (int)((p.n + 127) / 128), p.group_m, tm, tn);
  pipe2_tile<EPI, 128, NS, PRE, SDMA>(p, tm, tn, ring, __builtin_amdgcn_readfirstlane(lds_addr(ring)), vec,
                           __builtin_amdgcn_readfirstlane(lds_addr(vec)),
                           __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6));
}

template <int EPI, int PRE = -1, bool SDMA = false>
static hipError_t launch_pipe2(const GemmParams& p, hipStream_t s) {
  const int64_t tile_cols = EPI == EPI_SWIGLU ? (p.half_n + 127) / 128 : (p.n + 255) / 256;
  const int64_t tiles = ((p.m + 255) / 256) * tile_cols;
  fp8_gemm_pipe2<EPI, PRE, SDMA><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

template <int EPI, int NS, int PRE = -1, bool SDMA = false>
static hipError_t launch_pipe2s(const GemmParams& p, hipStream_t s) {
  const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128);
  fp8_gemm_pipe2s<EPI, NS, PRE, SDMA><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int EPI>
static hipError_t launch_cfg(const GemmParams& p, hipStream_t s) {
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  fp8_gemm_kernel<BM, BN, WGM, WGN, EPI><<<dim3((unsigned)tiles), dim3(64 * WGM * WGN), 0, s>>>(p);
  return hipGetLastError();
}

int compute_units();

// The three tilings and the rule that picks one from the shape alone:
//   GEMM_TILE_64:  register-staged 64x64 tiles, for grids of fewer than 256
//                  tiles of 128x128;
//   GEMM_TILE_128: the two-slot pipeline on 128x128 tiles (2x2 waves of 64x64),
//                  two workgroups per CU;
//   GEMM_TILE_256: the two-slot pipeline on 256x256 tiles (2x2 waves of
//                  128x128), barrier after K-substep 0, scalar-offset DMA in
//                  full tiles when K % 128 == 0; one workgroup per CU.
// Between the last two, whichever needs fewer rounds of tiles, a 128x128 round
// counting 0.5 x 1.15 of a 256x256 round (a quarter of the work at two per CU,
// at the 128x128 tile's lower efficiency).  The model gives the measured
// ratios: 1.16 in favour of 256x256 at 4096x3072x3072 (192 against 768 tiles)
// and 1.74 in favour of 128x128 at M=1024, K=1536, N=6144 (96 against 384
// tiles).  Every tiling multiplies each output's K stages in the same order
// with the same MFMA and shares the epilogue, so the choice never changes a
// result bit.
enum { GEMM_TILE_64 = 0, GEMM_TILE_128 = 1, GEMM_TILE_256 = 2 };

int pick_tile(const GemmParams& p) {
  auto tiles = [&](int bm, int bn) { return ((p.m + bm - 1) / bm) * ((p.n + bn - 1) / bn); };
  const int64_t t128 = tiles(128, 128), t256 = tiles(256, 256), cus = compute_units();
  if (t128 < 256) return GEMM_TILE_64;
  const double rounds256 = (double)((t256 + cus - 1) / cus);
  const double rounds128 = (double)((t128 + 2 * cus - 1) / (2 * cus)) * 0.5 * 1.15;
  return rounds256 <= rounds128 ? GEMM_TILE_256 : GEMM_TILE_128;
}

template <int EPI>
hipError_t launch_epi(const GemmParams& p, int tile, hipStream_t s) {
  switch (tile) {
    case GEMM_TILE_64: return launch_cfg<64, 64, 2, 2, EPI>(p, s);
    case GEMM_TILE_128: return launch_pipe2s<EPI, 2>(p, s);
    case GEMM_TILE_256:
      return p.k % 128 ? launch_pipe2<EPI, 0, false>(p, s) : launch_pipe2<EPI, 0, true>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Compute units of the current device (cached per device id).
int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

hipError_t launch_fp8_gemm(const GemmParams& p, int epi, hipStream_t s) {
  const int tile = pick_tile(p);
  switch (epi) {
    case EPI_BIAS: return launch_epi<EPI_BIAS>(p, tile, s);
    case EPI_GATE: return launch_epi<EPI_GATE>(p, tile, s);
    case EPI_LORA: return launch_epi<EPI_LORA>(p, tile, s);
    case EPI_SWIGLU:  // one tiling: 128 value + 128 gate columns, the 256x256 schedule
      return p.k % 128 ? launch_pipe2<EPI_SWIGLU, 0, false>(p, s)
                       : launch_pipe2<EPI_SWIGLU, 0, true>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vfa
