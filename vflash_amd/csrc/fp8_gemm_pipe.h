// Pipelined W8A8 E4M3 GEMM tile for gfx950 (CDNA4), shared by the
// translation units that instantiate it per epilogue (fp8_gemm_*.hip).
// Kernel-side only; not part of the C-ABI.
//
//   acc[m, n] = sum_k A[m, k] * W[n, k]          (E4M3 x E4M3, binary32 accumulate)
//   base      = bf16(bf16(acc * sa[m] * sw[n]) + bias[n])
//
// A workgroup of 2x2 waves computes a BM x BN tile; each wave owns
// (BM/2) x (BN/2) as 32x32 blocks of v_mfma_f32_32x32x64_f8f6f4.  The weight
// fragment is MFMA operand A and the activation fragment operand B, so a
// lane's accumulator holds 4 consecutive output columns of one row.  K
// advances 128 bytes per stage, always from k = 0 upwards in 64-byte MFMA
// steps: every tile shape multiplies each output's K stages in the same order
// with the same MFMA and shares the epilogue, so the tiling never changes a
// result bit.
#pragma once
#include "gemm_epilogue.h"

namespace vfa {

// ---------------------------------------------------------------------------
// Pipelined BM x BN main loop with 128-byte K stages in an NS-slot LDS ring.
//
// Each stage holds 128 bytes of K for the tile's BM activation rows and BN
// weight rows; NS slots rotate.  The DMA reads whole 128-byte row segments
// (eight lanes per row), which moves L2 data into LDS markedly faster than
// 64-byte segments.  Per stage kt, per wave (2x2 waves, BM/2 x BN/2 each):
//   the MFMAs of K-substep 0, interleaved with the LDS reads of substep 1;
//   PRE MFMAs of substep 1 (PRE < 0: half of them);
//   wait for this wave's DMA of stage kt+1 and its own LDS reads, s_barrier;
//   issue the DMA of stage kt+NS into the slot of stage kt (fully read now);
//   the remaining MFMAs of substep 1, interleaved with the DMA instructions
//   and with the reads of stage kt+1 substep 0.
// NS - 1 stages are in flight while one is multiplied; rows are stored with
// the lds_swizzle chunk permutation.
//
// NS = SPLIT_RING selects a split ring instead: two activation slots and three
// weight slots (160 KB for 256 x 256, 136 KB for 256 x 192).  The weight DMAs
// of stage kt+2 then go into the slot freed at the barrier of stage kt-1,
// issued during the first half of stage kt, and only the activation DMAs wait
// for the barrier of stage kt: the stage's DMA instructions are spread over
// both halves instead of all crowding the second.  The scale and bias vectors
// (and the SwiGLU silu table) are DMA'd during the last stage into the third
// weight slot, which the output staging tile does not cover.  With the plain
// and gate-residual epilogues the last stage ends after its first half: the
// epilogue issues the substep-1 MFMAs block by block, ahead of its phase-1
// work on each block, so they run under that VALU work.
constexpr int SPLIT_RING = 0;
// Ring bytes of an NS-slot ring (or of the split ring) for a BM x BN tile.
constexpr int pipe_lds(int bm, int bn, int ns) {
  return ns == SPLIT_RING ? (2 * bm + 3 * bn) * 128 : ns * (bm + bn) * 128;
}
// Workgroups per CU the LDS allows (at most two).
constexpr int pipe_occupancy(int bm, int bn, int ns) {
  return 2 * (pipe_lds(bm, bn, ns) + (ns == SPLIT_RING ? 0 : VEC_LDS)) <= 160 * 1024 ? 2 : 1;
}

// SDMA: K % 128 == 0; in full tiles the DMA advances K through the scalar
// offset and kills stages past the end by switching to an empty buffer
// resource, so issuing a DMA instruction costs no vector instruction.
template <int EPI, int BM, int BN, int NS, int PRE, bool SDMA>
__device__ __forceinline__ void pipe_tile(const GemmParams& p, int tm, int tn, uint8_t* ring,
                                          uint32_t ring_lds, uint8_t* vec, uint32_t vec_lds,
                                          int wave) {
  constexpr int BK = 128, WGM = 2, WGN = 2;
  constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
  constexpr bool SPLIT = NS == SPLIT_RING;
  // Split-ring tiles with the plain or gate-residual epilogue issue their last
  // K substep's MFMAs from the epilogue, under its phase-1 work; the adapter
  // and SwiGLU epilogues hold too many registers for the fragments to stay
  // live through them.
  constexpr bool EPI_OVERLAP = SPLIT && !epi_lora(EPI) && !epi_swiglu(EPI);
  constexpr int HA = BM * BK;              // activation rows of one stage
  constexpr int HW = BN * BK;              // weight rows of one stage
  constexpr int SLOT = (BM + BN) * BK;     // one stage: activation rows, then weight rows
  constexpr int DMA_A = BM / 32;           // one-KB DMA instructions per wave, activation rows
  constexpr int DMA_W = BN / 32;           // and weight rows
  constexpr int DMA = DMA_A + DMA_W;       // per wave per stage
  static_assert(MB >= 1 && NB >= 1 && WM % 32 == 0 && WN % 32 == 0, "32x32 blocks per wave");
  static_assert(SPLIT ? 2 * HA + 3 * HW == pipe_lds(BM, BN, NS) : NS * SLOT == pipe_lds(BM, BN, NS),
                "slot layout");
  static_assert(SPLIT || (NS >= 2 && (NS - 1) * DMA < 64), "vmcnt range");
  static_assert(!SPLIT || 2 * HA + 2 * HW >= BM * BN * 2, "the output staging tile leaves the "
                "third weight slot to the vectors");
  static_assert(DMA_A % 2 == 0 && DMA_W % 2 == 0,
                "blocks alternate between the two swizzle parities");

  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (epi_swiglu(EPI) ? BN / 2 : BN);
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
  if constexpr (epi_swiglu(EPI)) {
    // Waves 0-1 load tile rows 0..BN/2-1 = value rows n0.., waves 2-3 load tile
    // rows BN/2.. = gate rows half_n + n0.. (the resource is based BN/2 rows
    // earlier, so tile row r maps to half_n + n0 + r - BN/2).
    static_assert(BM == 256 && BN == 256 && DMA_W * 8 * 2 == BN / 2,
                  "each wave loads rows of one half");
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
  const int arow0 = wave * DMA_A * 8 + drow, wrow0 = wave * DMA_W * 8 + drow;
  const uint32_t a_base0 = (uint32_t)(arow0 * p.lda + dch0 * 16);
  const uint32_t a_base1 = (uint32_t)((arow0 + 8) * p.lda + dch1 * 16);
  const uint32_t w_base0 = (uint32_t)(wrow0 * p.ldw + dch0 * 16);
  const uint32_t w_base1 = (uint32_t)((wrow0 + 8) * p.ldw + dch1 * 16);
  const uint32_t a_step = (uint32_t)(16 * p.lda), w_step = (uint32_t)(16 * p.ldw);
  const int KT = (int)((p.k + BK - 1) / BK);
  const uint32_t a_lds = ring_lds + wave * DMA_A * 1024;  // this wave's activation blocks
  const uint32_t w_lds = ring_lds + wave * DMA_W * 1024;  // and weight blocks (+ slot offset)
  // Ring offsets of activation slot ja and weight slot jw: in the shared ring
  // slot j holds the activation rows, then the weight rows, of one stage; the
  // split ring has two activation slots, then three weight slots.
  auto a_slot = [](int ja) { return (uint32_t)(SPLIT ? ja * HA : ja * SLOT); };
  auto w_slot = [](int jw) { return (uint32_t)(SPLIT ? 2 * HA + jw * HW : jw * SLOT + HA); };

  // DMA of stage s into activation slot ja and weight slot jw: instruction
  // i < DMA_A is A block i, the rest W blocks; chunks past K (and whole stages
  // past the end) read as zeros.
  struct Dma {
    uint32_t aslot, wslot, kb, kill0, kill1;
  };
  auto dma_setup = [&](int ja, int jw, int s) {
    const uint32_t kb = (uint32_t)s * BK;
    return Dma{a_slot(ja), w_slot(jw), kb, ((int64_t)kb + dch0 * 16 < p.k) ? 0u : VFA_OOB,
               ((int64_t)kb + dch1 * 16 < p.k) ? 0u : VFA_OOB};
  };
  auto dma_one = [&](const Dma& d, auto i) {
    if constexpr (i < DMA_A) {
      const uint32_t off = (i % 2 ? a_base1 : a_base0) + (i / 2) * a_step + d.kb;
      lds_dma16(ra, a_lds + d.aslot + i * 1024, off | (i % 2 ? d.kill1 : d.kill0));
    } else {
      constexpr int w = i - DMA_A;
      const uint32_t off = (w % 2 ? w_base1 : w_base0) + (w / 2) * w_step + d.kb;
      lds_dma16(rw, w_lds + d.wslot + w * 1024, off | (w % 2 ? d.kill1 : d.kill0));
    }
  };
  // Scalar-offset form (SDMA): resources are selected per stage.
  const __amdgpu_buffer_rsrc_t ra_none = make_rsrc(p.a, 0u), rw_none = make_rsrc(p.w, 0u);
  struct SDma {
    __amdgpu_buffer_rsrc_t ra, rw;
    uint32_t aslot, wslot, kb;
  };
  auto sdma_setup = [&](int ja, int jw, int s) {
    const bool live = s < KT;
    return SDma{live ? ra : ra_none, live ? rw : rw_none, a_slot(ja), w_slot(jw),
                live ? (uint32_t)s * BK : 0u};
  };
  auto sdma_one = [&](const SDma& d, auto i) {
    if constexpr (i < DMA_A) {
      lds_dma16_so(d.ra, a_lds + d.aslot + i * 1024, i % 2 ? a_base1 : a_base0,
                   d.kb + (i / 2) * a_step);
    } else {
      constexpr int w = i - DMA_A;
      lds_dma16_so(d.rw, w_lds + d.wslot + w * 1024, w % 2 ? w_base1 : w_base0,
                   d.kb + (w / 2) * w_step);
    }
  };
  // DMA instructions i0 .. i1-1 of stage s.
  auto issue_range = [&](int ja, int jw, int s, auto use_sdma, auto i0, auto i1) {
    if constexpr (use_sdma) {
      const SDma d = sdma_setup(ja, jw, s);
      static_for<i1 - i0>([&](auto t) { sdma_one(d, std::integral_constant<int, i0 + t>{}); });
    } else {
      const Dma d = dma_setup(ja, jw, s);
      static_for<i1 - i0>([&](auto t) { dma_one(d, std::integral_constant<int, i0 + t>{}); });
    }
  };
  using IDA = std::integral_constant<int, DMA_A>;
  using IDMA = std::integral_constant<int, DMA>;
  auto issue = [&](int ja, int jw, int s, auto use_sdma) {
    issue_range(ja, jw, s, use_sdma, std::integral_constant<int, 0>{}, IDMA{});
  };

  const int fr = lane & 31, fh = lane >> 5;
  const int fsw = lds_swizzle(fr);
  v8i F[2][MB + NB];  // [K-substep][activation blocks, then weight blocks]
  // Fragments of K-substep ks of the stage in slots ja / jw into register set ks.
  auto read_one = [&](int ja, int jw, auto ks, auto f) {
    const int cc = ks * 4 + fh * 2;
    const int o0 = (cc ^ fsw) << 4, o1 = ((cc + 1) ^ fsw) << 4;
    // Weight block f - MB of this wave: tile rows block_col(wn, f - MB) .. +31
    // (SwiGLU tiles pair each value block with its gate block).
    const uint8_t* src =
        f < MB ? ring + a_slot(ja) + (wm * WM + fr) * BK + f * 32 * BK
               : ring + w_slot(jw) + (wave_col<BN, WN, epi_swiglu(EPI)>(wn) + fr) * BK +
                     block_off<BN, WN, epi_swiglu(EPI)>(f - MB) * BK;
    const v4i lo = *reinterpret_cast<const v4i*>(src + o0);
    const v4i hi = *reinterpret_cast<const v4i*>(src + o1);
    F[ks][f] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto read = [&](int ja, int jw, auto ks) {
    static_for<MB + NB>([&](auto f) { read_one(ja, jw, ks, f); });
  };
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
  static_assert(QA > 0, "MFMAs after the barrier carry the DMA");

  // Tiles of at most eight 32x32 blocks per wave compute their adapter products
  // before the K loop (up to 128 registers held through it), so the epilogue
  // does not wait on their loads; the 256x192 and 256x256 tiles, whose
  // registers hold the main loop, compute them in the epilogue.
  constexpr bool LORA_PRE = epi_lora(EPI) && MB * NB <= 8;
  v16f lora_d[LORA_PRE ? MB * NB : 1];
  if constexpr (LORA_PRE) lora_blocks<BM, BN, WGM, WGN, epi_swiglu(EPI)>(p, m0, n0, wm, wn, lane, lora_d);
  // Prologue and K loop; use_sdma selects the scalar-offset DMA (full tiles).
  auto main_loop = [&](auto use_sdma) {
    stage_vectors<BM, BN, epi_swiglu(EPI)>(p, m0, n0, wave, lane, vec_lds);
    static_for<NS>([&](auto s) { issue((int)s, (int)s, (int)s, use_sdma); });
    wait_vmcnt<(NS - 1) * DMA, true>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read(0, 0, I0{});
    // The first fragments have landed before the loop: the compiler's wait
    // tracking then sees the same pending LDS reads on both loop entries and
    // waits only for the fragments each MFMA needs.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt untouched
    int j = 0;  // slot of stage kt
    for (int kt = 0; kt < KT; ++kt) {
      const int jn = j + 1 == NS ? 0 : j + 1;  // slot of stage kt + 1
      // Substep 0 of stage kt, while reading substep 1 of the same stage.
      mfmas(I0{}, I0{}, std::integral_constant<int, Q>{});
      read(j, j, I1{});
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
      // Second half: each remaining MFMA is followed by its share of the DMA
      // instructions of stage kt+NS and by the reads of one fragment of stage
      // kt+1 (unused after the last stage), so DMA issue and reads overlap the
      // MFMA pipe.
      const Dma d = dma_setup(j, j, kt + NS);
      const SDma sd = sdma_setup(j, j, kt + NS);
      static_for<QA>([&](auto i) {
        constexpr int q = QB + i, nb = q / MB, mb = q % MB;
        acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            F[1][MB + nb], F[1][mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
        constexpr int d0 = i * DMA / QA, d1 = (i + 1) * DMA / QA;
        static_for<d1 - d0>([&](auto t) {
          constexpr int di = d0 + t;
          if constexpr (use_sdma)
            sdma_one(sd, std::integral_constant<int, di>{});
          else
            dma_one(d, std::integral_constant<int, di>{});
        });
        if constexpr (i < MB + NB) read_one(jn, jn, I0{}, i);
        __builtin_amdgcn_sched_barrier(0);
      });
      // Fragments not covered above (smaller tiles have fewer MFMAs than fragments).
      static_for<(MB + NB > QA ? MB + NB - QA : 0)>([&](auto i) {
        read_one(jn, jn, I0{}, std::integral_constant<int, QA + i>{});
      });
      j = jn;
    }
  };

  // The split ring's prologue and K loop.  Stage s sits in activation slot s % 2
  // and weight slot (s + c) % 3, with c = (1 - KT) mod 3 so that the last
  // stage's free weight slot, where the vectors go, is always slot 2.
  auto split_loop = [&](auto use_sdma) {
    const int c = ((1 - KT) % 3 + 3) % 3;
    issue(0, c, 0, use_sdma);
    issue(1, c == 2 ? 0 : c + 1, 1, use_sdma);
    wait_vmcnt<DMA, true>();  // stage 0 has landed (stage 1 may be in flight)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read(0, c, I0{});
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt untouched
    // One stage; `last` replaces the weight DMAs of stage kt+2 (past the end)
    // with the vectors' DMA into weight slot 2; `first` starts the accumulators
    // from the MFMAs of its substep 0 (a zero accumulator operand), so no
    // instruction zeroes them beforehand.
    auto stage = [&](int kt, int ja, int jw, auto last, auto first) {
      const int jan = ja ^ 1, jwn = jw == 2 ? 0 : jw + 1, jwf = jwn == 2 ? 0 : jwn + 1;
      // First half: the MFMAs of substep 0, each with the reads of one
      // substep-1 fragment and its share of the weight DMAs of stage kt+2 (into
      // the slot of stage kt-1, free since the last barrier).
      static_for<Q>([&](auto i) {
        constexpr int nb = i / MB, mb = i % MB;
        acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            F[0][MB + nb], F[0][mb], first ? v16f{} : acc[nb][mb], 0, 0, 0, 0, 0, 0);
        if constexpr (i < MB + NB) read_one(ja, jw, I1{}, i);
        if constexpr (!last) {
          constexpr int d0 = DMA_A + i * DMA_W / Q, d1 = DMA_A + (i + 1) * DMA_W / Q;
          issue_range(ja, jwf, kt + 2, use_sdma, std::integral_constant<int, d0>{},
                      std::integral_constant<int, d1>{});
        } else if constexpr (i == 0) {
          stage_vectors<BM, BN, epi_swiglu(EPI)>(p, m0, n0, wave, lane_id_fresh(), vec_lds);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      static_for<(MB + NB > Q ? MB + NB - Q : 0)>([&](auto i) {
        read_one(ja, jw, I1{}, std::integral_constant<int, Q + i>{});
      });
      if constexpr (last && EPI_OVERLAP) {
        // The last stage's substep-1 MFMAs are issued by the epilogue, between
        // its blocks.  Every DMA (the vectors included) has landed and the
        // ring is read: the epilogue may stage its output there.
        wait_vmcnt<0, true>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        return;
      }
      // Stage kt+1 has landed for every wave (the weight DMAs of stage kt+2 may
      // still be in flight); stage kt is fully read.
      wait_vmcnt<DMA_W, true>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // Second half: the MFMAs of substep 1, each with its share of the
      // activation DMAs of stage kt+2 (into the slot of stage kt) and the reads
      // of one fragment of stage kt+1.
      static_for<Q>([&](auto i) {
        constexpr int nb = i / MB, mb = i % MB;
        acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            F[1][MB + nb], F[1][mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
        constexpr int d0 = i * DMA_A / Q, d1 = (i + 1) * DMA_A / Q;
        issue_range(ja, jwf, kt + 2, use_sdma, std::integral_constant<int, d0>{},
                    std::integral_constant<int, d1>{});
        if constexpr (i < MB + NB) read_one(jan, jwn, I0{}, i);
        __builtin_amdgcn_sched_barrier(0);
      });
      static_for<(MB + NB > Q ? MB + NB - Q : 0)>([&](auto i) {
        read_one(jan, jwn, I0{}, std::integral_constant<int, Q + i>{});
      });
    };
    if (KT == 1) {
      stage(0, 0, c, std::true_type{}, std::true_type{});
      return;
    }
    stage(0, 0, c, std::false_type{}, std::true_type{});
    int ja = 1, jw = c == 2 ? 0 : c + 1;
    for (int kt = 1; kt < KT - 1; ++kt) {
      stage(kt, ja, jw, std::false_type{}, std::false_type{});
      ja ^= 1;
      jw = jw == 2 ? 0 : jw + 1;
    }
    stage(KT - 1, ja, jw, std::true_type{}, std::false_type{});
  };
  auto run = [&](auto use_sdma) {
    if constexpr (SPLIT)
      split_loop(use_sdma);
    else
      main_loop(use_sdma);
  };
  if constexpr (SDMA) {
    if (full)
      run(std::true_type{});
    else
      run(std::false_type{});
  } else {
    run(std::false_type{});
  }
  if constexpr (SPLIT && EPI_OVERLAP) {
    // The last stage's substep-1 MFMA of block q, issued by the epilogue.
    auto last_mfma = [&](auto q) {
      constexpr int nb = q / MB, mb = q % MB;
      acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          F[1][MB + nb], F[1][mb], acc[nb][mb], 0, 0, 0, 0, 0, 0);
    };
    // The thread index after the loop, recomputed rather than held through it.
    gemm_epilogue<BM, BN, WGM, WGN, EPI, true>(p, acc, m0, n0, wm, wn,
                                               wave * 64 + lane_id_fresh(), ring, vec,
                                               LORA_PRE ? lora_d : nullptr, last_mfma);
  } else {
    wait_vmcnt<0, true>();  // every DMA has landed before the ring is reused
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // The thread index after the loop, recomputed rather than held through it.
    gemm_epilogue<BM, BN, WGM, WGN, EPI, true>(p, acc, m0, n0, wm, wn,
                                               SPLIT ? wave * 64 + lane_id_fresh() : tid_v, ring,
                                               vec, LORA_PRE ? lora_d : nullptr);
  }
}

template <int EPI, int BM, int BN, int NS, int PRE, bool SDMA>
__global__ void __launch_bounds__(256, pipe_occupancy(BM, BN, NS)) fp8_gemm_pipe(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[pipe_lds(BM, BN, NS)];
  constexpr int VEC_BYTES = VEC_LDS + (epi_swiglu(EPI) ? SILU_LDS : 0);
  uint8_t* vec;
  if constexpr (NS == SPLIT_RING) {
    // The split ring keeps the vectors in its third weight slot.
    static_assert(VEC_BYTES <= BN * 128, "vectors fit one weight slot");
    vec = ring + (2 * BM + 2 * BN) * 128;
  } else {
    __shared__ __attribute__((aligned(1024))) uint8_t vec_own[VEC_BYTES];
    vec = vec_own;
  }
  int tm, tn;
  // SwiGLU tiles cover BN/2 value columns and their BN/2 gate columns.
  const int64_t tile_cols =
      epi_swiglu(EPI) ? (p.half_n + BN / 2 - 1) / (BN / 2) : (p.n + BN - 1) / BN;
  tile_coords((int)((p.m + BM - 1) / BM), (int)tile_cols, p.group_m, tm, tn);
  pipe_tile<EPI, BM, BN, NS, PRE, SDMA>(p, tm, tn, ring,
                                        __builtin_amdgcn_readfirstlane(lds_addr(ring)), vec,
                                        __builtin_amdgcn_readfirstlane(lds_addr(vec)),
                                        __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6));
}

// One pipelined configuration: tile, ring depth and the MFMAs of K-substep 1
// issued before the stage barrier.
template <int BM_, int BN_, int NS_, int PRE_>
struct PipeCfg {
  static constexpr int BM = BM_, BN = BN_, NS = NS_, PRE = PRE_;
};

template <int EPI, class C>
static hipError_t launch_pipe(const GemmParams& p, hipStream_t s) {
  const int64_t tile_cols =
      epi_swiglu(EPI) ? (p.half_n + C::BN / 2 - 1) / (C::BN / 2) : (p.n + C::BN - 1) / C::BN;
  const dim3 grid((unsigned)(((p.m + C::BM - 1) / C::BM) * tile_cols));
  // K not a multiple of 128 takes the vector-offset DMA everywhere; there the
  // split ring's extra lane offsets spill, so such shapes keep the two-slot ring.
  constexpr int NS_VOFF = C::NS == SPLIT_RING ? 2 : C::NS;
  if (p.k % 128)
    fp8_gemm_pipe<EPI, C::BM, C::BN, NS_VOFF, C::PRE, false><<<grid, dim3(256), 0, s>>>(p);
  else
    fp8_gemm_pipe<EPI, C::BM, C::BN, C::NS, C::PRE, true><<<grid, dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

// The tilings the launcher chooses from (fp8_gemm.hip, pick_tiling).
enum {
  GEMM_256x256 = 0,  // 2 slots, one workgroup per CU
  GEMM_256x192 = 1,  // 2 slots
  GEMM_256x128 = 2,  // 3 slots
  GEMM_128x192 = 3,  // 3 slots
  GEMM_128x128 = 4,  // 2 slots, two workgroups per CU
  GEMM_128x128_DEEP = 5,  // 3 slots, one workgroup per CU
  GEMM_128x64 = 6,   // 4 slots
  GEMM_64x64 = 7,    // 4 slots, two workgroups per CU
  GEMM_TILINGS = 8
};

template <int EPI>
hipError_t launch_tiling(const GemmParams& p, int tiling, hipStream_t s) {
  switch (tiling) {
    case GEMM_256x256: return launch_pipe<EPI, PipeCfg<256, 256, SPLIT_RING, 0>>(p, s);
    case GEMM_256x192: return launch_pipe<EPI, PipeCfg<256, 192, SPLIT_RING, 0>>(p, s);
    case GEMM_256x128: return launch_pipe<EPI, PipeCfg<256, 128, 3, 0>>(p, s);
    case GEMM_128x192: return launch_pipe<EPI, PipeCfg<128, 192, 3, 0>>(p, s);
    case GEMM_128x128: return launch_pipe<EPI, PipeCfg<128, 128, 2, -1>>(p, s);
    case GEMM_128x128_DEEP: return launch_pipe<EPI, PipeCfg<128, 128, 3, -1>>(p, s);
    case GEMM_128x64: return launch_pipe<EPI, PipeCfg<128, 64, 4, 0>>(p, s);
    case GEMM_64x64: return launch_pipe<EPI, PipeCfg<64, 64, 4, 0>>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vfa
