// W8A8 E4M3 GEMM with fused epilogues for gfx950 (CDNA4): the choice of tiling
// and the dispatch.  The kernel is the pipelined tile of fp8_gemm_pipe.h.
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
//   EPI_LORA_GATE   EPI_GATE on bf16(base + delta): the adapted gate-residual
//              (h3_native_denoiser.py:327-338, h3_fused_ops.py:341-418)
//   EPI_SWIGLU_LORA EPI_SWIGLU on bf16(base + delta) for value and gate columns
//              alike (h3_fused_ops.py:229-286, strict_ffn_adapter_silu_kernel)
// The LoRA delta may come from up to three adapter branches with their own
// scales, each owning a contiguous run of output columns (the Q/K/V adapters of
// a merged projection, h3_native_denoiser.py:301-316, h3_fused_ops.py:900-980).
#include "fp8_gemm_pipe.h"

namespace vfa {

extern template hipError_t launch_tiling<EPI_BIAS>(const GemmParams&, int, hipStream_t);
extern template hipError_t launch_tiling<EPI_GATE>(const GemmParams&, int, hipStream_t);
extern template hipError_t launch_tiling<EPI_LORA>(const GemmParams&, int, hipStream_t);
extern template hipError_t launch_tiling<EPI_LORA_GATE>(const GemmParams&, int, hipStream_t);

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

// The tiling of a call, from its shape alone.
//
// A tiling's cost is the work of the busiest CU: ceil(tiles / CUs) tiles of
// BM x BN outputs (two co-resident tiles share one CU's throughput), divided
// by the tiling's relative throughput per output (larger tiles read fewer
// operand bytes per MFMA).  The cheapest wins, larger tiles first on ties.
// The 3-slot 128x128 form runs only where the grid fits one round; with more
// tiles the 2-slot form, two per CU, hides each tile's latency behind the
// other's.  The throughputs come from a sweep of every tiling over the
// skinny, adapter, 4096x3072x3072 and 32760x5120x13824 shapes, and of the
// 256-row and 128x128 tilings over 2048-8192 rows of K = 5120 linears.
struct Tiling {
  int bm, bn;
  double rate;          // relative throughput per output
  bool one_round_only;  // only where every tile gets a CU of its own
};
constexpr Tiling kTilings[GEMM_TILINGS] = {
    {256, 256, 1.00, false}, {256, 192, 0.92, false}, {256, 128, 0.82, false},
    {128, 192, 0.85, false}, {128, 128, 0.75, false}, {128, 128, 0.85, true},
    {128, 64, 0.60, false},  {64, 64, 0.50, false},
};

// branch_cols > 0 (a LoRA epilogue with several adapter branches of that many
// columns): only tilings whose wave width (BN / 2) divides branch_cols, so that
// each wave's columns belong to one branch.  The 128x64 and 64x64 tilings
// (32-column waves) serve every multiple of 32.
int pick_tiling(int64_t m, int64_t n, int64_t cus, int64_t branch_cols) {
  auto allowed = [&](int t) { return branch_cols <= 0 || branch_cols % (kTilings[t].bn / 2) == 0; };
  // Grids of three or more rounds of 256x256 tiles are MFMA-bound, and there
  // the largest tile's operand reuse wins: at 4095 x 5120 x 13824 it takes
  // 0.246 ms against 0.251 for 256x192, 0.265 for 256x128 and 0.272-0.274 for
  // the 128-row tiles (whose throughputs below come from one-round grids).
  if (((m + 255) / 256) * ((n + 255) / 256) >= 3 * cus && allowed(GEMM_256x256))
    return GEMM_256x256;
  int best = -1;
  double best_cost = 0.0;
  for (int t = 0; t < GEMM_TILINGS; ++t) {
    const Tiling& c = kTilings[t];
    if (!allowed(t)) continue;
    const int64_t tiles = ((m + c.bm - 1) / c.bm) * ((n + c.bn - 1) / c.bn);
    if (c.one_round_only && tiles > cus) continue;
    const double cost = (double)((tiles + cus - 1) / cus) * c.bm * c.bn / c.rate;
    if (best < 0 || cost < best_cost) {
      best = t;
      best_cost = cost;
    }
  }
  return best;
}

// Tile-order group height.  The 256x256 tiling sweeps four tile rows at a time
// when the output has at most 48 tile columns (N <= 12288) and three when it
// has more; the tiles resident on one XCD then share a few A and W panels in
// that XCD's L2.  Measured at M = 32760 against heights 2, 3 and 4 in
// alternating runs: height 4 is the fastest or within 0.3 % for N of 3072 to
// 10240 and the FFN down projection (height 3 up to 2.5 % slower there);
// height 3 is 0.5-0.8 % faster than 2 at N = 13824 and 15360 and 2.5-3 % at
// N = 28672 and the SwiGLU projection (112 column tiles).  The other tilings,
// on grids of one or a few rounds, use eight.
int tiling_group_m(int tiling, int64_t tile_cols) {
  if (tiling != GEMM_256x256) return 8;
  return tile_cols <= 48 ? 4 : 3;
}

// GemmParams::group_m is set here from the tiling.
hipError_t launch_fp8_gemm(const GemmParams& params, int epi, hipStream_t s) {
  GemmParams p = params;
  if (epi_swiglu(epi)) {
    // One tiling: 128 value + 128 gate columns, the 256x256 schedule.
    p.group_m = tiling_group_m(GEMM_256x256, (p.half_n + 127) / 128);
    if (epi == EPI_SWIGLU_LORA) return launch_pipe<EPI_SWIGLU_LORA, PipeCfg<256, 256, SPLIT_RING, 0>>(p, s);
    return launch_pipe<EPI_SWIGLU, PipeCfg<256, 256, SPLIT_RING, 0>>(p, s);
  }
  const int tiling =
      pick_tiling(p.m, p.n, compute_units(), epi_lora(epi) ? p.lora_branch_cols : 0);
  if (tiling < 0) return hipErrorInvalidValue;
  p.group_m = tiling_group_m(tiling, (p.n + kTilings[tiling].bn - 1) / kTilings[tiling].bn);
  switch (epi) {
    case EPI_BIAS: return launch_tiling<EPI_BIAS>(p, tiling, s);
    case EPI_GATE: return launch_tiling<EPI_GATE>(p, tiling, s);
    case EPI_LORA: return launch_tiling<EPI_LORA>(p, tiling, s);
    case EPI_LORA_GATE: return launch_tiling<EPI_LORA_GATE>(p, tiling, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vfa
