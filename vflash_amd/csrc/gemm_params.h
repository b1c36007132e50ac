// Kernel-side parameter blocks of the E4M3 GEMM family and of the fused
// norm/modulation quantizer (not part of the C-ABI).
#pragma once
#include <stdint.h>

namespace vfa {

// Epilogues.  The LoRA merge (phase 1) combines with the plain store, the
// gate-residual (phase 2) and the SwiGLU activation (phase 2).
enum {
  EPI_BIAS = 0,
  EPI_GATE = 2,
  EPI_LORA = 3,
  EPI_SWIGLU = 4,
  EPI_LORA_GATE = 5,
  EPI_SWIGLU_LORA = 6
};
constexpr bool epi_lora(int e) { return e == EPI_LORA || e == EPI_LORA_GATE || e == EPI_SWIGLU_LORA; }
constexpr bool epi_gate(int e) { return e == EPI_GATE || e == EPI_LORA_GATE; }
constexpr bool epi_swiglu(int e) { return e == EPI_SWIGLU || e == EPI_SWIGLU_LORA; }

// Adapter branches of one LoRA epilogue (the three Q/K/V adapters of a merged
// projection): output column n belongs to branch n / lora_branch_cols.
constexpr int LORA_MAX_BRANCHES = 3;

struct GemmParams {
  const uint8_t* a;  // activation codes [m, k], row stride lda bytes
  const float* sa;   // per-row activation scales [m]
  const uint8_t* w;  // weight codes [n, k], row stride ldw bytes
  const float* sw;   // weight scales: sw[n * sw_step] (sw_step 0: one scalar)
  int64_t sw_step;
  const uint8_t* wsb;  // E2M1-weight GEMM: E4M3 block scales in the 128x4 order
  const uint8_t* asb;  // E2M1 activations (W4A4): their block scales, 128x4 order, rows
                       // padded to a multiple of 128; then sa is null
  int64_t lda, ldw, m, n, k;
  const uint16_t* bias;  // bf16 [n] or null
  uint16_t* out;         // bf16, row stride ldo elements
  int64_t ldo;
  int64_t plane_cols;    // > 0: column n goes to plane n / plane_cols
  int64_t plane_stride;  // elements between planes
  float* amax_part;      // EPI_SWIGLU: [m, ceil(n / 256)] per-row maxima of |out|
  const uint16_t* gate;  // EPI_GATE: gate[g * gate_ts + n * gate_hs] for output row m, with
  int64_t gate_ts, gate_hs;  // g = m % gate_tokens, or gate_index[m % gate_tokens] (< gate_rows)
  int64_t gate_tokens;
  const int64_t* gate_index;
  int64_t gate_rows;
  const uint16_t* residual;  // EPI_GATE: residual[m * ldr + n]
  int64_t ldr;
  // LoRA epilogues: delta[m, n] = sum_{r < rank} t[m * ldt + b * lora_t_branch + r] *
  // B[n * ldb + r] for the branch b of column n (0 when lora_branch_cols is 0),
  // then bf16(delta * lora_scale[b]) and bf16(delta * lora_strength).
  const uint16_t* lora_t;  // bf16
  int64_t ldt;
  const uint16_t* lora_b;  // bf16, row n of the (stacked) up-projection
  int64_t ldb;
  int rank;  // 1..128
  int64_t lora_branch_cols;  // 0: one branch; else a multiple of 32
  int64_t lora_t_branch;     // t columns between branches
  float lora_scale[LORA_MAX_BRANCHES], lora_strength;
  int64_t half_n;  // EPI_SWIGLU: columns [0, half_n) are values, [half_n, n) gates
  int group_m;  // tile-order group height
};

// RMSNorm + adaLN modulation + per-token E4M3 quantization (producer.hip).
struct NormModParams {
  const uint16_t* x;
  int64_t m, k, ldx;
  const uint16_t* norm_w;  // [k], or null for an RMSNorm without weight
  float eps;
  const uint16_t* scale;
  int64_t ld_scale;
  const uint16_t* shift;
  int64_t ld_shift;
  int64_t tokens;
  const int64_t* index;  // [tokens] modulation rows, or null
  int64_t mod_rows;      // rows addressable through index
  uint16_t* values;      // optional bf16 copy of y
  int64_t ldv;
  uint8_t* codes;
  float* scales;
  int64_t m_pad;
};

}  // namespace vfa
