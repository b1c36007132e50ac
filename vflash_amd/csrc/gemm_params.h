// Kernel-side parameter blocks of the E4M3 GEMM family and of the fused
// norm/modulation quantizer (not part of the C-ABI).
#pragma once
#include <stdint.h>

namespace vfa {

enum { EPI_BIAS = 0, EPI_GATE = 2, EPI_LORA = 3, EPI_SWIGLU = 4 };

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
  const uint16_t* lora_t;  // EPI_LORA: t[m * ldt + r], bf16
  int64_t ldt;
  const uint16_t* lora_b;  // EPI_LORA: B[n * ldb + r], bf16
  int64_t ldb;
  int rank;
  float lora_scale, lora_strength;
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
