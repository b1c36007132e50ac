// extern "C" entry points declared in include/vflash_amd.h.
//
// Each entry validates its arguments against the declared contract before any
// launch (no work is enqueued on a negative status), builds the kernel
// parameter block and enqueues on the caller's stream.  Nothing here
// allocates, synchronizes or retains a pointer.
#include <hip/hip_runtime.h>

#include "../../include/vflash_amd.h"
#include "common.h"
#include "gemm_params.h"

namespace vfa {
hipError_t launch_quant_rows(const uint16_t*, int64_t, int64_t, int64_t, uint8_t*, float*,
                             int64_t, hipStream_t);
hipError_t launch_norm_mod_quant(const NormModParams&, hipStream_t);
hipError_t launch_gelu_quant_rows(const uint16_t*, int64_t, int64_t, int64_t, uint16_t*, int64_t,
                                  uint8_t*, float*, int64_t, hipStream_t);
hipError_t launch_requant_rows(const uint16_t*, int64_t, int64_t, int64_t, const float*, int,
                               uint8_t*, float*, int64_t, hipStream_t);
hipError_t launch_fp8_gemm(const GemmParams&, int, hipStream_t);
int pick_tiling(int64_t m, int64_t n, int64_t cus, int64_t branch_cols);
hipError_t launch_lora_down(const uint16_t*, int64_t, int64_t, int64_t, const uint16_t*, int,
                            uint16_t*, int64_t, hipStream_t);
hipError_t launch_quant_lora(const uint16_t*, int64_t, int64_t, int64_t, const uint16_t*, int,
                             uint16_t*, int64_t, uint8_t*, float*, int64_t, hipStream_t);
hipError_t launch_nvfp4_quant(const uint16_t*, bool, int64_t, int64_t, int64_t, const float*,
                              uint8_t*, int64_t, uint8_t*, int64_t, hipStream_t);
hipError_t launch_nvfp4_w4a4(const uint8_t*, int64_t, const uint8_t*, const uint8_t*,
                             const uint8_t*, const float*, int64_t, int64_t, int64_t,
                             const uint16_t*, uint16_t*, int64_t, int, hipStream_t);
hipError_t launch_nvfp4(const uint8_t*, const float*, int64_t, const uint8_t*, const uint8_t*,
                        const float*, int64_t, int64_t, int64_t, const uint16_t*, uint16_t*, int64_t,
                        int, hipStream_t);
}  // namespace vfa

namespace {

// Tile-order group height of the E2M1-weight GEMMs, the fastest of a sweep over
// 1..32 at the large shapes.  The E4M3 launcher sets its own from the tiling.
constexpr int FP4_GROUP_M = 8;

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int status(hipError_t e) { return e == hipSuccess ? VFLASH_OK : VFLASH_ELAUNCH; }

// Shared contract of every E4M3 GEMM entry point.
bool gemm_args_ok(const void* a, const float* sa, int64_t lda, const void* w, const float* sw,
                  int64_t ldw, int64_t m, int64_t n, int64_t k, const void* bias) {
  if (!a || !sa || !w || !sw) return false;
  if (m < 1 || n < 1 || k < 16) return false;
  if (k % 16 || n % 16 || lda < k || ldw < k || lda % 16 || ldw % 16) return false;
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(sa, 4) || !aligned(sw, 4)) return false;
  if (bias && !aligned(bias, 8)) return false;
  // Per-tile buffer ranges (at most 256 rows) must stay below 2^31 bytes.
  if (256 * lda >= (int64_t(1) << 31) || 256 * ldw >= (int64_t(1) << 31)) return false;
  if (m >= (int64_t(1) << 31) / 256 * 256 || n >= (int64_t(1) << 31)) return false;
  return true;
}

vfa::GemmParams base_params(const void* a, const float* sa, int64_t lda, const void* w,
                            const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                            const void* bias, void* out, int64_t ldo) {
  vfa::GemmParams p{};
  p.a = static_cast<const uint8_t*>(a);
  p.sa = sa;
  p.w = static_cast<const uint8_t*>(w);
  p.sw = sw;
  p.sw_step = 1;
  p.lda = lda;
  p.ldw = ldw;
  p.m = m;
  p.n = n;
  p.k = k;
  p.bias = static_cast<const uint16_t*>(bias);
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.lora_scale[0] = p.lora_scale[1] = p.lora_scale[2] = 1.0f;
  p.lora_strength = 1.0f;
  return p;
}

// Adapter operands of the LoRA epilogues: rank 1..128; t rows hold `branches`
// runs of t_branch columns (branch b's rank positions at b * t_branch); reads
// stop at the rank rounded up to 8, inside rows whose strides are multiples of 8.
bool lora_args_ok(const void* t, int64_t ldt, const void* lora_b, int64_t ldb, int64_t rank,
                  int64_t branches, int64_t t_branch) {
  if (!t || !lora_b || rank < 1 || rank > 128 || ldb < rank || ldt % 8 || ldb % 8) return false;
  if (branches < 1 || branches > vfa::LORA_MAX_BRANCHES) return false;
  if (branches > 1 && (t_branch < rank || t_branch % 8)) return false;
  if (ldt < (branches - 1) * (branches > 1 ? t_branch : 0) + rank) return false;
  return aligned(t, 16) && aligned(lora_b, 16);
}

void set_lora(vfa::GemmParams& p, const void* t, int64_t ldt, const void* lora_b, int64_t ldb,
              int64_t rank, float strength) {
  p.lora_t = static_cast<const uint16_t*>(t);
  p.ldt = ldt;
  p.lora_b = static_cast<const uint16_t*>(lora_b);
  p.ldb = ldb;
  p.rank = (int)rank;
  p.lora_strength = strength;
}

// Gate and residual of the gate-residual epilogues.
bool gate_args_ok(const void* gate, int64_t gate_ts, int64_t gate_hs, int64_t gate_tokens,
                  const int64_t* gate_index, int64_t gate_rows, const void* residual, int64_t ldr,
                  int64_t n, const void* out, int64_t ldo) {
  if (!gate || !residual || ldr < n) return false;
  if (gate_ts < 0 || gate_hs < 0 || !aligned(gate, 2) || !aligned(residual, 2)) return false;
  if (gate_tokens < 1 || (gate_index && (gate_rows < 1 || !aligned(gate_index, 8)))) return false;
  if (out == residual && ldo != ldr) return false;
  return true;
}

void set_gate(vfa::GemmParams& p, const void* gate, int64_t gate_ts, int64_t gate_hs,
              int64_t gate_tokens, const int64_t* gate_index, int64_t gate_rows,
              const void* residual, int64_t ldr) {
  p.gate = static_cast<const uint16_t*>(gate);
  p.gate_ts = gate_ts;
  p.gate_hs = gate_hs;
  p.gate_tokens = gate_tokens;
  p.gate_index = gate_index;
  p.gate_rows = gate_rows;
  p.residual = static_cast<const uint16_t*>(residual);
  p.ldr = ldr;
}

// Output of the plain and plane-writing epilogues (plane_cols 0: one matrix).
bool out_args_ok(const void* out, int64_t ldo, int64_t m, int64_t n, int64_t plane_cols,
                 int64_t plane_stride) {
  if (!out || ldo % 4 || !aligned(out, 8)) return false;
  if (plane_cols == 0) return ldo >= n;
  if (plane_cols < 16 || plane_cols % 16 || n % plane_cols) return false;
  if (ldo < plane_cols || plane_stride % 4) return false;
  return plane_stride >= (m - 1) * ldo + plane_cols;  // planes may not overlap
}

}  // namespace

extern "C" {

int vflash_abi_version(void) { return 4; }

const char* vflash_status_string(int s) {
  switch (s) {
    case VFLASH_OK: return "ok";
    case VFLASH_EINVAL: return "argument outside the declared contract";
    case VFLASH_ELAUNCH: return "HIP launch failed";
    case VFLASH_ESCRATCH: return "the call needs more than the allocation-free entry's static scratch";
    default: return "unknown status";
  }
}

int vflash_quantize_rows_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx, void* codes,
                              float* scales, int64_t m_pad, void* stream) {
  if (!x || !codes || !scales || m < 1 || k < 1 || ldx < k || m_pad < m) return VFLASH_EINVAL;
  if (!aligned(x, 2) || !aligned(scales, 4) || m_pad >= (int64_t(1) << 33)) return VFLASH_EINVAL;
  return status(vfa::launch_quant_rows(static_cast<const uint16_t*>(x), m, k, ldx,
                                       static_cast<uint8_t*>(codes), scales, m_pad,
                                       static_cast<hipStream_t>(stream)));
}

int vflash_fp8_linear(const void* a, const float* sa, int64_t lda, const void* w,
                      const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                      const void* bias, void* out, int64_t ldo, void* stream) {
  if (!gemm_args_ok(a, sa, lda, w, sw, ldw, m, n, k, bias)) return VFLASH_EINVAL;
  if (!out || ldo < n || ldo % 4 || !aligned(out, 8)) return VFLASH_EINVAL;
  vfa::GemmParams p = base_params(a, sa, lda, w, sw, ldw, m, n, k, bias, out, ldo);
  return status(vfa::launch_fp8_gemm(p, vfa::EPI_BIAS, static_cast<hipStream_t>(stream)));
}

int vflash_fp8_linear_planes(const void* a, const float* sa, int64_t lda, const void* w,
                             const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                             const void* bias, void* out, int64_t ldo, int64_t plane_cols,
                             int64_t plane_stride, void* stream) {
  if (!gemm_args_ok(a, sa, lda, w, sw, ldw, m, n, k, bias)) return VFLASH_EINVAL;
  if (plane_cols < 1 || !out_args_ok(out, ldo, m, n, plane_cols, plane_stride))
    return VFLASH_EINVAL;
  vfa::GemmParams p = base_params(a, sa, lda, w, sw, ldw, m, n, k, bias, out, ldo);
  p.plane_cols = plane_cols;
  p.plane_stride = plane_stride;
  return status(vfa::launch_fp8_gemm(p, vfa::EPI_BIAS, static_cast<hipStream_t>(stream)));
}

int64_t vflash_swiglu_parts(int64_t n) { return n > 0 ? (n / 2 + 127) / 128 : 0; }

int vflash_fp8_gemm_tiling(int64_t m, int64_t n, int64_t compute_units, int64_t branch_cols) {
  if (m < 1 || n < 1 || compute_units < 1 || branch_cols < 0 || branch_cols % 32) return VFLASH_EINVAL;
  return vfa::pick_tiling(m, n, compute_units, branch_cols);
}

int vflash_fp8_linear_swiglu(const void* a, const float* sa, int64_t lda, const void* w,
                             const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                             const void* bias, void* h, int64_t ldh, float* amax_part,
                             void* stream) {
  return vflash_fp8_linear_swiglu_lora(a, sa, lda, w, sw, ldw, m, n, k, bias, nullptr, 0, nullptr,
                                       0, 0, 1.0f, 1.0f, h, ldh, amax_part, stream);
}

int vflash_fp8_linear_swiglu_lora(const void* a, const float* sa, int64_t lda, const void* w,
                                  const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                                  const void* bias, const void* t, int64_t ldt,
                                  const void* lora_b, int64_t ldb, int64_t rank, float scale,
                                  float strength, void* h, int64_t ldh, float* amax_part,
                                  void* stream) {
  if (!gemm_args_ok(a, sa, lda, w, sw, ldw, m, n, k, bias)) return VFLASH_EINVAL;
  if (n % 256 || !h || !amax_part || ldh < n / 2 || ldh % 8 || !aligned(h, 16) ||
      !aligned(amax_part, 4) || !aligned(sw, 16) || (bias && !aligned(bias, 16)))
    return VFLASH_EINVAL;
  const bool lora = t != nullptr || lora_b != nullptr;
  if (lora && !lora_args_ok(t, ldt, lora_b, ldb, rank, 1, 0)) return VFLASH_EINVAL;
  vfa::GemmParams p = base_params(a, sa, lda, w, sw, ldw, m, n, k, bias, h, ldh);
  p.half_n = n / 2;
  p.amax_part = amax_part;
  if (lora) {
    set_lora(p, t, ldt, lora_b, ldb, rank, strength);
    p.lora_scale[0] = scale;
  }
  return status(vfa::launch_fp8_gemm(p, lora ? vfa::EPI_SWIGLU_LORA : vfa::EPI_SWIGLU,
                                     static_cast<hipStream_t>(stream)));
}

int vflash_rmsnorm_modulate_quantize_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx,
                                          const void* norm_w, float eps, const void* scale,
                                          int64_t ld_scale, const void* shift, int64_t ld_shift,
                                          int64_t tokens, const int64_t* index, int64_t mod_rows,
                                          void* values, int64_t ldv, void* codes, float* scales,
                                          int64_t m_pad, void* stream) {
  if (!x || !scale || !shift || !codes || !scales) return VFLASH_EINVAL;
  if (m < 1 || k < 8 || k % 8 || k > 16384 || m_pad < m || m_pad >= (int64_t(1) << 33))
    return VFLASH_EINVAL;
  if (ldx < k || ldx % 8 || ld_scale < k || ld_scale % 8 || ld_shift < k || ld_shift % 8)
    return VFLASH_EINVAL;
  if (!aligned(x, 16) || !aligned(scale, 16) || !aligned(shift, 16) || !aligned(codes, 8) ||
      !aligned(scales, 4) || (norm_w && !aligned(norm_w, 16)))
    return VFLASH_EINVAL;
  if (!(eps >= 0.0f) || eps > 3.4e38f) return VFLASH_EINVAL;  // rejects NaN and infinity
  if (tokens < 1 || (index && (mod_rows < 1 || !aligned(index, 8)))) return VFLASH_EINVAL;
  if (values && (ldv < k || ldv % 8 || !aligned(values, 16))) return VFLASH_EINVAL;
  vfa::NormModParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.m = m;
  p.k = k;
  p.ldx = ldx;
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  p.scale = static_cast<const uint16_t*>(scale);
  p.ld_scale = ld_scale;
  p.shift = static_cast<const uint16_t*>(shift);
  p.ld_shift = ld_shift;
  p.tokens = tokens;
  p.index = index;
  p.mod_rows = index ? mod_rows : tokens;
  p.values = static_cast<uint16_t*>(values);
  p.ldv = ldv;
  p.codes = static_cast<uint8_t*>(codes);
  p.scales = scales;
  p.m_pad = m_pad;
  return status(vfa::launch_norm_mod_quant(p, static_cast<hipStream_t>(stream)));
}

int vflash_gelu_quantize_rows_e4m3(const void* y, int64_t m, int64_t k, int64_t ldy, void* g,
                                   int64_t ldg, void* codes, float* scales, int64_t m_pad,
                                   void* stream) {
  if (!y || !codes || !scales || m < 1 || k < 8 || k > 16384 || k % 8 || m_pad < m)
    return VFLASH_EINVAL;
  if (ldy < k || ldy % 8 || !aligned(y, 16) || !aligned(codes, 8) || !aligned(scales, 4))
    return VFLASH_EINVAL;
  if (g && (ldg < k || ldg % 8 || !aligned(g, 16))) return VFLASH_EINVAL;
  if (m_pad >= (int64_t(1) << 33)) return VFLASH_EINVAL;
  return status(vfa::launch_gelu_quant_rows(static_cast<const uint16_t*>(y), m, k, ldy,
                                            static_cast<uint16_t*>(g), ldg,
                                            static_cast<uint8_t*>(codes), scales, m_pad,
                                            static_cast<hipStream_t>(stream)));
}

int vflash_requant_rows_e4m3(const void* g, int64_t m, int64_t k, int64_t ldg,
                             const float* amax_part, int64_t parts, void* codes, float* scales,
                             int64_t m_pad, void* stream) {
  if (!g || !amax_part || !codes || !scales || m < 1 || k < 8 || m_pad < m) return VFLASH_EINVAL;
  if (k % 8 || ldg < k || ldg % 8 || !aligned(g, 16) || !aligned(codes, 8)) return VFLASH_EINVAL;
  if (parts < 1 || parts > (int64_t(1) << 30) || !aligned(scales, 4)) return VFLASH_EINVAL;
  return status(vfa::launch_requant_rows(static_cast<const uint16_t*>(g), m, k, ldg, amax_part,
                                         (int)parts, static_cast<uint8_t*>(codes), scales, m_pad,
                                         static_cast<hipStream_t>(stream)));
}

int vflash_fp8_linear_gate_residual(const void* a, const float* sa, int64_t lda, const void* w,
                                    const float* sw, int64_t ldw, int64_t m, int64_t n,
                                    int64_t k, const void* bias, const void* gate,
                                    int64_t gate_ts, int64_t gate_hs, int64_t gate_tokens,
                                    const int64_t* gate_index, int64_t gate_rows,
                                    const void* residual, int64_t ldr, void* out, int64_t ldo,
                                    void* stream) {
  return vflash_fp8_linear_lora_gate_residual(a, sa, lda, w, sw, ldw, m, n, k, bias, gate, gate_ts,
                                              gate_hs, gate_tokens, gate_index, gate_rows,
                                              residual, ldr, nullptr, 0, nullptr, 0, 0, 1.0f, 1.0f,
                                              out, ldo, stream);
}

int vflash_fp8_linear_lora_gate_residual(
    const void* a, const float* sa, int64_t lda, const void* w, const float* sw, int64_t ldw,
    int64_t m, int64_t n, int64_t k, const void* bias, const void* gate, int64_t gate_ts,
    int64_t gate_hs, int64_t gate_tokens, const int64_t* gate_index, int64_t gate_rows,
    const void* residual, int64_t ldr, const void* t, int64_t ldt, const void* lora_b,
    int64_t ldb, int64_t rank, float scale, float strength, void* out, int64_t ldo,
    void* stream) {
  if (!gemm_args_ok(a, sa, lda, w, sw, ldw, m, n, k, bias)) return VFLASH_EINVAL;
  if (!out_args_ok(out, ldo, m, n, 0, 0)) return VFLASH_EINVAL;
  if (!gate_args_ok(gate, gate_ts, gate_hs, gate_tokens, gate_index, gate_rows, residual, ldr, n,
                    out, ldo))
    return VFLASH_EINVAL;
  const bool lora = t != nullptr || lora_b != nullptr;
  if (lora && !lora_args_ok(t, ldt, lora_b, ldb, rank, 1, 0)) return VFLASH_EINVAL;
  vfa::GemmParams p = base_params(a, sa, lda, w, sw, ldw, m, n, k, bias, out, ldo);
  set_gate(p, gate, gate_ts, gate_hs, gate_tokens, gate_index, gate_rows, residual, ldr);
  if (lora) {
    set_lora(p, t, ldt, lora_b, ldb, rank, strength);
    p.lora_scale[0] = scale;
  }
  return status(vfa::launch_fp8_gemm(p, lora ? vfa::EPI_LORA_GATE : vfa::EPI_GATE,
                                     static_cast<hipStream_t>(stream)));
}

int vflash_lora_down(const void* x, int64_t m, int64_t k, int64_t ldx, const void* lora_a,
                     int64_t rank, void* t, int64_t ldt, void* stream) {
  if (!x || !lora_a || !t || m < 1 || k < 16 || k % 16 || ldx < k || ldx % 8) return VFLASH_EINVAL;
  if (rank < 1 || rank > 512 || ldt < (rank + 15) / 16 * 16 || ldt % 8) return VFLASH_EINVAL;
  if (!aligned(x, 16) || !aligned(lora_a, 16) || !aligned(t, 16)) return VFLASH_EINVAL;
  return status(vfa::launch_lora_down(static_cast<const uint16_t*>(x), m, k, ldx,
                                      static_cast<const uint16_t*>(lora_a), (int)rank,
                                      static_cast<uint16_t*>(t), ldt,
                                      static_cast<hipStream_t>(stream)));
}

int vflash_quantize_rows_lora_e4m3(const void* x, int64_t m, int64_t k, int64_t ldx,
                                   void* codes, float* scales, int64_t m_pad,
                                   const void* lora_a, int64_t rank, void* t, int64_t ldt,
                                   void* stream) {
  if (!x || !codes || !scales || !lora_a || !t || m < 1 || m_pad < m) return VFLASH_EINVAL;
  if (k < 16 || k % 16 || ldx < k || ldx % 8) return VFLASH_EINVAL;
  if (rank < 1 || rank > 512 || ldt < (rank + 15) / 16 * 16 || ldt % 8) return VFLASH_EINVAL;
  if (!aligned(x, 16) || !aligned(lora_a, 16) || !aligned(t, 16) || !aligned(codes, 8) ||
      !aligned(scales, 4))
    return VFLASH_EINVAL;
  return status(vfa::launch_quant_lora(static_cast<const uint16_t*>(x), m, k, ldx,
                                       static_cast<const uint16_t*>(lora_a), (int)rank,
                                       static_cast<uint16_t*>(t), ldt,
                                       static_cast<uint8_t*>(codes), scales, m_pad,
                                       static_cast<hipStream_t>(stream)));
}

int vflash_fp8_linear_lora(const void* a, const float* sa, int64_t lda, const void* w,
                           const float* sw, int64_t ldw, int64_t m, int64_t n, int64_t k,
                           const void* bias, const void* t, int64_t ldt, const void* lora_b,
                           int64_t ldb, int64_t rank, float scale, float strength, void* out,
                           int64_t ldo, void* stream) {
  return vflash_fp8_linear_lora_branches(a, sa, lda, w, sw, ldw, m, n, k, bias, t, ldt, 0, lora_b,
                                         ldb, rank, 1, &scale, strength, out, ldo, 0, 0, stream);
}

int vflash_fp8_linear_lora_branches(const void* a, const float* sa, int64_t lda, const void* w,
                                    const float* sw, int64_t ldw, int64_t m, int64_t n,
                                    int64_t k, const void* bias, const void* t, int64_t ldt,
                                    int64_t t_branch, const void* lora_b, int64_t ldb,
                                    int64_t rank, int64_t branches, const float* scales,
                                    float strength, void* out, int64_t ldo, int64_t plane_cols,
                                    int64_t plane_stride, void* stream) {
  if (!gemm_args_ok(a, sa, lda, w, sw, ldw, m, n, k, bias)) return VFLASH_EINVAL;
  if (plane_cols < 0 || !out_args_ok(out, ldo, m, n, plane_cols, plane_stride)) return VFLASH_EINVAL;
  if (!scales || !lora_args_ok(t, ldt, lora_b, ldb, rank, branches, t_branch)) return VFLASH_EINVAL;
  if (n % branches || (branches > 1 && (n / branches) % 32)) return VFLASH_EINVAL;
  vfa::GemmParams p = base_params(a, sa, lda, w, sw, ldw, m, n, k, bias, out, ldo);
  p.plane_cols = plane_cols;
  p.plane_stride = plane_stride;
  set_lora(p, t, ldt, lora_b, ldb, rank, strength);
  p.lora_branch_cols = branches > 1 ? n / branches : 0;
  p.lora_t_branch = branches > 1 ? t_branch : 0;
  for (int b = 0; b < branches; ++b) p.lora_scale[b] = scales[b];
  return status(vfa::launch_fp8_gemm(p, vfa::EPI_LORA, static_cast<hipStream_t>(stream)));
}

int vflash_nvfp4_linear(const void* a, const float* sa, int64_t lda, const void* w_packed,
                        const void* w_scales, const float* alpha, int64_t m, int64_t n, int64_t k,
                        const void* bias, void* out, int64_t ldo, void* stream) {
  if (!a || !sa || !w_packed || !w_scales || !alpha || !out || m < 1 || n < 128 || k < 64)
    return VFLASH_EINVAL;
  if (n % 128 || k % 64 || lda < k || lda % 16 || ldo < n || ldo % 4) return VFLASH_EINVAL;
  if (!aligned(a, 16) || !aligned(w_packed, 16) || !aligned(w_scales, 16) || !aligned(out, 8))
    return VFLASH_EINVAL;
  if (bias && !aligned(bias, 2)) return VFLASH_EINVAL;
  if (!aligned(alpha, 4) || !aligned(sa, 4)) return VFLASH_EINVAL;
  if (256 * lda >= (int64_t(1) << 31)) return VFLASH_EINVAL;
  return status(vfa::launch_nvfp4(static_cast<const uint8_t*>(a), sa, lda,
                                  static_cast<const uint8_t*>(w_packed),
                                  static_cast<const uint8_t*>(w_scales), alpha, m, n, k,
                                  static_cast<const uint16_t*>(bias),
                                  static_cast<uint16_t*>(out), ldo, FP4_GROUP_M,
                                  static_cast<hipStream_t>(stream)));
}

int vflash_nvfp4_quantize_rows(const void* x, int x_is_f16, int64_t m, int64_t k, int64_t ldx,
                               const float* global_sf, void* codes, int64_t ldc, void* scales,
                               int64_t m_pad, void* stream) {
  if (!x || !global_sf || !codes || !scales || m < 1 || k < 64 || k % 64) return VFLASH_EINVAL;
  if (ldx < k || ldx % 8 || ldc < k / 2 || ldc % 16 || m_pad < m || m_pad % 128) return VFLASH_EINVAL;
  if (m_pad >= (int64_t(1) << 33)) return VFLASH_EINVAL;
  if (!aligned(x, 16) || !aligned(codes, 16) || !aligned(scales, 4) || !aligned(global_sf, 4))
    return VFLASH_EINVAL;
  return status(vfa::launch_nvfp4_quant(static_cast<const uint16_t*>(x), x_is_f16 != 0, m, k, ldx,
                                        global_sf, static_cast<uint8_t*>(codes), ldc,
                                        static_cast<uint8_t*>(scales), m_pad,
                                        static_cast<hipStream_t>(stream)));
}

int vflash_nvfp4_w4a4_linear(const void* a, int64_t lda, const void* a_scales, const void* w_packed,
                             const void* w_scales, const float* alpha, int64_t m, int64_t n,
                             int64_t k, const void* bias, void* out, int64_t ldo, void* stream) {
  if (!a || !a_scales || !w_packed || !w_scales || !alpha || !out || m < 1 || n < 128 || k < 64)
    return VFLASH_EINVAL;
  if (n % 128 || k % 64 || lda < k / 2 || lda % 16 || ldo < n || ldo % 4) return VFLASH_EINVAL;
  if (!aligned(a, 16) || !aligned(a_scales, 16) || !aligned(w_packed, 16) ||
      !aligned(w_scales, 16) || !aligned(out, 8) || !aligned(alpha, 4))
    return VFLASH_EINVAL;
  if (bias && !aligned(bias, 2)) return VFLASH_EINVAL;
  if (256 * lda >= (int64_t(1) << 31)) return VFLASH_EINVAL;
  return status(vfa::launch_nvfp4_w4a4(
      static_cast<const uint8_t*>(a), lda, static_cast<const uint8_t*>(a_scales),
      static_cast<const uint8_t*>(w_packed), static_cast<const uint8_t*>(w_scales), alpha, m, n, k,
      static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, FP4_GROUP_M,
      static_cast<hipStream_t>(stream)));
}

}  // extern "C"
