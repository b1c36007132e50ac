// The allocation-free form of the SwiGLU projection and its requantization,
// for callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that forbid it).
//
// vflash_fp8_linear_swiglu hands its per-row partial maxima (amax_part) to the
// caller, who passes them to vflash_requant_rows_e4m3.  Here both launches run
// in one call and the partial maxima live in `scratch`, a file-scope device
// array of VFLASH_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds
// until the process ends.  Its address on a device comes from
// hipGetSymbolAddress, taken once per device on the first call there with that
// device current; host code never uses the array's name as an address.
// Every (row, group) entry a call reads is written earlier in the same call, so
// nothing needs clearing; calls that overlap on one GPU share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/vflash_amd.h"
#include "gemm_params.h"

namespace vfa {
hipError_t launch_fp8_gemm(const GemmParams&, int, hipStream_t);
hipError_t launch_requant_rows(const uint16_t*, int64_t, int64_t, int64_t, const float*, int,
                               uint8_t*, float*, int64_t, hipStream_t);
}  // namespace vfa

namespace {

constexpr int64_t SCRATCH_FLOATS = VFLASH_NOALLOC_SCRATCH_BYTES / 4;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

constexpr int MAX_DEVICES = 64;
std::once_flag g_once[MAX_DEVICES];
float* g_scratch[MAX_DEVICES];
hipError_t g_status[MAX_DEVICES];

// This device's copy of `scratch`, or null if its address could not be taken.
float* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_status[dev] == hipSuccess ? static_cast<float*>(p) : nullptr;
  });
  return g_scratch[dev];
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" {

int vflash_fp8_linear_swiglu_quantize_noalloc(const void* a, const float* sa, int64_t lda,
                                              const void* w, const float* sw, int64_t ldw,
                                              int64_t m, int64_t n, int64_t k, const void* bias,
                                              void* h, int64_t ldh, void* codes, float* scales,
                                              int64_t m_pad, void* stream) {
  // The argument contract of vflash_fp8_linear_swiglu and vflash_requant_rows_e4m3.
  if (!a || !sa || !w || !sw || !h || !codes || !scales) return VFLASH_EINVAL;
  if (m < 1 || k < 16 || k % 16 || n < 256 || n % 256 || m_pad < m) return VFLASH_EINVAL;
  if (lda < k || ldw < k || lda % 16 || ldw % 16 || ldh < n / 2 || ldh % 8) return VFLASH_EINVAL;
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(sa, 4) || !aligned(sw, 16) ||
      !aligned(h, 16) || !aligned(codes, 8) || !aligned(scales, 4) || (bias && !aligned(bias, 16)))
    return VFLASH_EINVAL;
  if (256 * lda >= (int64_t(1) << 31) || 256 * ldw >= (int64_t(1) << 31)) return VFLASH_EINVAL;
  if (m >= (int64_t(1) << 31) / 256 * 256 || m_pad >= (int64_t(1) << 33)) return VFLASH_EINVAL;
  const int64_t parts = vflash_swiglu_parts(n);
  if (m > SCRATCH_FLOATS / parts) return VFLASH_ESCRATCH;
  float* part_max = device_scratch();
  if (!part_max) return VFLASH_ELAUNCH;

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
  p.out = static_cast<uint16_t*>(h);
  p.ldo = ldh;
  p.half_n = n / 2;
  p.amax_part = part_max;
  p.lora_scale[0] = p.lora_scale[1] = p.lora_scale[2] = 1.0f;
  p.lora_strength = 1.0f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vfa::launch_fp8_gemm(p, vfa::EPI_SWIGLU, s) != hipSuccess) return VFLASH_ELAUNCH;
  return vfa::launch_requant_rows(static_cast<const uint16_t*>(h), m, n / 2, ldh, part_max,
                                  (int)parts, static_cast<uint8_t*>(codes), scales, m_pad,
                                  s) == hipSuccess
             ? VFLASH_OK
             : VFLASH_ELAUNCH;
}

}  // extern "C"
