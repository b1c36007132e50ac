// Exhaustive on-device check of the quantizers' fast row division
// (row_quotient<true>: Markstein's correction on y = RN(1/s)) against the IEEE
// quotient x / s.  For every bf16 row maximum amax > 0 whose scale
// s = max(amax / 448, FLT_MIN) takes the fast path, and every bf16 x with
// |x| <= amax, both quotients are clamped to +-448 and converted with the
// quantizers' hardware E4M3 conversion; the codes must agree.  Test
// infrastructure: built by __graft_entry__.build(), run by tests/test_gpu_quant.py.
// Prints "pairs <n> code_mismatches <m> quotient_mismatches <q>".
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "../../vflash_amd/csrc/quant_ops.h"

using namespace vfa;

constexpr uint32_t AMAX_LAST = 0x7f7f;  // largest finite bf16
constexpr uint32_t X_CHUNK = 256;       // x values per thread

__global__ void compare(unsigned long long* out) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t a = 1 + (uint32_t)(t / (0x10000 / X_CHUNK));
  unsigned long long pairs = 0, codes = 0, quotients = 0;
  if (a <= AMAX_LAST) {
    const float amax = bf16_to_f32(a);
    const float s = row_scale(amax);
    RowDivisor d;
    d.s = s;
    d.y = 1.0f / s;
    d.fast = true;
    if (s >= 0x1p-72f && s <= 3.40282347e38f) {
      const uint32_t x0 = (uint32_t)(t % (0x10000 / X_CHUNK)) * X_CHUNK;
      for (uint32_t xb = x0; xb < x0 + X_CHUNK; ++xb) {
        const float x = bf16_to_f32(xb);
        if (!(fabsf(x) <= amax)) continue;
        ++pairs;
        const float qf = clamped_row_quotient<true>(x, d);
        const float qe = clamped_row_quotient<false>(x, d);
        quotients += __float_as_uint(qf) != __float_as_uint(qe);
        const uint32_t cf = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qf, qf, 0, false) & 0xffu;
        const uint32_t ce = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qe, qe, 0, false) & 0xffu;
        codes += cf != ce;
      }
    }
  }
  atomicAdd(out, pairs);
  atomicAdd(out + 1, codes);
  atomicAdd(out + 2, quotients);
}

int main() {
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, 3 * sizeof(*d)) != hipSuccess || hipMemset(d, 0, 3 * sizeof(*d)) != hipSuccess) {
    std::printf("device setup failed\n");
    return 2;
  }
  const uint64_t threads = (uint64_t)AMAX_LAST * (0x10000 / X_CHUNK);
  compare<<<(unsigned)((threads + 255) / 256), 256>>>(d);
  unsigned long long h[3] = {~0ull, ~0ull, ~0ull};
  if (hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("device run failed\n");
    return 2;
  }
  std::printf("pairs %llu code_mismatches %llu quotient_mismatches %llu\n", h[0], h[1], h[2]);
  return 0;
}
