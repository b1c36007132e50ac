// Exhaustive check of the hardware binary32 -> OCP E2M1 conversion used by the
// NVFP4 activation quantizer (v_cvt_scalef32_pk_fp4_f32 with scale 1.0)
// against the software round-to-nearest-even encoder f32_to_e2m1, for every
// binary32 value with |x| <= 6 (the clamped range the quantizer converts),
// both signs; it also checks that the first source lands in the low nibble.
// Test infrastructure: built by __graft_entry__.build(), run by
// tests/test_gpu_nvfp4.py.  Prints "values <n> mismatches <m> order_mismatches <o>".
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "../../vflash_amd/csrc/common.h"

using namespace vfa;

__global__ void compare(unsigned long long* out) {
  const uint32_t limit = 0x40c00000u;  // 6.0f
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned long long n = 0, order = 0;
  for (uint32_t a = blockIdx.x * blockDim.x + threadIdx.x; a <= limit; a += stride) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float x = __uint_as_float(a | (s ? 0x80000000u : 0u));
      const uint32_t lo = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, x, 0.0f, 1.0f, 0);
      const uint32_t hi = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, 0.0f, x, 1.0f, 0);
      const uint32_t ref = f32_to_e2m1(x);
      n += (lo & 0xfu) != ref;
      order += (lo >> 4) != 0u || (hi & 0xfu) != 0u || (hi >> 4) != ref;
    }
  }
  atomicAdd(out, n);
  atomicAdd(out + 1, order);
}

int main() {
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, 2 * sizeof(*d)) != hipSuccess || hipMemset(d, 0, 2 * sizeof(*d)) != hipSuccess) {
    std::printf("device setup failed\n");
    return 2;
  }
  compare<<<8192, 256>>>(d);
  unsigned long long h[2] = {~0ull, ~0ull};
  if (hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("device run failed\n");
    return 2;
  }
  std::printf("values %llu mismatches %llu order_mismatches %llu\n", 2ull * (0x40c00000ull + 1),
              h[0], h[1]);
  return 0;
}
