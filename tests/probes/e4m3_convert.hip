// Exhaustive check of the hardware binary32 -> OCP E4M3 conversion used by the
// quantization kernels (v_cvt_pk_fp8_f32) against the software round-to-
// nearest-even encoder f32_to_e4m3, for every binary32 value with |x| <= 448
// (the clamped range the quantizers convert), both signs.  Test
// infrastructure: built by __graft_entry__.build(), run by tests/test_gpu_quant.py.
// Prints "values <n> mismatches <m>"; exit status 0 when the run completed.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "../../vflash_amd/csrc/common.h"

using namespace vfa;

__global__ void compare(unsigned long long* mismatches) {
  const uint32_t limit = 0x43e00000u;  // 448.0f
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned long long n = 0;
  for (uint32_t a = blockIdx.x * blockDim.x + threadIdx.x; a <= limit; a += stride) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float x = __uint_as_float(a | (s ? 0x80000000u : 0u));
      const uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, x, 0, false) & 0xffu;
      n += hw != f32_to_e4m3(x);
    }
  }
  atomicAdd(mismatches, n);
}

int main() {
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, sizeof(*d)) != hipSuccess || hipMemset(d, 0, sizeof(*d)) != hipSuccess) {
    std::printf("device setup failed\n");
    return 2;
  }
  compare<<<8192, 256>>>(d);
  unsigned long long h = ~0ull;
  if (hipMemcpy(&h, d, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("device run failed\n");
    return 2;
  }
  std::printf("values %llu mismatches %llu\n", 2ull * (0x43e00000ull + 1), h);
  return 0;
}
