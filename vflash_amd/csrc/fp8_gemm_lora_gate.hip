// The pipelined E4M3 GEMM tilings with the EPI_LORA_GATE epilogue (one
// translation unit per epilogue, so the tilings compile in parallel).
#include "fp8_gemm_pipe.h"

namespace vfa {
template hipError_t launch_tiling<EPI_LORA_GATE>(const GemmParams&, int, hipStream_t);
}  // namespace vfa
