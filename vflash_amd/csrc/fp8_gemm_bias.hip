// The pipelined E4M3 GEMM tilings with the EPI_BIAS epilogue (one translation
// unit per epilogue, so the tilings compile in parallel).
#include "fp8_gemm_pipe.h"

namespace vfa {
template hipError_t launch_tiling<EPI_BIAS>(const GemmParams&, int, hipStream_t);
}  // namespace vfa
