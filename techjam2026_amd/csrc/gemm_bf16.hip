// GEMM launches of MFMA mode bf16 (one translation unit per mode so the library's
// kernels compile in parallel).
#include "gemm_kernels.h"

namespace kf {
void gemm_launch_bf16(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st) {
  launch_mode<MODE_BF16, KF_BF16>(g, a_dtype, tile, epi, st);
}
}  // namespace kf
