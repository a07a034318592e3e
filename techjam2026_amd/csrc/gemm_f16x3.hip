// GEMM launches of MFMA mode f16x3 (one translation unit per mode so the library's
// kernels compile in parallel).
#include "gemm_kernels.h"

namespace kf {
void gemm_launch_f16x3(const GemmArgs& g, int a_dtype, int tile, int epi, hipStream_t st) {
  launch_mode<MODE_F16X3, KF_F16X2>(g, a_dtype, tile, epi, st);
}
}  // namespace kf
