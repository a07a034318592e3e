// GEMM launches of the fp32 MFMA mode (its own translation unit).
#include "gemm_kernels.h"

namespace kf {
void gemm_launch_f32(const GemmArgs& g, int a_dtype, hipStream_t st) {
  const int64_t blocks = ((int64_t)(g.M + GBM - 1) / GBM) * ((g.N + GBN - 1) / GBN);
  switch (a_dtype) {
    case KF_F32: hipLaunchKernelGGL((gemm32_kernel<KF_F32>), dim3((unsigned)blocks), dim3(256), 0, st, g); break;
    case KF_F16: hipLaunchKernelGGL((gemm32_kernel<KF_F16>), dim3((unsigned)blocks), dim3(256), 0, st, g); break;
    default: hipLaunchKernelGGL((gemm32_kernel<KF_BF16>), dim3((unsigned)blocks), dim3(256), 0, st, g); break;
  }
}
}  // namespace kf
