// FlashAttention launches of MFMA mode f16 (one translation unit per mode so the
// library's kernels compile in parallel).
#include "flash_kernels.h"

namespace kf {
void flash_launch_f16(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st) {
  launch_q<MODE_F16>(a, q_dtype, hdp, st);
}
}  // namespace kf
