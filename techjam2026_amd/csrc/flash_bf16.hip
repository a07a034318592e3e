// FlashAttention launches of MFMA mode bf16 (one translation unit per mode so the
// library's kernels compile in parallel).
#include "flash_kernels.h"

namespace kf {
void flash_launch_bf16(const FlashArgs& a, int q_dtype, int hdp, hipStream_t st) {
  launch_q<MODE_BF16>(a, q_dtype, hdp, st);
}
}  // namespace kf
