// head_dim 128 instantiations of the ragged prefill kernel (mi_prefill_kernel.h).
// They live in their own translation unit so that the build can give them the
// backend's max-ILP instruction scheduler: measured on the c4 batch, 586-591 us
// against 596-600 us with the default scheduler, while head_dim 256 runs 1.4%
// slower under it (1720 vs 1697 us) and keeps the default.
#include "mi_prefill_kernel.h"

namespace mi {

int prefill_d128_launch(const PrefillParams& pp, bool f16, bool fp8, int grid, hipStream_t stream) {
  const dim3 block(64 * pf_waves(128));
  if (f16) {
    if (fp8) hipLaunchKernelGGL((prefill_kernel<F16, true, 128>), dim3(grid), block, 0, stream, pp);
    else hipLaunchKernelGGL((prefill_kernel<F16, false, 128>), dim3(grid), block, 0, stream, pp);
  } else {
    if (fp8) hipLaunchKernelGGL((prefill_kernel<BF16, true, 128>), dim3(grid), block, 0, stream, pp);
    else hipLaunchKernelGGL((prefill_kernel<BF16, false, 128>), dim3(grid), block, 0, stream, pp);
  }
  return MI_OK;
}

}  // namespace mi
