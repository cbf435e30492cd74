// HBM read ceiling for the measurements beside the decode kernels.
//
// hbm_read_kernel streams a device buffer with the 16-byte non-temporal
// loads the decode kernels use: each workgroup reads 32 KiB chunks (8 load
// instructions of 4 KiB each, all in flight together) and folds what it read
// into one word per wavefront, so no load is dead.  Its rate over a KV pool
// layer is what a plain read of the same memory reaches on the box, the
// reference point for the decode kernel's achieved GB/s (chunks of 16, 64
// and 128 KiB and 2-16 workgroups per CU measured within the same
// 7.0-7.16 TB/s).  Measurement only: the reference has no counterpart.
#include "mi_common.h"

#ifndef MI_HBM_READ_UNR
#define MI_HBM_READ_UNR 8
#endif

namespace mi {

// Each workgroup reads contiguous chunks of 256 x UNR 16-byte pieces (one
// load instruction covers 4 KiB of a chunk; all UNR loads of a thread are in
// flight together), the chunks dealt to the workgroups round-robin.
template <int UNR>
__global__ __launch_bounds__(256) void hbm_read_kernel(const uint8_t* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ sink) {
  constexpr int64_t CH = 256 * UNR;
  uint32_t acc = 0;
  for (int64_t c = blockIdx.x; c * CH < n16; c += gridDim.x) {
    const int64_t base = c * CH + threadIdx.x;
    uint4 v[UNR];
    if ((c + 1) * CH <= n16) {
#pragma unroll
      for (int k = 0; k < UNR; ++k) v[k] = nt_load16(src + 16 * (base + 256 * k));
    } else {
#pragma unroll
      for (int k = 0; k < UNR; ++k)
        v[k] = base + 256 * k < n16 ? nt_load16(src + 16 * (base + 256 * k)) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, kWave);
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

}  // namespace mi

extern "C" int mi_hbm_read(const void* data, int64_t bytes, uint32_t* sink, int32_t grid, void* stream) {
  using namespace mi;
  if (!data || !sink || bytes <= 0 || bytes % 16 || grid <= 0) return MI_ERR_INVALID;
  if (((uintptr_t)data & 15) != 0) return MI_ERR_INVALID;
  hipLaunchKernelGGL(hbm_read_kernel<MI_HBM_READ_UNR>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)data, bytes / 16, sink);
  MI_CHECK_LAUNCH();
  return MI_OK;
}
