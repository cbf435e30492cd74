// Page-to-page KV copies (BatchedCacheManager.snapshot_all).
//
// Replaces the per-page torch copies of snapshot_all
// (mstar/engine/cache_manager.py:840-870: kv_cache[:, dst] = kv_cache[:, src]
// for each (src, dst) pair, all layers) with one launch: every (pair, layer)
// page is moved in 16-byte vectors by a grid-stride loop.  Pages whose ids
// fall outside [0, max_pages) are skipped.
#include "mi_common.h"

namespace mi {

struct CopyPagesParams {
  uint8_t* pool;
  int64_t layer_stride, page_stride, page_vecs, max_pages;
  const int32_t* src;
  const int32_t* dst;
  int32_t n, layers;
};

__global__ __launch_bounds__(256) void copy_pages_kernel(CopyPagesParams p) {
  const int64_t per_pair = p.page_vecs * p.layers;
  const int64_t total = per_pair * p.n;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int pair = (int)(i / per_pair);
    const int64_t r = i - pair * per_pair;
    const int layer = (int)(r / p.page_vecs);
    const int64_t v = r - (int64_t)layer * p.page_vecs;
    const int s = p.src[pair], d = p.dst[pair];
    if (s < 0 || s >= p.max_pages || d < 0 || d >= p.max_pages) continue;
    const uint8_t* from = p.pool + layer * p.layer_stride + s * p.page_stride + 16 * v;
    uint8_t* to = p.pool + layer * p.layer_stride + d * p.page_stride + 16 * v;
    *(uint4*)to = *(const uint4*)from;
  }
}

}  // namespace mi

extern "C" int mi_copy_pages(void* pool, int64_t layer_stride_bytes, int32_t num_layers, int64_t page_stride_bytes,
                             int64_t page_bytes, int64_t max_pages, const int32_t* src_pages,
                             const int32_t* dst_pages, int32_t num_pairs, void* stream) {
  using namespace mi;
  if (num_pairs < 0 || num_layers < 0 || page_bytes < 0 || max_pages < 0) return MI_ERR_INVALID;
  if (num_pairs == 0 || num_layers == 0 || page_bytes == 0) return MI_OK;
  if (!pool || !src_pages || !dst_pages) return MI_ERR_INVALID;
  if ((uintptr_t)pool % 16 || layer_stride_bytes % 16 || page_stride_bytes % 16 || page_bytes % 16 ||
      page_bytes > page_stride_bytes)
    return MI_ERR_INVALID;
  CopyPagesParams p;
  p.pool = (uint8_t*)pool;
  p.layer_stride = layer_stride_bytes;
  p.page_stride = page_stride_bytes;
  p.page_vecs = page_bytes / 16;
  p.max_pages = max_pages;
  p.src = src_pages;
  p.dst = dst_pages;
  p.n = num_pairs;
  p.layers = num_layers;
  const int64_t total = p.page_vecs * num_layers * (int64_t)num_pairs;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  MI_CHECK_LAUNCH();
  return MI_OK;
}
