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
  CopyPagesParams p{};
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

// ------------------------------------------------------------------------
// Token-range copies between two KV pools, and the KV page wire format.
//
// A record (src page, dst page, tokens [ts, te)) moves, for every layer of
// [layer_begin, layer_end), the K rows ts..te-1 and the V rows ts..te-1 of
// that page.  This is the unit of M*'s remote KV reads: KVReadInfo
// (mstar/engine/kv_store.py:177-183) with the byte arithmetic of
// MooncakeKVTransferEngine._get_ptr_nbytes (kv_store.py:233-259) — one
// contiguous segment of (te - ts) token rows per (layer, K|V) — which the
// reference issues as one transfer per segment (kv_store.py:261-285) or one
// torch copy per record (CudaIpcKVTransferEngine._do_read,
// kv_store.py:330-380).  Full-page records (ts = 0, te = page_size) are CPU
// offload and reload (mstar/engine/cpu_page_pool.py:63-124).  Here every
// segment of a call is one workgroup unit of a single launch.
//
// Wire format (pack/unpack): layer-major, so that a layer range is one
// contiguous block and layers can be sent as they are produced.  With
// rows_i = te_i - ts_i, R = sum rows_i and row_offset[i] = sum_{j<i} rows_j,
// the K rows of record i in layer l start at token row
//   2*R*(l - layer_begin) + 2*row_offset[i]
// and its V rows follow them; a token row is token_stride bytes.
// ------------------------------------------------------------------------
namespace mi {

enum { kSegPoolToPool = 0, kSegPoolToWire = 1, kSegWireToPool = 2 };

struct SegPool {
  uint8_t* data;
  int64_t layer_stride, page_stride, kv_stride, num_pages;
};

struct SegParams {
  SegPool src, dst;
  uint8_t* wire;
  int64_t wire_bytes;
  int64_t row_bytes;
  const int32_t* src_pages;
  const int32_t* dst_pages;
  const int32_t* ts;  // NULL: whole pages
  const int32_t* te;
  const int64_t* row_offset;  // wire modes; NULL: row_offset[i] = i * page_size
  int32_t n, layer_begin, num_layers, page_size;
};

// Byte address of token row `ts` of the K half of (layer, page).
MI_DEVICE uint8_t* seg_page_base(const SegPool& p, int layer, int page, int ts, int64_t row_bytes) {
  return p.data + (int64_t)layer * p.layer_stride + (int64_t)page * p.page_stride + (int64_t)ts * row_bytes;
}

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// Streaming copy: nothing moved here is read again soon, so loads and stores
// are non-temporal (measured ~2% faster than cached ones for pool copies).
template <int MODE>
__global__ __launch_bounds__(256) void kv_segments_kernel(SegParams p) {
  constexpr int U = 8;  // 16-byte vectors in flight per lane
  const int64_t units = (int64_t)p.n * p.num_layers;
  for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
    const int i = (int)(u / p.num_layers);
    const int layer = p.layer_begin + (int)(u - (int64_t)i * p.num_layers);
    int ts = 0, te = p.page_size;
    if (p.ts) {
      ts = p.ts[i];
      te = p.te[i];
    }
    if (ts < 0 || te > p.page_size || te <= ts) continue;
    const int rows = te - ts;
    const int64_t seg = (int64_t)rows * p.row_bytes;  // bytes of one half
    const uint8_t* from[2];
    uint8_t* to[2];
    if (MODE != kSegWireToPool) {
      const int sp = p.src_pages[i];
      if (sp < 0 || sp >= p.src.num_pages) continue;
      from[0] = seg_page_base(p.src, layer, sp, ts, p.row_bytes);
      from[1] = from[0] + p.src.kv_stride;
    }
    if (MODE != kSegPoolToWire) {
      const int dp = p.dst_pages[i];
      if (dp < 0 || dp >= p.dst.num_pages) continue;
      to[0] = seg_page_base(p.dst, layer, dp, ts, p.row_bytes);
      to[1] = to[0] + p.dst.kv_stride;
    }
    if (MODE != kSegPoolToPool) {
      int64_t r0, total;
      if (p.row_offset) {
        r0 = p.row_offset[i];
        total = p.row_offset[p.n];
        if (r0 < 0 || p.row_offset[i + 1] - r0 != rows) continue;  // inconsistent offsets
      } else {
        r0 = (int64_t)i * p.page_size;
        total = (int64_t)p.n * p.page_size;
      }
      const int64_t at = (2 * total * (layer - p.layer_begin) + 2 * r0) * p.row_bytes;
      if (at < 0 || at + 2 * seg > p.wire_bytes) continue;
      if (MODE == kSegPoolToWire) {
        to[0] = p.wire + at;
        to[1] = to[0] + seg;
      } else {
        from[0] = p.wire + at;
        from[1] = from[0] + seg;
      }
    }
    const int64_t nv = seg / 16;  // vectors per half
    for (int64_t v0 = threadIdx.x; v0 < 2 * nv; v0 += 256 * U) {
      u32x4 t[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int64_t v = v0 + 256 * k;
        if (v < 2 * nv) {
          const int h = v >= nv;
          t[k] = __builtin_nontemporal_load((const u32x4*)(from[h] + 16 * (v - h * nv)));
        }
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int64_t v = v0 + 256 * k;
        if (v < 2 * nv) {
          const int h = v >= nv;
          __builtin_nontemporal_store(t[k], (u32x4*)(to[h] + 16 * (v - h * nv)));
        }
      }
    }
  }
}

// Memory a kernel may touch: HIP device memory, or host memory that HIP
// allocated pinned (reachable over the bus at the same address).  Pageable
// host memory is not.
static bool device_reachable(const void* ptr) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeHost || a.type == hipMemoryTypeManaged;
}

static int seg_pool_check(const mi_kv_pool* p, int32_t layer_end) {
  if (!p || !p->data) return MI_ERR_INVALID;
  if ((uintptr_t)p->data % 16 || p->layer_stride % 16 || p->page_stride % 16 || p->kv_stride % 16 ||
      p->token_stride % 16 || p->token_stride <= 0 || p->page_size <= 0 || p->num_pages <= 0 ||
      p->num_layers <= 0 || layer_end > p->num_layers)
    return MI_ERR_INVALID;
  if (p->kv_stride < (int64_t)p->page_size * p->token_stride) return MI_ERR_INVALID;  // halves overlap
  return device_reachable(p->data) ? MI_OK : MI_ERR_INVALID;
}

static SegPool seg_pool(const mi_kv_pool* p) {
  SegPool s;
  s.data = (uint8_t*)p->data;
  s.layer_stride = p->layer_stride;
  s.page_stride = p->page_stride;
  s.kv_stride = p->kv_stride;
  s.num_pages = p->num_pages;
  return s;
}

template <int MODE>
static int seg_launch(SegParams& p, hipStream_t stream) {
  const int64_t units = (int64_t)p.n * p.num_layers;
  const int grid = (int)(units < 16384 ? units : 16384);
  hipLaunchKernelGGL(kv_segments_kernel<MODE>, dim3(grid), dim3(256), 0, stream, p);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

static int seg_common(const mi_kv_pool* pool, const int32_t* token_start, const int32_t* token_end,
                      int32_t num_records, int32_t layer_begin, int32_t layer_end, SegParams& p) {
  if (num_records < 0 || layer_begin < 0 || layer_end < layer_begin) return MI_ERR_INVALID;
  if ((token_start == nullptr) != (token_end == nullptr)) return MI_ERR_INVALID;
  if (const int rc = seg_pool_check(pool, layer_end)) return rc;
  p.ts = token_start;
  p.te = token_end;
  p.n = num_records;
  p.layer_begin = layer_begin;
  p.num_layers = layer_end - layer_begin;
  p.page_size = pool->page_size;
  p.row_bytes = pool->token_stride;
  p.wire = nullptr;
  p.wire_bytes = 0;
  p.row_offset = nullptr;
  p.src_pages = p.dst_pages = nullptr;
  return MI_OK;
}

}  // namespace mi

extern "C" int mi_kv_copy_tokens(const mi_kv_pool* src, const mi_kv_pool* dst, const int32_t* src_pages,
                                 const int32_t* dst_pages, const int32_t* token_start, const int32_t* token_end,
                                 int32_t num_records, int32_t layer_begin, int32_t layer_end, void* stream) {
  using namespace mi;
  SegParams p{};
  if (const int rc = seg_common(src, token_start, token_end, num_records, layer_begin, layer_end, p)) return rc;
  if (const int rc = seg_pool_check(dst, layer_end)) return rc;
  if (dst->token_stride != src->token_stride || dst->page_size != src->page_size) return MI_ERR_INVALID;
  if (num_records == 0 || layer_end == layer_begin) return MI_OK;
  if (!src_pages || !dst_pages) return MI_ERR_INVALID;
  p.src = seg_pool(src);
  p.dst = seg_pool(dst);
  p.src_pages = src_pages;
  p.dst_pages = dst_pages;
  return seg_launch<kSegPoolToPool>(p, (hipStream_t)stream);
}

extern "C" int mi_kv_wire_pack(const mi_kv_pool* pool, const int32_t* pages, const int32_t* token_start,
                               const int32_t* token_end, const int64_t* row_offset, int32_t num_records,
                               int32_t layer_begin, int32_t layer_end, void* wire, int64_t wire_bytes,
                               void* stream) {
  using namespace mi;
  SegParams p{};
  if (const int rc = seg_common(pool, token_start, token_end, num_records, layer_begin, layer_end, p)) return rc;
  if (token_start && !row_offset) return MI_ERR_INVALID;
  if (num_records == 0 || layer_end == layer_begin) return MI_OK;
  if (!pages || !wire || wire_bytes < 0 || (uintptr_t)wire % 16 || !device_reachable(wire)) return MI_ERR_INVALID;
  p.src = seg_pool(pool);
  p.src_pages = pages;
  p.wire = (uint8_t*)wire;
  p.wire_bytes = wire_bytes;
  p.row_offset = row_offset;
  return seg_launch<kSegPoolToWire>(p, (hipStream_t)stream);
}

extern "C" int mi_kv_wire_unpack(const void* wire, int64_t wire_bytes, const mi_kv_pool* pool,
                                 const int32_t* pages, const int32_t* token_start, const int32_t* token_end,
                                 const int64_t* row_offset, int32_t num_records, int32_t layer_begin,
                                 int32_t layer_end, void* stream) {
  using namespace mi;
  SegParams p{};
  if (const int rc = seg_common(pool, token_start, token_end, num_records, layer_begin, layer_end, p)) return rc;
  if (token_start && !row_offset) return MI_ERR_INVALID;
  if (num_records == 0 || layer_end == layer_begin) return MI_OK;
  if (!pages || !wire || wire_bytes < 0 || (uintptr_t)wire % 16 || !device_reachable(wire)) return MI_ERR_INVALID;
  p.dst = seg_pool(pool);
  p.dst_pages = pages;
  p.wire = (uint8_t*)wire;
  p.wire_bytes = wire_bytes;
  p.row_offset = row_offset;
  return seg_launch<kSegWireToPool>(p, (hipStream_t)stream);
}
