// Per-step batch packing (P1) on the GPU.
//
// Replaces the per-request Python loop of
// BatchedCacheManager._plan_attention_impl (mstar/engine/cache_manager.py:272-322)
// and its host->device copies.  Page ids stay owned by the host FIFO
// allocator (mstar/engine/kv_store.py:25-67, 463-482); a device block table
// keeps every live request's page list, and this kernel flattens the batch
// from it every step.  Pages allocated since the previous step arrive with
// the step's metadata and are written into the table by the same kernel.
//
// Every workgroup recomputes the exclusive prefix sums (new tokens, pages
// and newly sent pages per request) in LDS, so the grid needs no
// inter-block synchronisation; the flattening of kv_indices is then shared
// by all workgroups (grid-stride over the batch's pages, one binary search
// in LDS per page id; the grid is sized for about one page per thread).
#include <cstring>

#include "mi_common.h"
#include "mi_internal.h"
#include "mi_plan.h"

namespace mi {

constexpr int kPackThreads = 1024;

struct PackParams {
  const int32_t* req_slot;
  const int32_t* seq_len;
  const int32_t* new_len;
  const int32_t* num_pages;
  const int32_t* table_pages;  // leading pages already in the table (NULL: all)
  const int32_t* new_pages;    // the rest, request by request
  int32_t* block_table;
  int64_t bt_stride;
  int32_t* qo_indptr;
  int32_t* kv_indptr;
  int32_t* kv_indices;
  int32_t* last_page_len;
  int64_t* kv_locations;
  int32_t batch, page_size;
};

// Workgroup `block` of `nblocks` packing workgroups.
__device__ inline void pack_body(const PackParams& p, int block, int nblocks) {
  __shared__ int s_scan[16];
  __shared__ int s_off[kPackThreads + 1];  // window-relative exclusive page offsets
  __shared__ int s_slot[kPackThreads];
  __shared__ int s_old[kPackThreads];      // pages of the request already in the table
  __shared__ int s_noff[kPackThreads];     // window-relative offsets into new_pages
  const int tid = threadIdx.x;
  int carry_qo = 0, carry_kv = 0, carry_new = 0;
  for (int base = 0; base < p.batch; base += kPackThreads) {
    const int b = base + tid;
    const bool live = b < p.batch;
    const int sl = live ? p.new_len[b] : 0;
    const int np = live ? p.num_pages[b] : 0;
    const int old = live ? (p.table_pages ? min(p.table_pages[b], np) : np) : 0;
    int tot_qo, tot_kv, tot_new;
    const int ex_qo = block_exclusive_scan_1024(sl, tot_qo, s_scan);
    const int ex_kv = block_exclusive_scan_1024(np, tot_kv, s_scan);
    const int ex_new = block_exclusive_scan_1024(np - old, tot_new, s_scan);
    s_off[tid] = ex_kv;
    s_slot[tid] = live ? p.req_slot[b] : 0;
    s_old[tid] = old;
    s_noff[tid] = ex_new;
    if (tid == 0) s_off[kPackThreads] = tot_kv;
    if (block == 0 && live) {
      p.qo_indptr[b] = carry_qo + ex_qo;
      p.kv_indptr[b] = carry_kv + ex_kv;
      const int T = p.seq_len[b] + sl;
      int lpl = T % p.page_size;
      if (lpl == 0) lpl = p.page_size;
      p.last_page_len[b] = lpl;
      if (p.kv_locations && sl == 1) {
        // (last page of the request's list, last_page_len - 1): cache_manager.py:293-294
        int64_t page = -1, pos = -1;
        if (np > 0) {
          page = np - 1 < old ? p.block_table[(int64_t)s_slot[tid] * p.bt_stride + (np - 1)]
                              : p.new_pages[carry_new + ex_new + (np - 1 - old)];
          pos = lpl - 1;
        }
        p.kv_locations[2 * b] = page;
        p.kv_locations[2 * b + 1] = pos;
      }
    }
    __syncthreads();
    // flatten this window's page lists: kv_indices[carry_kv + f] for f < tot_kv;
    // pages past a request's table prefix come from new_pages and go into the table
    const int nreq = min(kPackThreads, p.batch - base);
    for (int f = block * kPackThreads + tid; f < tot_kv; f += nblocks * kPackThreads) {
      int lo = 0, hi = nreq - 1;  // last r with s_off[r] <= f
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= f) lo = mid; else hi = mid - 1;
      }
      const int j = f - s_off[lo];
      int32_t* row = p.block_table + (int64_t)s_slot[lo] * p.bt_stride;
      int page;
      if (j < s_old[lo]) {
        page = row[j];
      } else {
        page = p.new_pages[carry_new + s_noff[lo] + (j - s_old[lo])];
        row[j] = page;
      }
      p.kv_indices[carry_kv + f] = page;
    }
    carry_qo += tot_qo;
    carry_kv += tot_kv;
    carry_new += tot_new;
    __syncthreads();
  }
  if (block == 0 && tid == 0) {
    p.qo_indptr[p.batch] = carry_qo;
    p.kv_indptr[p.batch] = carry_kv;
  }
}

__global__ __launch_bounds__(kPackThreads) void pack_kernel(PackParams p) { pack_body(p, blockIdx.x, gridDim.x); }

// Pack and split-KV decode plan in one launch: workgroup 0 plans from the
// per-request page counts (it needs none of the pack's outputs), the others
// pack.
__global__ __launch_bounds__(kPackThreads) void pack_plan_kernel(PackParams p, PlanParams pl) {
  if (blockIdx.x == 0) {
    decode_plan_body(pl);
    return;
  }
  pack_body(p, blockIdx.x - 1, gridDim.x - 1);
}

// The step's metadata as a kernel argument (mi_pack_plan_host): up to
// MI_PACK_HOST_ARGS int32 values, either as given, [slot | seq_len | new_len |
// num_pages | pages on the device] (batch each) followed by the new pages, or
// compact, [seq_len | slot + num_pages * 2^16 | new_len + pages on the device
// * 2^16] (batch each) followed by the new pages.
static_assert(MI_PACK_HOST_ARGS >= MI_PACK_HOST_META, "the argument holds any metadata of MI_PACK_HOST_META values");
constexpr int kHostCompactMax = MI_PACK_HOST_ARGS / 3;  // requests of a compact step
struct HostMeta {
  int32_t v[MI_PACK_HOST_ARGS];
};

// pack_plan_kernel over the argument copy; with_plan == 0: pack only (no plan
// workgroup).  Every workgroup copies the per-request fields but seq_len into
// LDS (unpacking the compact form), so each of the kernel's array pointers
// has one address space whichever form arrived (a pointer that could be
// either the argument or LDS made the compiler copy the whole argument to
// scratch memory in every lane).
__global__ __launch_bounds__(kPackThreads) void pack_plan_host_kernel(PackParams p, PlanParams pl, HostMeta m,
                                                                      int32_t with_plan, int32_t compact) {
  __shared__ int32_t s_meta[4][kHostCompactMax];
  const int32_t* base = m.v;
  const int b = p.batch;
  for (int r = (int)threadIdx.x; r < b; r += kPackThreads) {
    if (compact) {
      const uint32_t a = (uint32_t)base[b + r], c = (uint32_t)base[2 * b + r];
      s_meta[0][r] = (int32_t)(a & 0xffffu);  // slot
      s_meta[1][r] = (int32_t)(c & 0xffffu);  // new tokens
      s_meta[2][r] = (int32_t)(a >> 16);      // pages
      s_meta[3][r] = (int32_t)(c >> 16);      // pages on the device
    } else {
      s_meta[0][r] = base[r];
      s_meta[1][r] = base[2 * b + r];
      s_meta[2][r] = base[3 * b + r];
      s_meta[3][r] = base[4 * b + r];
    }
  }
  __syncthreads();
  p.req_slot = s_meta[0];
  p.new_len = s_meta[1];
  p.num_pages = s_meta[2];
  p.table_pages = s_meta[3];
  p.seq_len = compact ? base : base + b;
  p.new_pages = base + (compact ? 3 : 5) * b;
  if (with_plan) {
    if (blockIdx.x == 0) {
      pl.num_pages = p.num_pages;
      decode_plan_body(pl);
      return;
    }
    pack_body(p, blockIdx.x - 1, gridDim.x - 1);
  } else {
    pack_body(p, blockIdx.x, gridDim.x);
  }
}

__global__ __launch_bounds__(256) void block_table_update_kernel(int32_t* table, int64_t stride,
                                                                 const int32_t* slot, const int32_t* pos,
                                                                 const int32_t* page, int32_t n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) table[(int64_t)slot[i] * stride + pos[i]] = page[i];
}

static int pack_params(const int32_t* req_slot, const int32_t* seq_len, const int32_t* new_len,
                       const int32_t* num_pages, int32_t batch, int32_t* block_table, int64_t block_table_stride,
                       const int32_t* table_pages, const int32_t* new_pages, int32_t page_size, int32_t* qo_indptr,
                       int32_t* kv_indptr, int32_t* kv_indices, int32_t* last_page_len, int64_t* kv_locations,
                       int32_t grid_blocks, PackParams* out) {
  if (batch < 0 || page_size <= 0 || grid_blocks <= 0 || block_table_stride <= 0) return MI_ERR_INVALID;
  if (!qo_indptr || !kv_indptr || !last_page_len) return MI_ERR_INVALID;
  if (batch > 0 && (!req_slot || !seq_len || !new_len || !num_pages || !block_table || !kv_indices))
    return MI_ERR_INVALID;
  if (table_pages && !new_pages) return MI_ERR_INVALID;
  PackParams& pp = *out;
  pp.req_slot = req_slot;
  pp.seq_len = seq_len;
  pp.new_len = new_len;
  pp.num_pages = num_pages;
  pp.table_pages = table_pages;
  pp.new_pages = new_pages;
  pp.block_table = block_table;
  pp.bt_stride = block_table_stride;
  pp.qo_indptr = qo_indptr;
  pp.kv_indptr = kv_indptr;
  pp.kv_indices = kv_indices;
  pp.last_page_len = last_page_len;
  pp.kv_locations = kv_locations;
  pp.batch = batch;
  pp.page_size = page_size;
  return MI_OK;
}

}  // namespace mi

extern "C" int mi_pack(const int32_t* req_slot, const int32_t* seq_len, const int32_t* new_len,
                       const int32_t* num_pages, int32_t batch, int32_t* block_table,
                       int64_t block_table_stride, const int32_t* table_pages, const int32_t* new_pages,
                       int32_t page_size, int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
                       int32_t* last_page_len, int64_t* kv_locations, int32_t grid_blocks, void* stream) {
  using namespace mi;
  PackParams pp{};
  const int st = pack_params(req_slot, seq_len, new_len, num_pages, batch, block_table, block_table_stride,
                             table_pages, new_pages, page_size, qo_indptr, kv_indptr, kv_indices, last_page_len,
                             kv_locations, grid_blocks, &pp);
  if (st != MI_OK) return st;
  hipLaunchKernelGGL(pack_kernel, dim3(grid_blocks), dim3(kPackThreads), 0, (hipStream_t)stream, pp);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

extern "C" int mi_pack_plan(const int32_t* req_slot, const int32_t* seq_len, const int32_t* new_len,
                            const int32_t* num_pages, int32_t batch, int32_t* block_table,
                            int64_t block_table_stride, const int32_t* table_pages, const int32_t* new_pages,
                            int32_t page_size, int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
                            int32_t* last_page_len, int64_t* kv_locations, int32_t grid_blocks,
                            int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  using namespace mi;
  PackParams pp{};
  int st = pack_params(req_slot, seq_len, new_len, num_pages, batch, block_table, block_table_stride, table_pages,
                       new_pages, page_size, qo_indptr, kv_indptr, kv_indices, last_page_len, kv_locations,
                       grid_blocks, &pp);
  if (st != MI_OK) return st;
  PlanParams pl{};
  st = decode_plan_params(nullptr, kv_indptr, kv_indices, last_page_len, batch, page_size, num_qo_heads,
                          num_kv_heads, head_dim, nullptr, workspace, workspace_bytes, 0, &pl);
  if (st != MI_OK) return st;
  pl.num_pages = num_pages;  // the plan reads the step's page counts, not the pack's outputs
  hipLaunchKernelGGL(pack_plan_kernel, dim3(grid_blocks + 1), dim3(kPackThreads), 0, (hipStream_t)stream, pp, pl);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

extern "C" int mi_pack_plan_host(const int32_t* meta, int32_t meta_len, int32_t batch, int32_t* block_table,
                                 int64_t block_table_stride, int32_t page_size, int32_t* qo_indptr,
                                 int32_t* kv_indptr, int32_t* kv_indices, int32_t* last_page_len,
                                 int64_t* kv_locations, int32_t grid_blocks, int32_t num_qo_heads,
                                 int32_t num_kv_heads, int32_t head_dim, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  using namespace mi;
  if (!meta || batch < 0 || meta_len > MI_PACK_HOST_META_MAX || (int64_t)meta_len < 5LL * batch)
    return MI_ERR_INVALID;
  // the new pages the kernel will read are exactly the ones meta carries
  int64_t new_pages = 0;
  bool fits16 = true;  // slot, new tokens, pages and pages on the device below 2^16
  for (int32_t r = 0; r < batch; ++r) {
    const int32_t slot = meta[r], sl = meta[2 * batch + r], np = meta[3 * batch + r], old = meta[4 * batch + r];
    if (np < 0 || old < 0) return MI_ERR_INVALID;
    new_pages += np - (old < np ? old : np);
    fits16 = fits16 && (uint32_t)slot < 65536u && (uint32_t)sl < 65536u && np < 65536 && old < 65536;
  }
  if (new_pages != (int64_t)meta_len - 5LL * batch) return MI_ERR_INVALID;
  HostMeta m;
  int32_t compact = 0;
  if (meta_len <= MI_PACK_HOST_ARGS) {
    memcpy(m.v, meta, sizeof(int32_t) * (size_t)meta_len);
  } else if (fits16 && batch <= kHostCompactMax && 3LL * batch + new_pages <= MI_PACK_HOST_ARGS) {
    compact = 1;
    for (int32_t r = 0; r < batch; ++r) {
      m.v[r] = meta[batch + r];
      m.v[batch + r] = (int32_t)((uint32_t)meta[r] | ((uint32_t)meta[3 * batch + r] << 16));
      m.v[2 * batch + r] = (int32_t)((uint32_t)meta[2 * batch + r] | ((uint32_t)meta[4 * batch + r] << 16));
    }
    memcpy(m.v + 3 * batch, meta + 5 * batch, sizeof(int32_t) * (size_t)new_pages);
  } else {
    return MI_ERR_UNSUPPORTED;  // the caller copies the metadata to the device (mi_pack_plan)
  }
  // pointers for the argument checks only: the kernel points them at its copy of meta
  const int32_t* chk = batch > 0 ? meta : nullptr;
  PackParams pp{};
  int st = pack_params(chk, chk, chk, chk, batch, block_table, block_table_stride, chk, chk, page_size, qo_indptr,
                       kv_indptr, kv_indices, last_page_len, kv_locations, grid_blocks, &pp);
  if (st != MI_OK) return st;
  PlanParams pl{};
  const int with_plan = workspace != nullptr;
  if (with_plan) {
    st = decode_plan_params(nullptr, kv_indptr, kv_indices, last_page_len, batch, page_size, num_qo_heads,
                            num_kv_heads, head_dim, nullptr, workspace, workspace_bytes, 0, &pl);
    if (st != MI_OK) return st;
  }
  hipLaunchKernelGGL(pack_plan_host_kernel, dim3(grid_blocks + with_plan), dim3(kPackThreads), 0,
                     (hipStream_t)stream, pp, pl, m, with_plan, compact);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

extern "C" int mi_block_table_update(int32_t* block_table, int64_t stride, const int32_t* slot,
                                     const int32_t* pos, const int32_t* page, int32_t n, void* stream) {
  if (n < 0 || stride <= 0) return MI_ERR_INVALID;
  if (n == 0) return MI_OK;
  if (!block_table || !slot || !pos || !page) return MI_ERR_INVALID;
  hipLaunchKernelGGL(mi::block_table_update_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, block_table, stride, slot, pos, page, n);
  MI_CHECK_LAUNCH();
  return MI_OK;
}
