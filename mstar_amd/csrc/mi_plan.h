// Split-KV decode plan shared by the decode, pack and prefill translation
// units: the plan workgroup's body, so a caller can run it inside a fused
// launch (pack + plan, prefill plan + decode plan).
#pragma once

#include "mi_internal.h"

namespace mi {

constexpr int kRows = 16;  // MFMA N: query rows per wave

// Which head_dim elements a decode lane holds.  A 16-lane row of a wavefront
// loads one key row with 16-byte loads, each load instruction covering 256
// contiguous bytes (a lane takes 16 bytes at 16*lane%16, then 256 bytes
// further on for the next part), so a lane holds runs of `run` consecutive
// elements, run = min(D/16, 16 / element bytes), and element j of the lane
// with row position i (the MFMA output row, 4*grp + r, or the lane's column
// when it loads) is dim
//   dim_of(run, i, j) = (j / run) * 16 * run + run * i + j % run.
// (Two 16-byte loads 16 bytes apart would touch every 128-byte line of a
// row in both instructions: measured 67% of HBM peak against 79% at
// head_dim 256.)
constexpr int lane_run(int head_dim, int elem_bytes) {
  return head_dim / 16 < 16 / elem_bytes ? head_dim / 16 : 16 / elem_bytes;
}
__host__ __device__ constexpr int dim_of(int run, int i, int j) { return (j / run) * 16 * run + run * i + j % run; }

// Header words written by the plan kernel.
enum { kHdrMagic = 0, kHdrBatch, kHdrChunks, kHdrChunkPages, kHdrMaxChunks };
constexpr int32_t kPlanMagic = 0x4d494450;

struct PlanParams {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* num_pages;  // non-null: per-request page counts (kv_indptr unused)
  const int32_t* kv_indices;
  const int32_t* last_page_len;
  int32_t batch, target, min_chunk_pages, max_chunks, group;
  int32_t slots, floor_pages;  // small jobs: items of down to floor_pages while at most `slots` items
  int32_t short_rows = kShortRowsMax;  // ragged batch: requests with qo_len * group <= short_rows
  int32_t* hdr;
  int32_t* chunk_indptr;
  int4* work;
  int64_t* kv_locations;
};

// Work list order: longest first.  Every request's full items (item_pages
// pages) come first, then the requests' shorter remainder items in
// descending size (64 size buckets, counting sort in LDS): the last
// workgroups to start are the shortest, so the machine drains evenly instead
// of waiting on full-size items that started late.  An item is
// (request, index within the request, end page, items of the request); its
// partial lives at chunk_indptr[request] + index whatever its list position.
constexpr int kSizeBuckets = 64;
// Small jobs cut a request into at most this many items: the merge of its
// partials (one workgroup per request and kv-head) stays short.
constexpr int kMaxSmallItems = 16;

// One 1024-thread workgroup builds the plan.
__device__ inline void decode_plan_body(const PlanParams& p) {
  __shared__ int smem[16];
  __shared__ int s_bucket[kSizeBuckets];
  int total_pages = 0;
  if (p.num_pages) {
    for (int base = 0; base < p.batch; base += 1024) {
      const int b = base + (int)threadIdx.x;
      int tot;
      block_exclusive_scan_1024(b < p.batch ? p.num_pages[b] : 0, tot, smem);
      total_pages += tot;
    }
  } else {
    total_pages = p.kv_indptr[p.batch] - p.kv_indptr[0];
  }
  // items of request b at `c` pages per item (0 for requests this kernel does not serve)
  auto count_of = [&](int b, int c, int& np) {
    np = p.num_pages ? p.num_pages[b] : p.kv_indptr[b + 1] - p.kv_indptr[b];
    int n = np > 0 ? (np + c - 1) / c : 0;
    if (p.qo_indptr) {  // ragged batch: only short-query requests belong to this kernel
      const int qo_len = p.qo_indptr[b + 1] - p.qo_indptr[b];
      if (qo_len <= 0 || qo_len * p.group > p.short_rows) n = 0;
    }
    return n;
  };
  int cp = (total_pages + p.target - 1) / p.target;
  if (cp < p.min_chunk_pages) {
    // A small job: the shortest items, down to floor_pages, whose count still
    // fits one round of resident workgroups, so a handful of requests is not
    // streamed by a handful of workgroups (a one-request decode over 1k
    // tokens would otherwise be one workgroup's work), and no more than
    // kMaxSmallItems items for the longest request.
    // Page counts are read once (batch <= 1024: one request per thread).
    const bool one = p.batch <= 1024;
    int mine = 0;  // pages of this thread's request if this kernel serves it
    if (one && (int)threadIdx.x < p.batch) {
      int np = 0;
      if (count_of((int)threadIdx.x, 1, np) > 0) mine = np;
    }
    auto items_at = [&](int c) {  // the workgroup's item count at c pages per item
      if (one) return block_sum_1024(mine > 0 ? (mine + c - 1) / c : 0, smem);
      int cnt = 0;
      for (int base = 0; base < p.batch; base += 1024) {
        const int b = base + (int)threadIdx.x;
        int np = 0;
        cnt += block_sum_1024(b < p.batch ? count_of(b, c, np) : 0, smem);
      }
      return cnt;
    };
    int longest = 0;
    if (one) {
      longest = block_max_1024(mine, smem);
    } else {
      int m = 0;
      for (int b = (int)threadIdx.x; b < p.batch; b += 1024) {
        int np = 0;
        if (count_of(b, 1, np) > 0) m = max(m, np);
      }
      longest = block_max_1024(m, smem);
    }
    const int hi = p.min_chunk_pages;
    int lo = p.floor_pages;
    if (lo < cp) lo = cp;
    if (lo < (longest + kMaxSmallItems - 1) / kMaxSmallItems) lo = (longest + kMaxSmallItems - 1) / kMaxSmallItems;
    if (lo > hi) lo = hi;
    if (lo < 1) lo = 1;
    // The smallest size in [lo, hi] whose items fit the slots (counts fall as
    // the size grows), or hi when none does.  Uniform across the workgroup:
    // every thread sees the same totals.
    if (lo < hi && items_at(hi) <= p.slots) {
      int h = hi;
      while (lo < h) {
        const int mid = (lo + h) >> 1;
        if (items_at(mid) <= p.slots) h = mid;
        else lo = mid + 1;
      }
      cp = lo;
    } else {
      cp = lo < hi ? hi : lo;
    }
  }
  if (threadIdx.x < kSizeBuckets) s_bucket[threadIdx.x] = 0;
  __syncthreads();
  auto items_of = [&](int b, int& np, int& n, int& full, int& rem_bucket) {
    n = count_of(b, cp, np);
    full = n > 0 ? np / cp : 0;
    const int rem = n > 0 ? np - full * cp : 0;
    rem_bucket = rem > 0 ? (int)(((int64_t)rem * kSizeBuckets - 1) / cp) : -1;
  };
  // pass 1: item offsets per request, full items in place, remainder histogram
  int carry = 0, carry_full = 0;
  for (int base = 0; base < p.batch; base += 1024) {
    const int b = base + (int)threadIdx.x;
    int np = 0, n = 0, full = 0, rb = -1;
    if (b < p.batch) items_of(b, np, n, full, rb);
    int total, total_full;
    const int first = block_exclusive_scan_1024(n, total, smem) + carry;
    const int ffirst = block_exclusive_scan_1024(full, total_full, smem) + carry_full;
    if (b < p.batch) {
      p.chunk_indptr[b] = first;
      for (int c = 0; c < full && ffirst + c < p.max_chunks; ++c) p.work[ffirst + c] = make_int4(b, c, (c + 1) * cp, n);
      if (rb >= 0) atomicAdd(&s_bucket[rb], 1);
      if (p.kv_locations) {
        int64_t page = -1, pos = -1;
        if (np > 0) {
          page = p.kv_indices[p.kv_indptr[b + 1] - 1];
          pos = p.last_page_len[b] - 1;
        }
        p.kv_locations[2 * b] = page;
        p.kv_locations[2 * b + 1] = pos;
      }
    }
    carry += total;
    carry_full += total_full;
  }
  __syncthreads();
  // bucket start positions, largest bucket first, after all full items
  if (threadIdx.x == 0) {
    int off = carry_full;
    for (int k = kSizeBuckets - 1; k >= 0; --k) {
      const int c = s_bucket[k];
      s_bucket[k] = off;
      off += c;
    }
  }
  __syncthreads();
  // pass 2: remainder items
  for (int base = 0; base < p.batch; base += 1024) {
    const int b = base + (int)threadIdx.x;
    if (b < p.batch) {
      int np, n, full, rb;
      items_of(b, np, n, full, rb);
      if (rb >= 0) {
        const int pos = atomicAdd(&s_bucket[rb], 1);
        if (pos < p.max_chunks) p.work[pos] = make_int4(b, full, np, n);
      }
    }
  }
  if (threadIdx.x == 0) {
    p.chunk_indptr[p.batch] = carry;
    p.hdr[kHdrMagic] = kPlanMagic;
    p.hdr[kHdrBatch] = p.batch;
    p.hdr[kHdrChunks] = min(carry, p.max_chunks);
    p.hdr[kHdrChunkPages] = cp;
    p.hdr[kHdrMaxChunks] = p.max_chunks;
  }
}

}  // namespace mi
