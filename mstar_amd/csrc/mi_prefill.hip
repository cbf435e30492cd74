// Ragged paged prefill (P3 + P7) for MI355X (gfx950).
//
// Replaces FlashInferPrefillWrapper.plan/run (mstar/utils/flashinfer_utils.py:162-269).
//
// plan:  one launch (prefill_plan_kernel): the token map (the per-new-token
//        (page, slot) of flashinfer_utils.py:211-256), the tiles of every
//        long-query request, costed and cut as (kv-head, tile) units into 8
//        cost-balanced per-XCD queues, and, for the short-query requests
//        (qo_len * group <= 16, e.g. the decode rows of a mixed batch), a
//        split-KV plan for the decode kernel in the same workspace.
// run:   mi_prefill_short (decode kernel + merge for the short-query
//        requests) and mi_prefill_tiles (prefill_kernel).
//
// prefill_kernel (persistent, one workgroup per CU): a unit is a tile of
// 256 (query token, q-head) rows of one request and kv-head -- GQA rows
// packed token-major, so K/V are read once per group of q-heads -- and each
// of the 8 wavefronts owns 2 groups of 16 rows.  Keys go in 32-key steps
// through a three-stage LDS ring filled from registers loaded two steps
// ahead (page ids staged in LDS, so no load waits on an index load); a
// tile's V^T fragments are read in the step that computes its scores and
// consumed by the next step's P.V MFMAs:
//   S^T[16 keys x 16 rows] = K . Q^T    (v_mfma_f32_16x16x32, K from LDS)
//   online softmax in fp32 (exp2 domain), causal mask aligned to the end of the KV
//   O^T[16 dims x 16 rows] += V^T . P^T (v_mfma_f32_16x16x32, V^T from the
//                                        transposing LDS read ds_read_b64_tr_b16)
// The two wavefronts of each SIMD run their softmax on opposite sides of
// their MFMA work (ping-pong), so vector and matrix work overlap.
// At head_dim 256, prefill_rs_kernel (mi_prefill_rs.h) runs the same units
// (128-row tiles), plan, queues, loader and LDS ring with the work split by
// role inside each wavefront pair: one computes the scores and the softmax
// of 32 rows, the other accumulates their P.V over all 256 dims.
// fp8 K/V are converted to the MFMA type when a tile is stored to LDS; the
// per-head scales multiply the scores and the output.
#include "mi_prefill_kernel.h"
#include "mi_prefill_rs.h"

namespace mi {
constexpr int kShortRows = kShortRowsMax;  // qo_len * group <= 16 -> decode kernel (8 on a paired plan)

// Workspace: header | per-XCD queue counters + finished-workgroup counter |
// tile list | tile cost prefix | unit order | decode split plan.
// Header words: [0] tiles, [1] units (tiles x kv-heads), [8 + x] first unit
// of XCD x's queue (x = 0..8, [16] = units).
struct PrefillLayout {
  int64_t hdr, ctr, tiles, tcum, order, split;
  int32_t max_tiles;
};

static PrefillLayout prefill_layout(int32_t batch, int32_t max_qo_tokens, int32_t group, int32_t nkv,
                                    int32_t head_dim) {
  const int tile_rows = pf_rows(head_dim);
  PrefillLayout L;
  const int64_t rows = (int64_t)max_qo_tokens * group;
  int64_t mt = (rows + tile_rows - 1) / tile_rows + batch;
  if (mt > (1 << 21)) mt = 1 << 21;
  L.max_tiles = (int32_t)mt;
  L.hdr = 0;
  L.ctr = 256;
  L.tiles = L.ctr + 9 * kCtrStride * 4;
  L.tcum = mi_align_up(L.tiles + 8LL * L.max_tiles, 256);
  L.order = mi_align_up(L.tcum + 4LL * (L.max_tiles + 1), 256);
  L.split = mi_align_up(L.order + 4LL * L.max_tiles * nkv, 256);
  return L;
}

// ------------------------------------------------------------ token map
struct TokenMapArgs {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* last_page_len;
  int32_t batch, page_size;
  int64_t* t2p;
  int64_t* t2c;
  int32_t map_len;
};

__device__ inline void token_map_body(const TokenMapArgs& m, int t) {
  const int32_t* qo_indptr = m.qo_indptr;
  const int32_t* kv_indptr = m.kv_indptr;
  const int32_t* kv_indices = m.kv_indices;
  const int32_t* last_page_len = m.last_page_len;
  const int batch = m.batch, page_size = m.page_size;
  int64_t* t2p = m.t2p;
  int64_t* t2c = m.t2c;
  if (t >= m.map_len) return;
  const int total = qo_indptr[batch];
  if (t >= total) {  // graph-mode tail (flashinfer_utils.py:251-253)
    t2p[t] = 0;
    t2c[t] = 0;
    return;
  }
  int lo = 0, hi = batch - 1;  // last request r with qo_indptr[r] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qo_indptr[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int r = lo;
  const int qo_len = qo_indptr[r + 1] - qo_indptr[r];
  const int np = kv_indptr[r + 1] - kv_indptr[r];
  const int kv_len = (np - 1) * page_size + last_page_len[r];
  const int g = kv_len - qo_len + (t - qo_indptr[r]);  // absolute position of the new token
  if (g < 0 || g / page_size >= np) {  // inconsistent metadata: nothing to write
    t2p[t] = -1;
    t2c[t] = -1;
    return;
  }
  t2p[t] = kv_indices[kv_indptr[r] + g / page_size];
  t2c[t] = g % page_size;
}

// ------------------------------------------------------------ tile plan
// Tiles of tile_rows (token, q-head) rows, request by request, heaviest
// (latest rows, most keys under the causal mask) first within a request.
// A tile's cost is its number of 32-key steps.  Units (kv-head, tile) in
// head-major order are cut into 8 contiguous runs of equal cost, one queue
// per XCD, so each XCD's L2 serves few (request, head) KV streams and the
// XCDs finish together; within a queue the units are taken heaviest first
// (longest-processing-time order), so the kernel's tail holds short units.
__device__ int pf_tile_cost(int kv_len, int qo_len, int rows_total, int row0, int tile_rows, int group,
                            int causal) {
  const int last_row = min(row0 + tile_rows, rows_total) - 1;
  const int kv_end = causal ? min(kv_len, kv_len - qo_len + last_row / group + 1) : kv_len;
  return kv_end > 0 ? (kv_end + kPfKeys - 1) / kPfKeys : 0;
}

struct PfPlanArgs {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int32_t batch, page_size, group, nkv, tile_rows, max_tiles, causal;
  int32_t short_rows;  // requests with qo_len * group <= short_rows are the decode plan's, not tiles
  int32_t* hdr;
  int2* tiles;
  int32_t* tcum;
  int32_t* order;
  int32_t* ctr;
};

// One 1024-thread workgroup.  Requests go in windows of 1024 (one per
// thread: tile count, exclusive scan); the window's tiles are then listed
// 1024 at a time, one per thread, each finding its request by a binary
// search over the window's scan in LDS, so no thread loops over a long
// request's tiles.
__device__ inline void prefill_plan_body(const PfPlanArgs& a) {
  __shared__ int smem[16];
  __shared__ int s_cut[9];
  __shared__ int s_first[1025];  // window-relative first tile of each request, [1024] = window total
  __shared__ int s_kvl[1024], s_qol[1024];
  __shared__ int s_bin[8 * 1024];
  const int tid = (int)threadIdx.x;
  const int group = a.group, tile_rows = a.tile_rows, causal = a.causal, max_tiles = a.max_tiles;
  int carry = 0, carry_cost = 0;
  for (int base = 0; base < a.batch; base += 1024) {
    const int b = base + tid;
    int n = 0;
    if (b < a.batch) {
      const int qo_len = a.qo_indptr[b + 1] - a.qo_indptr[b];
      const int rows = qo_len * group;
      n = rows > a.short_rows ? (rows + tile_rows - 1) / tile_rows : 0;
      s_qol[tid] = qo_len;
      s_kvl[tid] = (a.kv_indptr[b + 1] - a.kv_indptr[b] - 1) * a.page_size + a.last_page_len[b];
    }
    int total;
    s_first[tid] = block_exclusive_scan_1024(n, total, smem);
    if (tid == 0) s_first[1024] = total;
    __syncthreads();
    const int nreq = min(1024, a.batch - base);
    for (int j0 = 0; j0 < total; j0 += 1024) {
      const int j = j0 + tid;
      int cost = 0, r = 0, row0 = 0;
      if (j < total) {
        int lo = 0, hi = nreq - 1;  // last request whose first tile is <= j (it has tiles)
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_first[mid] <= j) lo = mid; else hi = mid - 1;
        }
        r = lo;
        const int nr = s_first[r + 1] - s_first[r];
        row0 = (nr - 1 - (j - s_first[r])) * tile_rows;
        cost = pf_tile_cost(s_kvl[r], s_qol[r], s_qol[r] * group, row0, tile_rows, group, causal);
      }
      int tot_cost;
      const int cum = block_exclusive_scan_1024(cost, tot_cost, smem);
      if (j < total && carry + j < max_tiles) {
        a.tiles[carry + j] = make_int2(base + r, row0);
        a.tcum[carry + j] = carry_cost + cum;
      }
      carry_cost += tot_cost;
    }
    carry += total;
    __syncthreads();  // s_first / s_kvl / s_qol are rewritten by the next window
  }
  const int n_tiles = min(carry, max_tiles);
  if (tid == 0) a.tcum[n_tiles] = carry_cost;  // truncated lists keep a consistent prefix end
  __threadfence_block();
  __syncthreads();
  const int64_t ct = carry_cost;
  const int64_t units = (int64_t)n_tiles * a.nkv;
  const int64_t total = ct * a.nkv;
  if (tid == 0) {
    a.hdr[0] = n_tiles;
    a.hdr[1] = (int32_t)units;
  }
  // Queue cuts: queue x starts at the first unit whose cost prefix
  // h*ct + tcum[t] (unit u = h*n_tiles + t) reaches ceil(x * total / 8).
  // The prefix never decreases, so that unit is the one u with
  // prefix(u-1) < target <= prefix(u); every thread tests its units.
  if (tid <= 8) s_cut[tid] = tid == 0 ? 0 : (int)units;
  __syncthreads();
  if (total > 0) {
    auto prefix = [&](int64_t u) -> int64_t {
      const int64_t h = u / n_tiles, t = u - h * n_tiles;
      return h * ct + a.tcum[t];
    };
    for (int64_t u = 1 + tid; u < units; u += 1024) {
      const int64_t pu = prefix(u), pp = prefix(u - 1);
#pragma unroll
      for (int x = 1; x < 8; ++x) {
        const int64_t target = (x * total + 7) / 8;
        if (pp < target && target <= pu) s_cut[x] = (int)u;
      }
    }
  }
  __syncthreads();
  if (tid <= 8) a.hdr[8 + tid] = s_cut[tid];
  // Within each queue, units go heaviest first: one counting sort over
  // (queue, 1023 - min(cost, 1023)) keys in LDS.  Queues are contiguous unit
  // ranges, so the sorted positions of queue x start at its first unit.
  for (int i = tid; i < 8 * 1024; i += 1024) s_bin[i] = 0;
  __syncthreads();
  const int32_t* tcum = a.tcum;
  auto key_of = [&](int u) {
    int x = 0;
#pragma unroll
    for (int k = 1; k < 8; ++k) x += u >= s_cut[k];
    const int t = u % n_tiles;
    return x * 1024 + 1023 - min(tcum[t + 1] - tcum[t], 1023);
  };
  for (int u = tid; u < (int)units; u += 1024) atomicAdd(&s_bin[key_of(u)], 1);
  __syncthreads();
  {
    int loc[8], sum = 0;  // thread t owns bins [8t, 8t + 8)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      loc[k] = sum;
      sum += s_bin[8 * tid + k];
    }
    int tot;
    const int base = block_exclusive_scan_1024(sum, tot, smem);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) s_bin[8 * tid + k] = base + loc[k];
  }
  __syncthreads();
  for (int u = tid; u < (int)units; u += 1024) a.order[atomicAdd(&s_bin[key_of(u)], 1)] = u;
  if (tid < 9) a.ctr[tid * kCtrStride] = 0;  // queues of the first run
}

// The whole plan in one launch: workgroup 0 lists and orders the MFMA tiles,
// workgroup 1 builds the split-KV plan of the short-query requests, the
// others write the token map (1024 tokens each).  None reads another's output.
__global__ __launch_bounds__(1024) void prefill_plan_kernel(PfPlanArgs a, PlanParams d, TokenMapArgs m) {
  if (blockIdx.x == 0) {
    prefill_plan_body(a);
  } else if (blockIdx.x == 1) {
    decode_plan_body(d);
  } else {
    token_map_body(m, ((int)blockIdx.x - 2) * 1024 + (int)threadIdx.x);
  }
}


template <typename MT, bool FP8>
static int launch_prefill(const PrefillParams& pp, int head_dim, int grid, hipStream_t stream) {
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 64>), dim3(grid), dim3(64 * pf_waves(64)), 0, stream, pp); break;
    case 128: return prefill_d128_launch(pp, MT::kDtype == MI_F16, FP8, grid, stream);
    case 256: hipLaunchKernelGGL((prefill_rs_kernel<MT, FP8, 256>), dim3(grid), dim3(512), 0, stream, pp); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

static bool ok_head_dim(int d) { return d == 64 || d == 128 || d == 256; }

}  // namespace mi

extern "C" int64_t mi_prefill_workspace_bytes(int32_t batch, int32_t max_qo_tokens, int32_t num_qo_heads,
                                              int32_t num_kv_heads, int32_t head_dim) {
  using namespace mi;
  if (batch < 0 || max_qo_tokens < 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return MI_ERR_INVALID;
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, num_qo_heads / num_kv_heads, num_kv_heads, head_dim);
  return L.split + split_layout(batch, num_kv_heads, head_dim, -1).total;
}

extern "C" int32_t mi_prefill_short_rows(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim) {
  using namespace mi;
  if (batch < 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads) return MI_ERR_INVALID;
  const int32_t G = num_qo_heads / num_kv_heads;
  return pair_short_rows(pair_heads(nullptr, batch, num_kv_heads, G, head_dim, true));
}

extern "C" int mi_prefill_plan(const int32_t* qo_indptr, const int32_t* kv_indptr,
                               const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                               int32_t max_qo_tokens, int32_t page_size, int32_t num_qo_heads,
                               int32_t num_kv_heads, int32_t head_dim, int64_t* token_to_page,
                               int64_t* token_to_cache, int32_t token_map_len, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  using namespace mi;
  if (batch < 0 || max_qo_tokens < 0 || token_map_len < 0 || !workspace) return MI_ERR_INVALID;
  if (!qo_indptr || !kv_indptr || !last_page_len || (batch > 0 && !kv_indices)) return MI_ERR_INVALID;
  if (token_map_len > 0 && (!token_to_page || !token_to_cache)) return MI_ERR_INVALID;
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads) return MI_ERR_INVALID;
  if (page_size <= 0) return MI_ERR_INVALID;
  if (page_size % 16 || !ok_head_dim(head_dim)) return MI_ERR_UNSUPPORTED;
  const int G = num_qo_heads / num_kv_heads;
  if (G > kShortRows) return MI_ERR_UNSUPPORTED;
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, G, num_kv_heads, head_dim);
  if (workspace_bytes < L.split) return MI_ERR_WORKSPACE;
  uint8_t* ws = (uint8_t*)workspace;
  PlanParams d{};
  const int st = decode_plan_params(qo_indptr, kv_indptr, kv_indices, last_page_len, batch, page_size, num_qo_heads,
                                    num_kv_heads, head_dim, nullptr, workspace, workspace_bytes, L.split, &d, true);
  if (st != MI_OK) return st;
  PfPlanArgs a;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.last_page_len = last_page_len;
  a.batch = batch;
  a.page_size = page_size;
  a.group = G;
  a.nkv = num_kv_heads;
  a.tile_rows = pf_rows(head_dim);
  a.max_tiles = L.max_tiles;
  a.causal = 1;  // cost model: causal
  a.short_rows = d.short_rows;  // the decode plan's threshold: every request goes to exactly one of the two
  a.hdr = (int32_t*)(ws + L.hdr);
  a.tiles = (int2*)(ws + L.tiles);
  a.tcum = (int32_t*)(ws + L.tcum);
  a.order = (int32_t*)(ws + L.order);
  a.ctr = (int32_t*)(ws + L.ctr);
  TokenMapArgs m;
  m.qo_indptr = qo_indptr;
  m.kv_indptr = kv_indptr;
  m.kv_indices = kv_indices;
  m.last_page_len = last_page_len;
  m.batch = batch;
  m.page_size = page_size;
  m.t2p = token_to_page;
  m.t2c = token_to_cache;
  m.map_len = token_map_len;
  const int grid = 2 + (token_map_len + 1023) / 1024;
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(grid), dim3(1024), 0, (hipStream_t)stream, a, d, m);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

namespace mi {

constexpr int kPhaseShort = 1;  // short-query requests: split-KV decode kernel + merge
constexpr int kPhaseTiles = 2;  // long-query requests: MFMA prefill tiles

static int prefill_run_impl(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                            const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                            const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                            int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, float sm_scale,
                            void* workspace, int64_t workspace_bytes, void* out, int64_t out_stride_token,
                            int64_t out_stride_head, int phases, void* stream) {
  if (!kv || batch < 0 || max_qo_tokens < 0 || !workspace) return MI_ERR_INVALID;
  if (batch == 0) return MI_OK;
  if (!q || !out || !kv->data || !qo_indptr || !kv_indptr || !kv_indices || !last_page_len) return MI_ERR_INVALID;
  const int nkv = kv->num_kv_heads, D = kv->head_dim;
  if (nkv <= 0 || num_qo_heads <= 0 || num_qo_heads % nkv) return MI_ERR_INVALID;
  const int G = num_qo_heads / nkv;
  if (G > kShortRows || kv->page_size % 16 || !ok_head_dim(D)) return MI_ERR_UNSUPPORTED;
  const bool fp8 = kv->dtype == MI_FP8_E4M3;
  if (q_dtype != MI_BF16 && q_dtype != MI_F16 && q_dtype != MI_F32) return MI_ERR_UNSUPPORTED;
  if (!fp8 && kv->dtype != q_dtype) return MI_ERR_UNSUPPORTED;
  if (fp8 && q_dtype == MI_F32) return MI_ERR_UNSUPPORTED;
  if (fp8 && (!kv->k_scale || !kv->v_scale)) return MI_ERR_INVALID;
  const int qesz = q_dtype == MI_F32 ? 4 : 2;
  if (!rows_aligned16(q, q_stride_token, q_stride_head, qesz) ||
      !rows_aligned16(out, out_stride_token, out_stride_head, qesz) || !kv_aligned16(kv))
    return MI_ERR_INVALID;
  // the tile loader keeps a chunk's offset within a page (K/V half, token
  // row, column) in 32 bits
  const int64_t kvesz = fp8 ? 1 : kv->dtype == MI_F32 ? 4 : 2;
  if (kv->kv_stride < 0 || kv->token_stride < 0 ||
      (kv->kv_stride + (int64_t)kv->page_size * kv->token_stride) * kvesz >= (1LL << 31))
    return MI_ERR_UNSUPPORTED;
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, G, nkv, D);
  if (workspace_bytes < L.split) return MI_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  int st = MI_OK;
  if (phases & kPhaseShort) {
    st = decode_run_impl(q, q_dtype, q_stride_token, q_stride_head, kv, qo_indptr, kv_indptr, kv_indices,
                         last_page_len, batch, num_qo_heads, causal, sm_scale, workspace, workspace_bytes,
                         L.split, out, out_stride_token, out_stride_head, kPhaseAttend | kPhaseMerge, s, true);
    if (st != MI_OK) return st;
  }
  if (!(phases & kPhaseTiles)) return MI_OK;
  const uint8_t* ws = (const uint8_t*)workspace;
  if (q_dtype == MI_F32) {  // fp32 KV: one workgroup per (tile, kv-head, 16-row block) of the plan's tiles
    DecodeParams dp{};
    dp.q = q;
    dp.q_stride_tok = q_stride_token;
    dp.q_stride_head = q_stride_head;
    dp.kv = kv->data;
    dp.page_stride = kv->page_stride;
    dp.kv_stride = kv->kv_stride;
    dp.token_stride = kv->token_stride;
    dp.head_stride = kv->head_stride;
    dp.qo_indptr = qo_indptr;
    dp.kv_indptr = kv_indptr;
    dp.kv_indices = kv_indices;
    dp.last_page_len = last_page_len;
    dp.out = out;
    dp.out_stride_tok = out_stride_token;
    dp.out_stride_head = out_stride_head;
    dp.num_kv_heads = nkv;
    dp.group = G;
    dp.page_size = kv->page_size;
    dp.causal = causal ? 1 : 0;
    dp.scale_log2 = sm_scale * 1.4426950408889634f;
    st = f32_prefill_launch(dp, (const int32_t*)(ws + L.hdr), (const int2*)(ws + L.tiles), L.max_tiles,
                            pf_rows(D), D, s);
    if (st != MI_OK) return st;
    MI_CHECK_LAUNCH();
    return MI_OK;
  }
  // long-query requests: MFMA prefill tiles
  PrefillParams pp{};
  pp.q = q;
  pp.q_stride_tok = q_stride_token;
  pp.q_stride_head = q_stride_head;
  pp.kv = kv->data;
  pp.page_stride = kv->page_stride;
  pp.kv_stride = kv->kv_stride;
  pp.token_stride = kv->token_stride;
  pp.head_stride = kv->head_stride;
  pp.k_scale = kv->k_scale;
  pp.v_scale = kv->v_scale;
  pp.qo_indptr = qo_indptr;
  pp.kv_indptr = kv_indptr;
  pp.kv_indices = kv_indices;
  pp.last_page_len = last_page_len;
  pp.hdr = (const int32_t*)(ws + L.hdr);
  pp.tiles = (const int2*)(ws + L.tiles);
  pp.order = (const int32_t*)(ws + L.order);
  pp.ctr = (int32_t*)((uint8_t*)workspace + L.ctr);
  pp.out = out;
  pp.out_stride_tok = out_stride_token;
  pp.out_stride_head = out_stride_head;
  pp.num_kv_heads = nkv;
  pp.group = G;
  pp.page_size = kv->page_size;
  pp.causal = causal ? 1 : 0;
  pp.scale_log2 = sm_scale * 1.4426950408889634f;
  // persistent grid: one workgroup per CU (each holds two wavefronts per SIMD),
  // never more than there are units
  int dev = 0, ncu = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return MI_ERR_LAUNCH;
  const int64_t units = (int64_t)L.max_tiles * nkv;
  const int grid = (int)(((units < ncu ? units : (int64_t)ncu) + 7) / 8 * 8);
  if (q_dtype == MI_BF16)
    st = fp8 ? launch_prefill<BF16, true>(pp, D, grid, s) : launch_prefill<BF16, false>(pp, D, grid, s);
  else
    st = fp8 ? launch_prefill<F16, true>(pp, D, grid, s) : launch_prefill<F16, false>(pp, D, grid, s);
  if (st != MI_OK) return st;
  MI_CHECK_LAUNCH();
  return MI_OK;
}

}  // namespace mi

#define MI_PREFILL_ARGS                                                                                          \
  const void *q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head, const mi_paged_kv *kv,          \
      const int32_t *qo_indptr, const int32_t *kv_indptr, const int32_t *kv_indices,                             \
      const int32_t *last_page_len, int32_t batch, int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, \
      float sm_scale, void *workspace, int64_t workspace_bytes, void *out, int64_t out_stride_token,             \
      int64_t out_stride_head, void *stream
#define MI_PREFILL_FWD(phases)                                                                                    \
  mi::prefill_run_impl(q, q_dtype, q_stride_token, q_stride_head, kv, qo_indptr, kv_indptr, kv_indices,          \
                       last_page_len, batch, max_qo_tokens, num_qo_heads, causal, sm_scale, workspace,           \
                       workspace_bytes, out, out_stride_token, out_stride_head, phases, stream)

extern "C" int mi_prefill_run(MI_PREFILL_ARGS) { return MI_PREFILL_FWD(mi::kPhaseShort | mi::kPhaseTiles); }
extern "C" int mi_prefill_short(MI_PREFILL_ARGS) { return MI_PREFILL_FWD(mi::kPhaseShort); }
extern "C" int mi_prefill_tiles(MI_PREFILL_ARGS) { return MI_PREFILL_FWD(mi::kPhaseTiles); }
