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
// 256 (query token, q-head) rows (128 for head_dim 256) of one request and
// kv-head -- GQA rows packed token-major, so K/V are read once per group of
// q-heads -- and each of the 8 wavefronts owns 2 groups of 16 rows.  Keys go
// in 32-key steps through a three-stage LDS ring filled from registers
// loaded three steps ahead (page ids staged in LDS, so no load waits on an
// index load); a tile's V^T fragments are read in the step that computes its
// scores and consumed by the next step's P.V MFMAs:
//   S^T[16 keys x 16 rows] = K . Q^T    (v_mfma_f32_16x16x32, K from LDS)
//   online softmax in fp32 (exp2 domain), causal mask aligned to the end of the KV
//   O^T[16 dims x 16 rows] += V^T . P^T (v_mfma_f32_16x16x32, V^T from the
//                                        transposing LDS read ds_read_b64_tr_b16)
// The two wavefronts of each SIMD run their softmax on opposite sides of
// their MFMA work (ping-pong), so vector and matrix work overlap.
// fp8 K/V are converted to the MFMA type when a tile is stored to LDS; the
// per-head scales multiply the scores and the output.
#include "mi_common.h"
#include "mi_internal.h"
#include "mi_plan.h"

namespace mi {

// Wavefronts per prefill workgroup (32 rows each): 8 (two per SIMD) while
// the per-wave state fits 256 registers, 4 for head_dim 256.
// Eight wavefronts (two per SIMD, in ping-pong) with two 16-row groups each;
// head_dim 256 keeps its accumulators within a two-wavefront register share
// with one 16-row group per wavefront.
constexpr int pf_waves(int) { return 8; }
constexpr int pf_rg(int head_dim) { return head_dim > 128 ? 1 : 2; }  // 16-row groups per wavefront
constexpr int pf_rows(int head_dim) { return 16 * pf_rg(head_dim) * pf_waves(head_dim); }  // (token, q-head) rows per workgroup
constexpr int kPfKeys = 32;                // keys per K/V tile
constexpr int kPfPageCap = 2048;           // page ids staged in LDS at a time
constexpr int kShortRows = 16;  // qo_len * group <= 16 -> decode kernel

// Workspace: header | per-XCD queue counters + finished-workgroup counter |
// tile list | tile cost prefix | unit order | decode split plan.
// Header words: [0] tiles, [1] units (tiles x kv-heads), [8 + x] first unit
// of XCD x's queue (x = 0..8, [16] = units).
struct PrefillLayout {
  int64_t hdr, ctr, tiles, tcum, order, split;
  int32_t max_tiles;
};
constexpr int kCtrStride = 32;  // one 128-byte line per XCD counter

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
      n = rows > kShortRows ? (rows + tile_rows - 1) / tile_rows : 0;
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

// ------------------------------------------------------------ attention
struct PrefillParams {
  const void* q;
  int64_t q_stride_tok, q_stride_head;
  const void* kv;
  int64_t page_stride, kv_stride, token_stride, head_stride;
  const float* k_scale;
  const float* v_scale;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* last_page_len;
  const int32_t* hdr;
  const int2* tiles;
  const int32_t* order;
  int32_t* ctr;
  void* out;
  int64_t out_stride_tok, out_stride_head;
  int32_t num_kv_heads, group, page_size, causal;
  float scale_log2;
};

template <typename MT, bool FP8, int D>
struct PrefillCfg {
  static constexpr int THREADS = 64 * pf_waves(D);
  static constexpr int ROWS = pf_rows(D);
  static constexpr int KEYS = kPfKeys;                     // keys per K/V tile
  // LDS row strides (bytes, MFMA-type elements).  K rows step 8 banks: the
  // 16-byte fragment reads of 16 rows at one column then hit distinct banks
  // (a 4-bank step left 28% of the LDS cycles in bank conflicts, 8 none).
  // V rows step 8 banks so the 4 rows x 32 bytes of one transposing read do.
  static constexpr int RSK = D * 2 + 32;
  static constexpr int RSV = D * 2 + 32;
  static constexpr int ESZ = FP8 ? 1 : 2;                  // cache element size
  static constexpr int CPR = D * ESZ / 16;                 // 16-byte chunks per cached row
  static constexpr int HALF = KEYS * CPR;                  // chunks of the K (or V) half of a tile
  static constexpr int NL = (2 * HALF + THREADS - 1) / THREADS;  // loader chunks per thread
  static constexpr int STAGE = KEYS * (RSK + RSV);         // one LDS stage: K rows then V rows
  static_assert(HALF % 64 == 0, "a wavefront's loader chunks must stay in one half");
  static_assert((2 * HALF) % THREADS == 0 || 2 * HALF < THREADS, "loader mapping");
};

template <typename MT, bool FP8, int D>
__global__ __launch_bounds__(64 * pf_waves(D)) void prefill_kernel(PrefillParams p) {
  using C = PrefillCfg<MT, FP8, D>;
  constexpr int KS = D / 32, VW = D / 16, KEYS = C::KEYS, RSK = C::RSK, RSV = C::RSV, ESZ = C::ESZ, CPR = C::CPR;
  constexpr int THREADS = C::THREADS, NL = C::NL, HALF = C::HALF, STAGE = C::STAGE;
  constexpr int RG = pf_rg(D), WROWS = 16 * RG;  // 16-row groups and rows per wavefront
  constexpr int LCH = FP8 ? 32 : 16;  // LDS bytes per loaded chunk
  constexpr float kNegInf = -__builtin_inff();
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * STAGE];
  __shared__ int32_t lds_pages[kPfPageCap];

  __shared__ int s_unit;
  const int nkv = p.num_kv_heads;
  const int n_tiles = p.hdr[0];
  const int xcd = (int)blockIdx.x & 7;  // workgroups are dispatched to the 8 XCDs round-robin

  // ---- persistent: take units from this XCD's queue, then steal from the others
  for (;;) {
  if (threadIdx.x == 0) {
    int u = -1;
    for (int k = 0; k < 8 && u < 0; ++k) {
      const int y = (xcd + k) & 7;
      const int first = p.hdr[8 + y], len = p.hdr[9 + y] - first;
      if (len <= 0 || __hip_atomic_load(p.ctr + y * kCtrStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= len)
        continue;
      const int i = atomicAdd(p.ctr + y * kCtrStride, 1);
      if (i < len) u = p.order[first + i];
    }
    s_unit = u;
  }
  __syncthreads();
  const int unit = s_unit;
  __syncthreads();
  if (unit < 0) break;
  const int h = unit / n_tiles;
  const int tile = unit - h * n_tiles;
  const int2 te = p.tiles[tile];
  const int b = te.x, row0 = te.y;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int ps = p.page_size, G = p.group;
  const int qo_start = p.qo_indptr[b];
  const int qo_len = p.qo_indptr[b + 1] - qo_start;
  const int page_base = p.kv_indptr[b];
  const int np = p.kv_indptr[b + 1] - page_base;
  const int kv_len = (np - 1) * ps + p.last_page_len[b];
  const int rows_total = qo_len * G;

  // ---- this lane's query rows (one per 16-row group)
  uint4 qf[RG][KS];
  int lim[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const int n = row0 + WROWS * wave + 16 * rg + col;
    const int tok = n / G, g = n - tok * G;
    const bool valid = n < rows_total;
    const int l = p.causal ? (kv_len - qo_len + tok) : (kv_len - 1);
    lim[rg] = min(l, kv_len - 1);
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(qo_start + tok) * p.q_stride_tok +
                           (int64_t)(h * G + g) * p.q_stride_head;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[rg][s] = valid ? *(const uint4*)(qrow + 32 * s + 8 * grp) : make_uint4(0, 0, 0, 0);
  }
  // ---- keys this workgroup needs, and where per-row masking starts
  const int last_row = min(row0 + C::ROWS, rows_total) - 1;
  const int max_tok = last_row / G, min_tok = row0 / G;
  const int kv_end = p.causal ? min(kv_len, kv_len - qo_len + max_tok + 1) : kv_len;
  const int mask_from = p.causal ? (kv_len - qo_len + min_tok + 1) : kv_len;
  const int n_kt = kv_end > 0 ? (kv_end + KEYS - 1) / KEYS : 0;

  float kscale = 1.f, vscale = 1.f;
  if constexpr (FP8) {
    kscale = p.k_scale[h];
    vscale = p.v_scale[h];
  }
  const float sl2 = p.scale_log2 * kscale;

  // ---- loader: chunk c = tid + i*THREADS -> (half, row, 16-byte column).
  // A wavefront's 64 chunks of one load cover 64/CPR <= 16 consecutive rows
  // of one half starting at a multiple of 64/CPR, so they lie in one
  // 16-row group of keys and hence in one page (page_size is a multiple of
  // 16, tiles start at multiples of 32): page and slot base are scalars.
  const uint8_t* kvb = (const uint8_t*)p.kv + (int64_t)h * p.head_stride * ESZ;
  const int64_t tok_bytes = p.token_stride * ESZ;
  uint32_t l_off[NL];   // per-thread byte offset within (page, first slot of its group)
  int l_grp[NL];        // first key row of the 16-row group (wave-uniform)
  int l_row[NL];        // key row within the tile
  bool l_v[NL];         // V half
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int c = tid + i * THREADS;
    const int half = c / HALF, rem = c - half * HALF;
    const int row = rem / CPR, ch = rem - row * CPR;
    l_row[i] = row;
    l_grp[i] = uniform(row) & ~15;
    l_v[i] = half == 1;
    l_off[i] = (uint32_t)((int64_t)half * p.kv_stride * ESZ + (int64_t)(row - (row & ~15)) * tok_bytes + 16 * ch);
  }
  const int key_cap = np * ps - 16;  // last 16-row group inside the request's pages
  int c0 = 0;  // first page of the page ids staged in LDS
  // NB register buffers (even): tile t+NB is loaded while tile t is computed
  // Three register buffers: tile i is loaded three steps before it is stored
  constexpr int NB = 3;
  uint4 rr[NB][NL];
  // A tile's loads in two parts: the page ids (LDS reads) and the global
  // loads, so a step can read its page ids early and issue the loads later.
  auto tile_pages = [&](int t, int (&pg)[NL]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      // groups past the request's last page re-read its last group (masked, V zeroed)
      const int gkey = uniform(min(t * KEYS + l_grp[i], key_cap));
      pg[i] = lds_pages[gkey / ps - c0];
    }
  };
  auto load_tile_at = [&](int t, const int (&pg)[NL], uint4 (&r)[NL]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (2 * HALF % THREADS == 0 || tid + i * THREADS < 2 * HALF) {
        const int gkey = uniform(min(t * KEYS + l_grp[i], key_cap));
        const int page = uniform(pg[i]);
        const uint8_t* base = kvb + (int64_t)page * p.page_stride * ESZ + (int64_t)(gkey % ps) * tok_bytes;
        r[i] = *(const uint4*)(base + l_off[i]);
      }
    }
  };
  auto load_tile = [&](int t, uint4 (&r)[NL]) {
    int pg[NL];
    tile_pages(t, pg);
    load_tile_at(t, pg, r);
  };
  auto store_tile = [&](int t, const uint4 (&r)[NL], int stage) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * THREADS;
      if (2 * HALF % THREADS == 0 || c < 2 * HALF) {
        const int half = c / HALF, rem = c - half * HALF;
        const int row = rem / CPR, ch = rem - row * CPR;
        uint4 v = r[i];
        // V rows past the KV end may hold anything (unwritten slots of the last page)
        if (l_v[i] && t * KEYS + l_row[i] >= kv_len) v = make_uint4(0, 0, 0, 0);
        uint8_t* dst = lds + stage * STAGE + (half ? KEYS * RSK + row * RSV : row * RSK) + LCH * ch;
        if constexpr (FP8) {  // 16 fp8 -> 16 MFMA-type elements (32 bytes)
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
          uint32_t o[8];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            o[2 * k] = fp8x2_to_mt<MT>(w[k], false);
            o[2 * k + 1] = fp8x2_to_mt<MT>(w[k], true);
          }
          *(uint4*)dst = make_uint4(o[0], o[1], o[2], o[3]);
          *(uint4*)(dst + 16) = make_uint4(o[4], o[5], o[6], o[7]);
        } else {
          *(uint4*)dst = v;
        }
      }
    }
  };

  f32x4 acc[RG][VW];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int jj = 0; jj < VW; ++jj) acc[rg][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Running max in raw-score units.  It is raised only when a tile's max
  // exceeds it by more than kLazy (exp2 units): probabilities then stay
  // <= 2^kLazy, harmless in fp32 sums and bf16/fp16 P, and the O rescale
  // is skipped on almost every tile.
  constexpr float kLazy = 8.f;
  const float lazy_raw = kLazy / sl2;
  float m_run[RG], l_run[RG], thr[RG];  // thr = m_run + lazy_raw
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    m_run[rg] = kNegInf;
    l_run[rg] = 0.f;
    thr[rg] = kNegInf;
  }

  // first tile that reaches past some row's limit: (t+1)*KEYS > mask_from
  const int t_mask = mask_from > 0 ? mask_from / KEYS : 0;

  // One 32-key tile: S^T = K.Q^T as two 16-key sub-tiles (16x16x32 MFMAs,
  // K fragments from LDS shared by both row groups), online softmax, then
  // O^T += V^T.P^T as one 16x16x32 MFMA per 16 output dims.  The MFMA k
  // index i of lane group grp stands for key 4*grp+i (i < 4) or 16+4*grp+i-4
  // (i >= 4): exactly the keys whose scores that lane holds, so P^T needs no
  // shuffle.
  auto qk = [&](int stage, f32x4 (&s)[RG][2]) {
    const uint8_t* sk = lds + stage * STAGE;
    uint4 a[2][KS];
#pragma unroll
    for (int js = 0; js < 2; ++js)
#pragma unroll
      for (int st = 0; st < KS; ++st) a[js][st] = *(const uint4*)(sk + (16 * js + col) * RSK + (8 * grp + 32 * st) * 2);
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int js = 0; js < 2; ++js) s[rg][js] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int js = 0; js < 2; ++js)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) s[rg][js] = MT::mma_16x16x32(a[js][st], qf[rg][st], s[rg][js]);
    // K fragment reads of slice st+1 ahead of the MFMAs of slice st (fewer
    // live fragment registers; c4 592 -> 586 us against all reads first).
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int st = 1; st < KS; ++st) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * RG, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * RG, 0);
  };
  // Softmax in two parts: sm_max masks (tail tiles only), takes the row max
  // and raises the running max when needed (a rare branch); sm_exp forms
  // the probabilities and their row sums.
  auto sm_max = [&](int t, f32x4 (&s)[RG][2]) {
    const int kb = t * KEYS;
    if (t >= t_mask) {  // wave-uniform: only the tiles that reach past some row's limit
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int js = 0; js < 2; ++js)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kb + 16 * js + 4 * grp + r > lim[rg]) s[rg][js][r] = kNegInf;
    }
    // A row's max exceeds the threshold iff one of its four lanes' maxima
    // does, so the cross-lane row max is only needed on the rare branch.
    float ml[RG];
    bool any_need = false;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      float m = kNegInf;
#pragma unroll
      for (int js = 0; js < 2; ++js)
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, s[rg][js][r]);
      ml[rg] = m;
      any_need |= m > thr[rg];
    }
    if (__builtin_amdgcn_ballot_w64(any_need)) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const float mt = rows4_max(ml[rg]);
        const bool grow = mt > thr[rg];
        const float alpha = grow ? fast_exp2((m_run[rg] - mt) * sl2) : 1.f;
        if (grow) {
          m_run[rg] = mt;
          thr[rg] = mt + lazy_raw;
        }
        l_run[rg] *= alpha;
#pragma unroll
        for (int jj = 0; jj < VW; ++jj) acc[rg][jj] *= alpha;
      }
    }
  };
  auto sm_exp = [&](const f32x4 (&s)[RG][2], uint4 (&pb)[RG]) {
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      const float moff = m_run[rg] == kNegInf ? 0.f : -m_run[rg] * sl2;
      float pr[2][4];
#pragma unroll
      for (int js = 0; js < 2; ++js)
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[js][r] = fast_exp2(fmaf(s[rg][js][r], sl2, moff));
      pb[rg] = make_uint4(MT::pack2(pr[0][0], pr[0][1]), MT::pack2(pr[0][2], pr[0][3]),
                          MT::pack2(pr[1][0], pr[1][1]), MT::pack2(pr[1][2], pr[1][3]));
      // row sums of the rounded probabilities the PV product uses
      l_run[rg] = MT::sum2(pb[rg].w, MT::sum2(pb[rg].z, MT::sum2(pb[rg].y, MT::sum2(pb[rg].x, l_run[rg]))));
    }
  };
  // V^T fragments with the transposing LDS read: in each 16-lane group,
  // lane j addresses row 4*grp + j/4 (+16 for MFMA k-slots 4..7) at dims
  // 16*jj + 4*(j%4) .. +3, and lane l receives the group's 4 keys at dim
  // 16*jj + l%16 -- the A operand of output tile jj (A row a = dim 16*jj + a).
  // The fragments of tile T are read in the step that computes its scores
  // and kept in registers across the barrier: the P.V MFMAs of the next
  // step then start without waiting on LDS, while that step's K reads run.
  // head_dim 256 (64 registers of fragments) reads them just before use.
  constexpr bool VPRE = D <= 128;
  auto vfrag = [&](int stage, uint4 (&a)[VW]) {
    const uint8_t* vt0 = lds + stage * STAGE + KEYS * RSK + (4 * grp + ((lane & 15) >> 2)) * RSV + 8 * (lane & 3);
#pragma unroll
    for (int jj = 0; jj < VW; ++jj) {
      const v4i16 x0 = ds_read_tr16(vt0 + 32 * jj);
      const v4i16 x1 = ds_read_tr16(vt0 + 16 * RSV + 32 * jj);
      const uint2 a0 = bitcast<uint2>(x0), a1 = bitcast<uint2>(x1);
      a[jj] = make_uint4(a0.x, a0.y, a1.x, a1.y);
    }
  };
  auto pv = [&](const uint4 (&a)[VW], const uint4 (&pb)[RG]) {
#pragma unroll
    for (int jj = 0; jj < VW; ++jj)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) acc[rg][jj] = MT::mma_16x16x32(a[jj], pb[rg], acc[rg][jj]);
    if constexpr (!VPRE) {  // fragments read just before: the reads of tile jj+1 ahead of its MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int jj = 1; jj < VW; ++jj) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, RG, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RG, 0);
    }
  };
  // Ping-pong: the two wavefronts that share a SIMD (one of waves {0,2,5,7},
  // one of {1,3,4,6}, for either round-robin or paired wave placement) put
  // their softmax on opposite sides of their MFMA work, so one's vector
  // work runs under the other's matrix work.  Group A finishes tile T-1's
  // softmax at the start of step T, group B finishes tile T's at its end.
  const bool grp_a = ((wave ^ (wave >> 2)) & 1) == 0;

  // ---- page chunks (one for contexts up to kPfPageCap pages).  Loads past
  // the last tile repeat the last tile, so the steady loop has no
  // conditional loads and the compiler's vmcnt waits stay exact.
  for (c0 = 0; c0 * ps < kv_end; c0 += kPfPageCap) {
    const int npg = min(np - c0, kPfPageCap);
    __syncthreads();
    for (int i = tid; i < npg; i += THREADS) lds_pages[i] = p.kv_indices[page_base + c0 + i];
    __syncthreads();
    const int t0 = c0 * ps / KEYS;
    const int t1 = min(n_kt, (c0 + kPfPageCap) * ps / KEYS);
    const int tl = t1 - 1;
    // Three-stage LDS ring: in step T both groups read V of tile T-1 (P.V)
    // and K of tile T (scores), and tile T+1 is stored into the stage tile
    // T-2 used.  Register buffer j holds the tiles t0 + j (mod 3), loaded
    // three steps before they are stored.
    const int n = t1 - t0;
#pragma unroll
    for (int u = 0; u < NB; ++u) load_tile(min(t0 + u, tl), rr[u]);
    store_tile(t0, rr[0], 0);
    load_tile(min(t0 + 3, tl), rr[0]);
    __syncthreads();
    f32x4 sc[RG][2];
    uint4 pbk[RG];
    uint4 va[VW];
    // step 0: scores and V^T fragments of tile t0; group B also its softmax
    qk(0, sc);
    if constexpr (VPRE) vfrag(0, va);
    if (!grp_a) {
      sm_max(t0, sc);
      sm_exp(sc, pbk);
    }
    store_tile(min(t0 + 1, tl), rr[1], 1);
    load_tile(min(t0 + 4, tl), rr[1]);
    __syncthreads();
    // steps 1 .. n-1
    for (int i = 1; i < n; i += 3) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int ii = i + u;
        if (ii >= n) break;
        const int T = t0 + ii;
        // Tile T+1 goes into the stage tile T-2 used, which no wave reads in
        // this step; each group stores it (and issues the loads of tile T+4)
        // in its vector half, under the other group's MFMA work.
        int pg4[NL];
        tile_pages(min(T + 4, tl), pg4);
        // Each group's vector half runs at raised wave priority, so its softmax
        // issues ahead of the partner's MFMA stream on the shared SIMD
        // (c4 583 -> 580 us, head_dim 256 1794 -> 1747 us).
        if (grp_a) {
          __builtin_amdgcn_s_setprio(1);
          store_tile(min(T + 1, tl), rr[(u + 2) % 3], (u + 2) % 3);
          sm_max(T - 1, sc);
          sm_exp(sc, pbk);
          load_tile_at(min(T + 4, tl), pg4, rr[(u + 2) % 3]);
          __builtin_amdgcn_s_setprio(0);
        }
        // scores of tile T first (group B's softmax waits on them), then P.V of
        // tile T-1; V^T fragments of tile T replace those of T-1 after it
        qk((u + 1) % 3, sc);       // stage of tile T = ii % 3
        if constexpr (!VPRE) vfrag(u % 3, va);  // stage of tile T-1 = (ii-1) % 3 = u
        pv(va, pbk);               // tile T-1
        if constexpr (VPRE) vfrag((u + 1) % 3, va);
        if (!grp_a) {
          __builtin_amdgcn_s_setprio(1);
          store_tile(min(T + 1, tl), rr[(u + 2) % 3], (u + 2) % 3);
          load_tile_at(min(T + 4, tl), pg4, rr[(u + 2) % 3]);
          sm_max(T, sc);
          sm_exp(sc, pbk);
          __builtin_amdgcn_s_setprio(0);
        }
        __syncthreads();
      }
    }
    // last step: P.V of tile t1-1
    if (grp_a) {
      sm_max(t1 - 1, sc);
      sm_exp(sc, pbk);
    }
    if constexpr (!VPRE) vfrag((n - 1) % 3, va);
    pv(va, pbk);
  }

  // ---- epilogue: lane holds dims 16*jj + 4*grp + r of its row
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const float l_tot = rows4_sum(l_run[rg]);
    const float inv = l_tot > 0.f ? vscale / l_tot : 0.f;
    const int n = row0 + WROWS * wave + 16 * rg + col;
    if (n >= rows_total) continue;
    const int tok = n / G, g = n - tok * G;
    uint16_t* orow = (uint16_t*)p.out + (int64_t)(qo_start + tok) * p.out_stride_tok +
                     (int64_t)(h * G + g) * p.out_stride_head;
#pragma unroll
    for (int jj = 0; jj < VW; ++jj) {
      const f32x4 o = acc[rg][jj];
      *(uint2*)(orow + 16 * jj + 4 * grp) = make_uint2(MT::pack2(o[0] * inv, o[1] * inv), MT::pack2(o[2] * inv, o[3] * inv));
    }
  }
  }  // unit loop
  // The last workgroup to finish resets the queues for the next run with
  // this plan (every other workgroup has taken its last unit by then).
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(p.ctr + 8 * kCtrStride, 1) == (int)gridDim.x - 1) {
#pragma unroll
      for (int y = 0; y < 9; ++y) __hip_atomic_store(p.ctr + y * kCtrStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <typename MT, bool FP8>
static int launch_prefill(const PrefillParams& pp, int head_dim, int grid, hipStream_t stream) {
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 64>), dim3(grid), dim3(64 * pf_waves(64)), 0, stream, pp); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 128>), dim3(grid), dim3(64 * pf_waves(128)), 0, stream, pp); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 256>), dim3(grid), dim3(64 * pf_waves(256)), 0, stream, pp); break;
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
                                    num_kv_heads, head_dim, nullptr, workspace, workspace_bytes, L.split, &d);
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
                         L.split, out, out_stride_token, out_stride_head, kPhaseAttend | kPhaseMerge, s);
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
