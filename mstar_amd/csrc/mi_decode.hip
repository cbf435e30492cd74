// Split-KV paged GQA decode for MI355X (gfx950).
//
// Replaces FlashInfer's BatchDecodeWithPagedKVCacheWrapper plan/run as used by
// FlashInferDecodeWrapper (mstar/utils/flashinfer_utils.py:369-465), and the
// short-query part of the prefill wrapper (requests whose
// qo_len * group <= 16).
//
// Work decomposition
//   plan  : one 1024-thread workgroup splits every request's page list into
//           items of at most `item_pages` pages (chosen on the GPU from the
//           batch's total page count so the machine gets ~8K wavefronts) and
//           writes the item list into the caller's workspace.
//   decode: one workgroup per (item, kv-head); its 4 wavefronts take
//           contiguous quarters of the item's 16-token tiles.  A wavefront's
//           16 MFMA columns are the (query token, q-head-in-group) rows that
//           share the kv-head, so K/V are read from HBM once per GQA group.
//           Per tile:
//             S^T[16 tok x 16 rows] = K[16 x D] . Q^T      (v_mfma 16x16x32)
//             online softmax on S (fp32, exp2 domain)
//             O^T[D x 16 rows]     += V^T[D x 16 tok] . P^T (v_mfma 16x16x16)
//           K and V rows are read as whole head_dim rows (16 lanes x 128 bits
//           per row for D=128; every load instruction covers 256 contiguous
//           bytes of a row, see dim_of) with non-temporal loads, two tiles
//           ahead of the MFMA work.  The MFMA A operand wants one token per lane%16, which
//           a register-only layout can only feed with 64-byte row segments
//           (measured ~15% slower to stream from HBM), so K passes through a
//           small per-wave LDS buffer: ds_write of the rows, ds_read of the
//           fragments.  V is transposed in registers (v_perm_b32): output
//           row i of output tile m is the dim lane i loaded as its element m
//           (dim_of), which turns the transpose into a 4x(D/16) shuffle
//           inside each lane.
//           The 4 wavefronts' softmax states are merged in LDS; an item that
//           covers its whole request writes the final output, otherwise a
//           partial (o, lse).  Partial stores are HBM writes interleaved with
//           a read-saturated stream and cost far more than their bytes
//           (measured: ~33 MB of partials added ~14% to the kernel), which
//           is why an item spans 4 wavefronts' worth of pages.
//   merge : log-sum-exp merge of the item partials of split requests, in the
//           same register-order layout (whole-cache-line loads and stores).
#include "mi_common.h"
#include "mi_internal.h"
#include "mi_plan.h"

namespace mi {

constexpr int kMinChunkTokens = 1024;  // never split a request finer than this (4 waves x 256)
// ... except in small jobs, down to this, while the items fit one round of
// resident workgroups (decode_plan_body)
constexpr int kSmallChunkTokens = 256;

// Compute units of the current device (cached per device).
static int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}


// Target number of wavefronts for one plan: ~4K (item, kv-head, quarter)
// wave units fill 256 CUs x 2 resident workgroups about twice; with the
// longest-first work order the drain tail stays short while few requests
// need partials (measured on c3: 4096 -> 545 us, 8192 -> 558 us,
// 16384 -> 586 us; 2048 and 1024 units: 538-540 and 609 us).
constexpr int32_t kDecodeTargetUnits = 4096;
// head_dim 256: one resident workgroup per CU and twice the bytes per token,
// so fewer and longer items: c3's contexts at 16 q / 2 kv heads 536 -> 507 us
// (1536 units: 524 us); smaller batches, whose items kMinChunkTokens bounds
// (Pi0.5's 8 q / 1 kv), are unchanged.
constexpr int32_t kDecodeTargetUnitsWide = 1024;

SplitLayout split_layout(int32_t batch, int32_t nkv, int32_t head_dim, int64_t ws_avail, bool pair) {
  SplitLayout L;
  // a paired plan is a head_dim 256 plan over half the kv-heads
  const int32_t tnkv = pair ? nkv / 2 : nkv, thd = pair ? 2 * head_dim : head_dim;
  const int32_t units = thd > 128 ? kDecodeTargetUnitsWide : kDecodeTargetUnits;
  int32_t target = units / (4 * (tnkv > 0 ? tnkv : 1));  // 4 waves per item
  if (target < 16) target = 16;
  int64_t max_chunks = (int64_t)target + batch;
  if (ws_avail >= 0) {  // fewer, longer chunks when the caller's workspace is smaller
    const int64_t fixed = 256 + mi_align_up(4LL * (batch + 1), 256) + 3 * 256;
    const int64_t per_chunk = 16 + 4LL * nkv * kRows + 4LL * nkv * kRows * head_dim;
    const int64_t fit = (ws_avail - fixed) / per_chunk;
    if (fit < max_chunks) max_chunks = fit;
  }
  L.max_chunks = (int32_t)max_chunks;
  int64_t off = 0;
  L.hdr = off;
  off += 256;
  L.chunk_indptr = off;
  off = mi_align_up(off + 4LL * (batch + 1), 256);
  L.work = off;
  off = mi_align_up(off + 16LL * L.max_chunks, 256);
  L.lse = off;
  off = mi_align_up(off + 4LL * L.max_chunks * nkv * kRows, 256);
  L.opart = off;
  off = mi_align_up(off + 4LL * L.max_chunks * nkv * kRows * head_dim, 256);
  L.total = off;
  return L;
}

__global__ __launch_bounds__(1024) void decode_plan_kernel(PlanParams p) { decode_plan_body(p); }

// ---------------------------------------------------------------- decode

// Per-lane registers of one 16-token tile.
template <bool FP8, int D>
struct TileRegs;

template <int D>
struct TileRegs<false, D> {  // 16-bit KV: K and V as row slices (D/16 elements per row)
  uint32_t k[4][D / 32];
  uint32_t v[4][D / 32];
};

template <int D>
struct TileRegs<true, D> {  // fp8 KV: raw bytes (D/16 per row), converted right before use
  uint32_t k[4][D / 64 > 0 ? D / 64 : 1];
  uint32_t v[4][D / 64 > 0 ? D / 64 : 1];
};

template <int N>
MI_DEVICE void load_words(uint32_t (&dst)[N], const uint8_t* src) {
  if constexpr (N == 1) {
    dst[0] = nt_load4(src);
  } else if constexpr (N == 2) {
    const uint2 t = nt_load8(src);
    dst[0] = t.x;
    dst[1] = t.y;
  } else {  // 16-byte chunk k of the lane's elements sits 256*k bytes into the row (see dim_of)
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const uint4 t = nt_load16(src + 64 * i);
      dst[i] = t.x;
      dst[i + 1] = t.y;
      dst[i + 2] = t.z;
      dst[i + 3] = t.w;
    }
  }
}

// PAIR (D = 256): two adjacent head_dim 128 kv-heads read as one 256-element
// row; p.num_kv_heads counts the pairs, p.group is the real group size, query
// row col belongs to kv-head 2h + (col >= group) (see pair_heads).
template <typename MT, bool FP8, int D, bool PAIR = false>
__global__ __launch_bounds__(256) void decode_kernel(DecodeParams p) {
  static_assert(!PAIR || D == 256, "paired kv-heads form 256-element rows");
  constexpr int KS = D / 32;  // MFMA k-steps over head_dim for S
  constexpr int VW = D / 16;  // V elements per lane per row == output d-tiles
  constexpr int ESZ = FP8 ? 1 : 2;
  constexpr int KRS = D * 2 + 32;  // LDS row stride of the K transpose buffer (8-bank step: conflict-free fragment reads)
  constexpr int RUN = lane_run(D, ESZ);  // consecutive elements per lane (dim_of)
  constexpr int NS = VW / 4;       // float4 groups per lane per output row segment
  constexpr float kNegInf = -__builtin_inff();
  // LDS: during the tile loop, per-wave K staging (rows arrive as whole
  // head_dim rows and leave as MFMA A fragments); after it, the 4 waves'
  // softmax states for the in-workgroup merge.
  constexpr int kStageBytes = 4 * 16 * KRS;
  constexpr int kMergeBytes = 4 * (4 * NS * 64 * 16);
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes];
  __shared__ float lds_m[4][kRows], lds_l[4][kRows];

  const int lane = lane_id();
  const int wave = uniform((int)threadIdx.x >> 6);
  const int nkv = p.num_kv_heads;
  // workgroup = (item, kv-head); its 4 waves split the item's tiles
  // all kv-heads of an item on one XCD (blocks go to XCDs round-robin), 8 blocks apart
  const int gsz = 8 * nkv;
  const int gi = uniform((int)blockIdx.x / gsz);
  const int gr = (int)blockIdx.x - gi * gsz;
  const int h = uniform(gr >> 3);
  const int item = uniform(gi * 8 + (gr & 7));
  if (item >= p.hdr[kHdrChunks]) return;  // uniform across the workgroup
  const int4 wk = p.work[item];
  const int b = uniform(wk.x), kidx = uniform(wk.y), pg1 = uniform(wk.z), nitems_b = uniform(wk.w);
  const int pg0 = kidx * p.hdr[kHdrChunkPages];

  const int ps = p.page_size;
  const int page_base = p.kv_indptr[b];
  const int np = p.kv_indptr[b + 1] - page_base;
  const int kv_len = (np - 1) * ps + p.last_page_len[b];
  int qo_start = b, qo_len = 1;
  if (p.qo_indptr) {
    qo_start = p.qo_indptr[b];
    qo_len = p.qo_indptr[b + 1] - qo_start;
  }
  const int G = p.group;
  const int rows = min((PAIR ? 2 : 1) * qo_len * G, kRows);
  const int item_tok0 = pg0 * ps;
  const int item_tok1 = min(pg1 * ps, kv_len);
  const int item_tiles = item_tok1 > item_tok0 ? (item_tok1 - item_tok0 + 15) >> 4 : 0;
  // this wave's contiguous quarter of the item's tiles
  const int tq = item_tiles >> 2, trem = item_tiles & 3;
  const int my_t0 = wave * tq + min(wave, trem);
  const int ntiles = tq + (wave < trem ? 1 : 0);
  const int tok_begin = item_tok0 + 16 * my_t0;

  const int col = lane & 15;  // query row handled in MFMA column `col`
  const int grp = lane >> 4;  // 0..3
  const int half = PAIR && col >= qo_len * G ? 1 : 0;  // PAIR: which head of the pair
  const int rcol = col - half * qo_len * G;
  const int hq = PAIR ? 2 * h + half : h;  // the row's kv-head
  const int qtok = rcol / G;
  const int g = rcol - qtok * G;
  const bool row_valid = col < rows;
  // Keys this row may attend: [0, lim]  (causal: aligned to the end of the KV).
  int lim = p.causal ? (kv_len - qo_len + qtok) : (kv_len - 1);
  lim = min(lim, kv_len - 1);
  // Keys >= mask_from need a per-row check (uniform bound).
  const int mask_from = p.causal ? (kv_len - qo_len + 1) : kv_len;

  // ---- Q as the B operand of S^T = K Q^T: lane holds Q[row col][8*grp + 32*s ...].
  // PAIR: only the row's own 128 elements; both heads' score products use
  // them, and each column keeps the product with its own head's keys.
  constexpr int QS = PAIR ? KS / 2 : KS;
  uint4 qf[QS];
  {
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(qo_start + qtok) * p.q_stride_tok +
                           (int64_t)(hq * G + g) * p.q_stride_head;
#pragma unroll
    for (int s = 0; s < QS; ++s)
      qf[s] = row_valid ? *(const uint4*)(qrow + 32 * s + 8 * grp) : make_uint4(0, 0, 0, 0);
  }
  float kscale = 1.0f, vscale = 1.0f;
  if constexpr (FP8) {
    kscale = p.k_scale[hq];
    vscale = p.v_scale[hq];
  }
  const float sl2 = p.scale_log2 * kscale;

  const uint8_t* kv = (const uint8_t*)p.kv;
  const int64_t head_off = (int64_t)h * p.head_stride * ESZ;
  // per-lane byte offset inside a tile: rows 4*grp + r, elements [VW*col, VW*col + VW)
  const uint32_t voff0 = (uint32_t)((4 * grp) * p.token_stride + RUN * col) * ESZ;
  const uint32_t vrow = (uint32_t)(p.token_stride * ESZ);
  const int64_t kvhalf = p.kv_stride * ESZ;

  // page ids, slots and strides are non-negative: unsigned scalar arithmetic
  // (a signed division and 64-bit multiply per tile cost ~30 scalar ops)
  const uint64_t page_bytes = (uint64_t)p.page_stride * ESZ;
  auto tile_base = [&](int page, int r0) -> const uint8_t* {
    return kv + (uint64_t)(uint32_t)page * page_bytes + (uint32_t)r0 * vrow + head_off;
  };
  auto load_tile = [&](TileRegs<FP8, D>& t, const uint8_t* base) {
    const uint8_t* kb = base + voff0;
#pragma unroll
    for (int r = 0; r < 4; ++r) load_words(t.k[r], kb + r * vrow);
    const uint8_t* vb = kb + kvhalf;
#pragma unroll
    for (int r = 0; r < 4; ++r) load_words(t.v[r], vb + r * vrow);
  };
  uint8_t* kst = &lds[wave * 16 * KRS];

  f32x4 acc[VW];
#pragma unroll
  for (int j = 0; j < VW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  auto compute_tile = [&](TileRegs<FP8, D>& t, int ti) {
    const int tb = tok_begin + 16 * ti;
    // ---- K rows -> LDS (row 4*grp + r, elements [VW*col, +VW)) -> A fragments
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t w[VW / 2];
      if constexpr (FP8) {
#pragma unroll
        for (int i = 0; i < VW / 4; ++i) {
          w[2 * i] = fp8x2_to_mt<MT>(t.k[r][i], false);
          w[2 * i + 1] = fp8x2_to_mt<MT>(t.k[r][i], true);
        }
      } else {
#pragma unroll
        for (int i = 0; i < VW / 2; ++i) w[i] = t.k[r][i];
      }
      uint8_t* dst = kst + (4 * grp + r) * KRS;  // row in natural dim order
      if constexpr (VW == 4) {
        *(uint2*)(dst + 2 * dim_of(RUN, col, 0)) = make_uint2(w[0], w[1]);
      } else {
#pragma unroll
        for (int i = 0; i < VW / 2; i += 4)
          *(uint4*)(dst + 2 * dim_of(RUN, col, 2 * i)) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
      }
    }
    // ---- S^T = K . Q^T  (A fragment: row col, elements 8*grp + 32*st .. +8)
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (PAIR) {
      // One accumulator per head of the pair: s takes the keys' k-steps
      // [0, KS/2) (head 2h's elements), s1 the k-steps [KS/2, KS) (head
      // 2h+1's), both against the row's own 128 query elements.  A column
      // keeps the product with its own head's keys (a select, so the other
      // product's values, non-finite ones included, never reach it).
      f32x4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < KS / 2; ++st) {
        const uint4 a0 = *(const uint4*)(kst + col * KRS + (8 * grp + 32 * st) * 2);
        const uint4 a1 = *(const uint4*)(kst + col * KRS + (8 * grp + 32 * (st + KS / 2)) * 2);
        s = MT::mma_16x16x32(a0, qf[st], s);
        s1 = MT::mma_16x16x32(a1, qf[st], s1);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = half ? s1[r] : s[r];
    } else {
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const uint4 a = *(const uint4*)(kst + col * KRS + (8 * grp + 32 * st) * 2);
        s = MT::mma_16x16x32(a, qf[st], s);
      }
    }
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sv[r] = s[r] * sl2;
    const bool need_mask = tb + 16 > mask_from;
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = tb + 4 * grp + r;
        if (key > lim) sv[r] = kNegInf;
        if (key >= kv_len) {  // slots past the end hold stale data: keep NaN/Inf out of P.V
#pragma unroll
          for (int i = 0; i < (int)(sizeof(t.v[r]) / 4); ++i) t.v[r][i] = 0u;
        }
      }
    }
    // ---- online softmax (row = col; the 4 lane groups share a row)
    const float mt = rows4_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(sv[r] - m_use);
    l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    if (__builtin_amdgcn_ballot_w64(m_new > m_run)) {
#pragma unroll
      for (int j = 0; j < VW; ++j) acc[j] *= alpha;
    }
    m_run = m_new;
    const uint2 pb = make_uint2(MT::pack2(pr[0], pr[1]), MT::pack2(pr[2], pr[3]));
    // ---- O^T += V^T . P^T, V transposed in registers
    uint32_t vv[4][VW / 2];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (FP8) {
#pragma unroll
        for (int i = 0; i < VW / 4; ++i) {
          vv[r][2 * i] = fp8x2_to_mt<MT>(t.v[r][i], false);
          vv[r][2 * i + 1] = fp8x2_to_mt<MT>(t.v[r][i], true);
        }
      } else {
#pragma unroll
        for (int i = 0; i < VW / 2; ++i) vv[r][i] = t.v[r][i];
      }
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      uint2 a;
      if (j & 1) {
        a.x = pack_hi16(vv[0][j >> 1], vv[1][j >> 1]);
        a.y = pack_hi16(vv[2][j >> 1], vv[3][j >> 1]);
      } else {
        a.x = pack_lo16(vv[0][j >> 1], vv[1][j >> 1]);
        a.y = pack_lo16(vv[2][j >> 1], vv[3][j >> 1]);
      }
      acc[j] = MT::mma_16x16x16(a, pb, acc[j]);
    }
  };

  // ---- tile loop, in windows of 64 pages.  The window's page ids sit in one
  // VGPR (lane i: page i of the window) and v_readlane hands each tile's page
  // to the scalar unit, so no memory access sits between the loads of
  // consecutive tiles; inside a window the loads run two tiles ahead of the
  // MFMA work (three register buffers).
  for (int w0 = 0; w0 < ntiles;) {
    const int wtok = tok_begin + 16 * w0;  // first token of the window
    const int first = (int)((unsigned)wtok / (unsigned)ps);  // its page (request-relative)
    const int wt = min(ntiles - w0, ((first + 64) * ps - wtok) >> 4);
    const int pwin = first + lane < pg1 ? p.kv_indices[page_base + first + lane] : 0;
    auto tile_ptr = [&](int t) -> const uint8_t* {  // t: tile within the window
      const unsigned tok = (unsigned)(wtok + 16 * t);
      const unsigned pg = tok / (unsigned)ps;
      return tile_base(__builtin_amdgcn_readlane(pwin, (int)pg - first), (int)(tok - pg * (unsigned)ps));
    };
    TileRegs<FP8, D> A, B, C;
    load_tile(A, tile_ptr(0));
    if (wt > 1) load_tile(B, tile_ptr(1));
    int t = 0;
    // Steady state: every load in the body is in range, so the compiler's
    // vmcnt waits stay exact (two tiles in flight while one is computed).
    for (; t + 4 < wt; t += 3) {
      load_tile(C, tile_ptr(t + 2));
      compute_tile(A, w0 + t);
      load_tile(A, tile_ptr(t + 3));
      compute_tile(B, w0 + t + 1);
      load_tile(B, tile_ptr(t + 4));
      compute_tile(C, w0 + t + 2);
    }
    // Tail: at most four tiles left; A holds tile t, B tile t+1.
    if (t + 2 < wt) load_tile(C, tile_ptr(t + 2));
    if (t < wt) compute_tile(A, w0 + t);
    if (t + 3 < wt) load_tile(A, tile_ptr(t + 3));
    if (t + 1 < wt) compute_tile(B, w0 + t + 1);
    if (t + 2 < wt) compute_tile(C, w0 + t + 2);
    if (t + 3 < wt) compute_tile(A, w0 + t + 3);
    w0 += wt;
  }

  // ---- epilogue: merge the 4 waves' states (m, l, acc) in LDS.  The acc
  // register layout is the same in every wave (lane -> row col, elements
  // d = VW*(4*grp + r) + j), so the merge is lane-local; wave w finishes the
  // elements with r == w.
  __syncthreads();  // all waves are done with their K staging buffers
  {
    const float l_row = rows4_sum(l_run);
    if (grp == 0) {
      lds_m[wave][col] = m_run;
      lds_l[wave][col] = l_row;
    }
    float4* st = (float4*)lds + (size_t)wave * 4 * NS * 64 + lane;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < VW; j += 4)
        st[(r * NS + j / 4) * 64] = make_float4(acc[j][r], acc[j + 1][r], acc[j + 2][r], acc[j + 3][r]);
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, lds_m[w][col]);
  const float M_use = M == kNegInf ? 0.f : M;
  float sc[4], L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    sc[w] = fast_exp2(lds_m[w][col] - M_use);  // m = -inf -> 0
    L += sc[w] * lds_l[w][col];
  }
  float4 o[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) o[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4* src = (const float4*)lds + (size_t)w * 4 * NS * 64 + (size_t)wave * NS * 64 + lane;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float4 v = src[i * 64];
      o[i].x += sc[w] * v.x;
      o[i].y += sc[w] * v.y;
      o[i].z += sc[w] * v.z;
      o[i].w += sc[w] * v.w;
    }
  }
  const float inv = L > 0.f ? vscale / L : (L == 0.f ? 0.f : __builtin_nanf(""));  // NaN L: keep the row NaN
  if (!row_valid) return;
  if (nitems_b == 1) {
    // elements j of output row 4*grp + wave: dims dim_of(RUN, 4*grp + wave, j), row col
    uint16_t* dst = (uint16_t*)p.out + (int64_t)(qo_start + qtok) * p.out_stride_tok +
                    (int64_t)(hq * G + g) * p.out_stride_head;
    uint32_t w[VW / 2];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      w[2 * i] = MT::pack2(o[i].x * inv, o[i].y * inv);
      w[2 * i + 1] = MT::pack2(o[i].z * inv, o[i].w * inv);
    }
    if constexpr (VW == 4) {
      *(uint2*)(dst + dim_of(RUN, 4 * grp + wave, 0)) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int i = 0; i < VW / 2; i += 4) {
        const int d0 = dim_of(RUN, 4 * grp + wave, 2 * i);  // 8 consecutive elements
        if (PAIR && (d0 >= D / 2) != (half == 1)) continue;  // the other head's half
        *(uint4*)(dst + d0 - (PAIR ? (D / 2) * half : 0)) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
      }
    }
  } else {
    // Partial (o, lse) of this item, o in register order: store index
    // i = r*NS + j/4 of every lane is one contiguous 64 x 16-byte block.
    const int64_t unit_idx = (int64_t)(p.chunk_indptr[b] + kidx) * nkv + h;
    float* ob = p.o_part + unit_idx * kRows * D + 4 * lane;
#pragma unroll
    for (int i = 0; i < NS; ++i)
      *(float4*)(ob + 256 * (wave * NS + i)) = make_float4(o[i].x * inv, o[i].y * inv, o[i].z * inv, o[i].w * inv);
    // lse: -inf for an empty partial; NaN when the row met a NaN or +inf score,
    // so the merge propagates it as a single softmax over the keys would.
    if (wave == 0 && grp == 0)
      p.lse_part[unit_idx * kRows + col] = L > 0.f ? M + fast_log2(L) : (L == 0.f ? kNegInf : __builtin_nanf(""));
  }
}

// ----------------------------------------------------------------- merge
// One workgroup per (request, kv-head); its 4 wavefronts split the output
// elements as the decode kernel's did: lane l of wavefront w merges row l%16,
// elements d = VW*(4*(l/16) + w) + j, read from the register-order partial
// layout with 64-lane contiguous (cache-line) loads.
template <typename MT, int D, int RUN, bool PAIR = false>
__global__ __launch_bounds__(256) void merge_kernel(DecodeParams p, int32_t batch) {
  static_assert(!PAIR || D == 256, "paired kv-heads form 256-element rows");
  constexpr int VW = D / 16;
  constexpr int NS = VW / 4;  // float4 groups per lane per partial
  constexpr float kNegInf = -__builtin_inff();
  const int nkv = p.num_kv_heads;
  const int pair = (int)blockIdx.x;
  if (pair >= batch * nkv) return;
  const int b = pair / nkv;
  const int h = pair - b * nkv;
  const int c0 = p.chunk_indptr[b];
  const int nb = p.chunk_indptr[b + 1] - c0;
  if (nb == 1) return;  // written directly by the decode kernel
  int qo_start = b, qo_len = 1;
  if (p.qo_indptr) {
    qo_start = p.qo_indptr[b];
    qo_len = p.qo_indptr[b + 1] - qo_start;
  }
  const int G = p.group;
  const int rows = (PAIR ? 2 : 1) * qo_len * G;
  if (qo_len * G > p.short_rows) return;  // long-query request: written by the prefill kernel
  const int lane = lane_id();
  const int wave = (int)threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  if (col >= rows) return;
  const int half = PAIR && col >= qo_len * G ? 1 : 0;
  const int rcol = col - half * qo_len * G;
  const int hq = PAIR ? 2 * h + half : h;
  const int qtok = rcol / G, g = rcol - qtok * G;
  float4 acc[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  const int64_t u0 = (int64_t)c0 * nkv + h;  // unit of chunk c: u0 + c * nkv
  // One pass: each group of U partials is loaded with its lse values at
  // once (no separate max pass ahead of the loads), and the running sum is
  // rescaled when a partial raises the running max.
  float M = kNegInf, wsum = 0.f;
  constexpr int U = D > 128 ? 4 : 8;  // partials in flight per step
  for (int c = 0; c < nb; c += U) {
    float w[U];
    float4 o[U][NS];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = kNegInf;
      if (c + u < nb) {
        const int64_t unit = u0 + (int64_t)(c + u) * nkv;
        w[u] = p.lse_part[unit * kRows + col];
        const float* src = p.o_part + unit * kRows * D + 4 * lane + 256 * wave * NS;
#pragma unroll
        for (int i = 0; i < NS; ++i) o[u][i] = *(const float4*)(src + 256 * i);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (w[u] == kNegInf) continue;  // past the end, or an empty partial (a NaN lse makes the row NaN)
      if (w[u] > M) {
        const float sc = fast_exp2(M - w[u]);  // 0 while M is -inf
        wsum *= sc;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
          acc[i].x *= sc;
          acc[i].y *= sc;
          acc[i].z *= sc;
          acc[i].w *= sc;
        }
        M = w[u];
      }
      const float wgt = fast_exp2(w[u] - M);
      wsum += wgt;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        acc[i].x += wgt * o[u][i].x;
        acc[i].y += wgt * o[u][i].y;
        acc[i].z += wgt * o[u][i].z;
        acc[i].w += wgt * o[u][i].w;
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int64_t orow_off = (int64_t)(qo_start + qtok) * p.out_stride_tok + (int64_t)(hq * G + g) * p.out_stride_head;
  // this wave's elements of the row: group i holds d = dim_of(RUN, 4*grp + wave, 4*i) .. +3
  if constexpr (MT::kDtype == MI_F32) {
    float* orow = (float*)p.out + orow_off;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float4 a = acc[i];
      *(float4*)(orow + dim_of(RUN, 4 * grp + wave, 4 * i)) = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
    }
  } else {
    uint16_t* orow = (uint16_t*)p.out + orow_off;
    uint32_t w[VW / 2];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      w[2 * i] = MT::pack2(acc[i].x * inv, acc[i].y * inv);
      w[2 * i + 1] = MT::pack2(acc[i].z * inv, acc[i].w * inv);
    }
    if constexpr (VW == 4) {
      *(uint2*)(orow + dim_of(RUN, 4 * grp + wave, 0)) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int i = 0; i < VW / 2; i += 4) {
        const int d0 = dim_of(RUN, 4 * grp + wave, 2 * i);  // 8 consecutive elements
        if (PAIR && (d0 >= D / 2) != (half == 1)) continue;  // the other head's half
        *(uint4*)(orow + d0 - (PAIR ? (D / 2) * half : 0)) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
      }
    }
  }
}

// ------------------------------------------------------------ host side
static bool supported_head_dim(int d) { return d == 64 || d == 128 || d == 256; }

int decode_plan_params(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                       const int32_t* last_page_len, int32_t batch, int32_t page_size,
                       int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                       int64_t* kv_locations, void* workspace, int64_t workspace_bytes,
                       int64_t ws_offset, PlanParams* out, bool ragged_pair) {
  if (batch < 0 || !kv_indptr || !last_page_len || !workspace) return MI_ERR_INVALID;
  if (batch > 0 && !kv_indices) return MI_ERR_INVALID;
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads) return MI_ERR_INVALID;
  if (num_qo_heads / num_kv_heads > kRows) return MI_ERR_UNSUPPORTED;
  if (page_size <= 0) return MI_ERR_INVALID;
  if (page_size % 16) return MI_ERR_UNSUPPORTED;
  if (!supported_head_dim(head_dim)) return MI_ERR_UNSUPPORTED;
  const bool pair = pair_heads(qo_indptr, batch, num_kv_heads, num_qo_heads / num_kv_heads, head_dim, ragged_pair);
  const SplitLayout L = split_layout(batch, num_kv_heads, head_dim, workspace_bytes - ws_offset, pair);
  if (L.max_chunks <= batch || workspace_bytes < ws_offset + L.total) return MI_ERR_WORKSPACE;
  uint8_t* ws = (uint8_t*)workspace + ws_offset;
  PlanParams& pp = *out;
  pp.short_rows = pair_short_rows(pair);
  pp.qo_indptr = qo_indptr;
  pp.kv_indptr = kv_indptr;
  pp.num_pages = nullptr;
  pp.kv_indices = kv_indices;
  pp.last_page_len = last_page_len;
  pp.batch = batch;
  pp.target = L.max_chunks - batch;
  pp.min_chunk_pages = (kMinChunkTokens + page_size - 1) / page_size;
  pp.max_chunks = L.max_chunks;
  // resident workgroups per kv-head (or pair): two per CU at head_dim <= 128,
  // one for the head_dim 256 kernels
  const int heads = pair ? num_kv_heads / 2 : num_kv_heads;
  const int per_cu = (pair || head_dim > 128) ? 1 : 2;
  const int slots = device_cu_count() * per_cu / heads;
  pp.slots = slots < 1 ? 1 : (slots < L.max_chunks ? slots : L.max_chunks);
  pp.floor_pages = (kSmallChunkTokens + page_size - 1) / page_size;
  pp.group = num_qo_heads / num_kv_heads;
  pp.hdr = (int32_t*)(ws + L.hdr);
  pp.chunk_indptr = (int32_t*)(ws + L.chunk_indptr);
  pp.work = (int4*)(ws + L.work);
  pp.kv_locations = kv_locations;
  return MI_OK;
}

int decode_plan_impl(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                     const int32_t* last_page_len, int32_t batch, int32_t page_size,
                     int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                     int64_t* kv_locations, void* workspace, int64_t workspace_bytes,
                     int64_t ws_offset, hipStream_t stream) {
  PlanParams pp{};
  const int st = decode_plan_params(qo_indptr, kv_indptr, kv_indices, last_page_len, batch, page_size, num_qo_heads,
                                    num_kv_heads, head_dim, kv_locations, workspace, workspace_bytes, ws_offset, &pp);
  if (st != MI_OK) return st;
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(1024), 0, stream, pp);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

template <typename MT, bool FP8, int D>
static void launch_decode(const DecodeParams& dp, int grid, int batch, int phases, hipStream_t stream) {
  if (phases & kPhaseAttend)
    hipLaunchKernelGGL((decode_kernel<MT, FP8, D>), dim3(grid), dim3(256), 0, stream, dp);
  if ((phases & kPhaseMerge) && batch > 0)
    hipLaunchKernelGGL((merge_kernel<MT, D, lane_run(D, FP8 ? 1 : 2)>), dim3(batch * dp.num_kv_heads),
                       dim3(256), 0, stream, dp, batch);
}

// Paired kv-heads (dp.num_kv_heads counts pairs): the head_dim 256 kernels.
template <typename MT, bool FP8>
static void launch_decode_pair(const DecodeParams& dp, int grid, int batch, int phases, hipStream_t stream) {
  if (phases & kPhaseAttend)
    hipLaunchKernelGGL((decode_kernel<MT, FP8, 256, true>), dim3(grid), dim3(256), 0, stream, dp);
  if ((phases & kPhaseMerge) && batch > 0)
    hipLaunchKernelGGL((merge_kernel<MT, 256, lane_run(256, FP8 ? 1 : 2), true>),
                       dim3(batch * dp.num_kv_heads), dim3(256), 0, stream, dp, batch);
}

template <int D>
static void launch_merge_f32(const DecodeParams& dp, int batch, hipStream_t stream) {
  hipLaunchKernelGGL((merge_kernel<F32Out, D, lane_run(D, 4)>), dim3(batch * dp.num_kv_heads), dim3(256),
                     0, stream, dp, batch);
}

int merge_launch(const DecodeParams& dp, int head_dim, int out_dtype, int batch, hipStream_t stream) {
  if (out_dtype != MI_F32) return MI_ERR_UNSUPPORTED;
  if (batch <= 0) return MI_OK;
  switch (head_dim) {
    case 64: launch_merge_f32<64>(dp, batch, stream); break;
    case 128: launch_merge_f32<128>(dp, batch, stream); break;
    case 256: launch_merge_f32<256>(dp, batch, stream); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

template <typename MT, bool FP8>
static int dispatch_d(const DecodeParams& dp, int head_dim, int grid, int batch, int phases, hipStream_t stream) {
  switch (head_dim) {
    case 64: launch_decode<MT, FP8, 64>(dp, grid, batch, phases, stream); break;
    case 128: launch_decode<MT, FP8, 128>(dp, grid, batch, phases, stream); break;
    case 256: launch_decode<MT, FP8, 256>(dp, grid, batch, phases, stream); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

int decode_run_impl(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                    const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                    const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                    int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                    int64_t workspace_bytes, int64_t ws_offset, void* out,
                    int64_t out_stride_token, int64_t out_stride_head, int phases, hipStream_t stream,
                    bool ragged_pair) {
  if (!kv || batch < 0 || !workspace) return MI_ERR_INVALID;
  if (batch == 0) return MI_OK;
  if (!q || !out || !kv->data || !kv_indptr || !kv_indices || !last_page_len) return MI_ERR_INVALID;
  const int nkv = kv->num_kv_heads, D = kv->head_dim;
  if (nkv <= 0 || num_qo_heads <= 0 || num_qo_heads % nkv) return MI_ERR_INVALID;
  if (num_qo_heads / nkv > kRows) return MI_ERR_UNSUPPORTED;
  if (kv->page_size <= 0) return MI_ERR_INVALID;
  if (kv->page_size % 16 || !supported_head_dim(D)) return MI_ERR_UNSUPPORTED;
  const bool fp8 = kv->dtype == MI_FP8_E4M3;
  if (q_dtype != MI_BF16 && q_dtype != MI_F16 && q_dtype != MI_F32) return MI_ERR_UNSUPPORTED;
  if (!fp8 && kv->dtype != q_dtype) return MI_ERR_UNSUPPORTED;
  if (fp8 && q_dtype == MI_F32) return MI_ERR_UNSUPPORTED;
  if (fp8 && (!kv->k_scale || !kv->v_scale)) return MI_ERR_INVALID;
  const int qesz = q_dtype == MI_F32 ? 4 : 2;
  if (!rows_aligned16(q, q_stride_token, q_stride_head, qesz) ||
      !rows_aligned16(out, out_stride_token, out_stride_head, qesz) || !kv_aligned16(kv))
    return MI_ERR_INVALID;
  // the same pairing decision as the plan's (shapes only), so the layouts agree
  const bool pair = pair_heads(qo_indptr, batch, nkv, num_qo_heads / nkv, D, ragged_pair);
  const SplitLayout L = split_layout(batch, nkv, D, workspace_bytes - ws_offset, pair);
  if (L.max_chunks <= batch || workspace_bytes < ws_offset + L.total) return MI_ERR_WORKSPACE;
  uint8_t* ws = (uint8_t*)workspace + ws_offset;
  // the paired kernels: 16-bit caches whose pairs' two 128-element rows are
  // adjacent (NHD pools); fp8, fp32 and other layouts run the per-head
  // kernels on the same plan
  const bool pair_kernel = pair && !fp8 && q_dtype != MI_F32 && kv->head_stride == D;

  DecodeParams dp{};
  dp.q = q;
  dp.q_stride_tok = q_stride_token;
  dp.q_stride_head = q_stride_head;
  dp.kv = kv->data;
  dp.page_stride = kv->page_stride;
  dp.kv_stride = kv->kv_stride;
  dp.token_stride = kv->token_stride;
  dp.head_stride = kv->head_stride;
  dp.k_scale = kv->k_scale;
  dp.v_scale = kv->v_scale;
  dp.qo_indptr = qo_indptr;
  dp.kv_indptr = kv_indptr;
  dp.kv_indices = kv_indices;
  dp.last_page_len = last_page_len;
  dp.hdr = (const int32_t*)(ws + L.hdr);
  dp.work = (const int4*)(ws + L.work);
  dp.chunk_indptr = (const int32_t*)(ws + L.chunk_indptr);
  dp.lse_part = (float*)(ws + L.lse);
  dp.o_part = (float*)(ws + L.opart);
  dp.out = out;
  dp.out_stride_tok = out_stride_token;
  dp.out_stride_head = out_stride_head;
  dp.num_kv_heads = nkv;
  dp.group = num_qo_heads / nkv;
  dp.page_size = kv->page_size;
  dp.causal = causal ? 1 : 0;
  dp.scale_log2 = sm_scale * 1.4426950408889634f;
  dp.short_rows = pair_short_rows(pair);
  const int grid = (int)((L.max_chunks + 7) / 8 * 8 * (int64_t)nkv);
  int st;
  if (pair_kernel) {
    dp.num_kv_heads = nkv / 2;
    dp.head_stride = 2 * kv->head_stride;
    const int pgrid = (int)((L.max_chunks + 7) / 8 * 8 * (int64_t)(nkv / 2));
    if (q_dtype == MI_BF16)
      fp8 ? launch_decode_pair<BF16, true>(dp, pgrid, batch, phases, stream)
          : launch_decode_pair<BF16, false>(dp, pgrid, batch, phases, stream);
    else
      fp8 ? launch_decode_pair<F16, true>(dp, pgrid, batch, phases, stream)
          : launch_decode_pair<F16, false>(dp, pgrid, batch, phases, stream);
    MI_CHECK_LAUNCH();
    return MI_OK;
  }
  if (q_dtype == MI_F32) {  // fp32 q, cache and output
    st = MI_OK;
    if (phases & kPhaseAttend) st = f32_attend_launch(dp, D, grid, stream);
    if (st == MI_OK && (phases & kPhaseMerge)) st = merge_launch(dp, D, MI_F32, batch, stream);
    if (st != MI_OK) return st;
    MI_CHECK_LAUNCH();
    return MI_OK;
  }
  if (q_dtype == MI_BF16)
    st = fp8 ? dispatch_d<BF16, true>(dp, D, grid, batch, phases, stream)
             : dispatch_d<BF16, false>(dp, D, grid, batch, phases, stream);
  else
    st = fp8 ? dispatch_d<F16, true>(dp, D, grid, batch, phases, stream)
             : dispatch_d<F16, false>(dp, D, grid, batch, phases, stream);
  if (st != MI_OK) return st;
  MI_CHECK_LAUNCH();
  return MI_OK;
}

int64_t decode_workspace_bytes_impl(int32_t batch, int32_t num_kv_heads, int32_t head_dim) {
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0) return MI_ERR_INVALID;
  return split_layout(batch, num_kv_heads, head_dim, -1).total;
}

}  // namespace mi

extern "C" {

int64_t mi_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim) {
  if (num_qo_heads <= 0) return MI_ERR_INVALID;
  return mi::decode_workspace_bytes_impl(batch, num_kv_heads, head_dim);
}

int mi_decode_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                   const int32_t* last_page_len, int32_t batch, int32_t page_size,
                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                   int64_t* kv_locations, void* workspace, int64_t workspace_bytes, void* stream) {
  return mi::decode_plan_impl(qo_indptr, kv_indptr, kv_indices, last_page_len, batch, page_size,
                              num_qo_heads, num_kv_heads, head_dim, kv_locations, workspace,
                              workspace_bytes, 0, (hipStream_t)stream);
}

#define MI_DECODE_ARGS                                                                           \
  const void *q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,                 \
      const mi_paged_kv *kv, const int32_t *qo_indptr, const int32_t *kv_indptr,                 \
      const int32_t *kv_indices, const int32_t *last_page_len, int32_t batch, int32_t num_qo_heads, \
      int32_t causal, float sm_scale, void *workspace, int64_t workspace_bytes, void *out,       \
      int64_t out_stride_token, int64_t out_stride_head, void *stream
#define MI_DECODE_FWD(phases)                                                                      \
  mi::decode_run_impl(q, q_dtype, q_stride_token, q_stride_head, kv, qo_indptr, kv_indptr,         \
                      kv_indices, last_page_len, batch, num_qo_heads, causal, sm_scale, workspace, \
                      workspace_bytes, 0, out, out_stride_token, out_stride_head, phases,          \
                      (hipStream_t)stream)

int mi_decode_run(MI_DECODE_ARGS) { return MI_DECODE_FWD(mi::kPhaseAttend | mi::kPhaseMerge); }
int mi_decode_attend(MI_DECODE_ARGS) { return MI_DECODE_FWD(mi::kPhaseAttend); }
int mi_decode_merge(MI_DECODE_ARGS) { return MI_DECODE_FWD(mi::kPhaseMerge); }

}  // extern "C"
