// fp32 paged attention (fp32 KV cache, fp32 q and output) for MI355X (gfx950).
//
// The reference allocates the KV pool in the model's autocast dtype, fp32
// included (mstar/engine/kv_cache_engine.py:104-105, 132-136; Pi0.5 runs its
// real weights with kv_cache_type=torch.float32), and plans its wrappers in
// the cache's dtype (mstar/engine/cache_manager.py:241-247), so q, K, V and
// the output are fp32.  This file computes that case in fp32 throughout with
// the fp32 matrix instruction v_mfma_f32_16x16x4_f32:
//
//   decode  (the decode plan's split-KV items: decode steps and the
//           short-query requests of a ragged batch): one workgroup per
//           (item, kv-head), its 4 wavefronts over contiguous quarters of
//           the item's 16-token tiles; partials in the bf16 decode kernel's
//           layout, so its merge (with fp32 output) finishes split requests;
//   prefill (the long-query requests): one workgroup per (tile of the
//           prefill plan, kv-head, 16-row block), its 4 wavefronts over
//           contiguous quarters of the keys the block's rows can see.
//
// Per 16-token tile, a wavefront holds 16 (query token, q-head) rows of one
// kv-head as the 16 MFMA columns (GQA rows packed token-major, so a K/V row
// is read once per q-head group):
//   S^T[16 keys x 16 rows] = K . Q^T     D/4 MFMAs; k slot g of step s is dim
//                                         (D/4)*g + s, so a lane's Q and K
//                                         operands are D/4 consecutive floats
//                                         of one row
//   online softmax in fp32 (exp2 domain), causal limit aligned to the end of
//   the KV
//   O^T[16 dims x 16 rows] += V^T . P^T  4 MFMAs per 16-dim output tile; k
//                                         slot g of step t is key 4g + t, so
//                                         the B operand is the lane's own
//                                         probability of key 4g + t; output
//                                         row i of tile m is the dim that
//                                         lane i loaded as its element m, so
//                                         the A operand is one of the lane's
//                                         own V floats
// Each lane loads, for its 4 keys 4g..4g+3, D/16 floats with 16-byte loads,
// each load instruction covering 256 contiguous bytes of the key row
// (dim_of in mi_plan.h).  K takes the same load layout and passes through a
// per-wavefront LDS buffer in natural dim order, where each lane reads back
// its key's D/4-float operand run.
#include "mi_common.h"
#include "mi_internal.h"
#include "mi_plan.h"

namespace mi {

struct F32Tiles {
  const int32_t* hdr;  // [0]: tiles listed by the prefill plan
  const int2* tiles;   // (request, first row)
  int32_t tile_rows;
};

template <int D>
struct F32Regs {  // lane: keys 4*grp + r, dims dim_of(lane_run(D, 4), col, j), j < D/16
  float4 k[4][D / 64];
  float4 v[4][D / 64];
};

template <int N>
MI_DEVICE void load_f4(float4 (&dst)[N], const uint8_t* src) {  // float4 i: 256*i bytes into the row (dim_of)
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint4 u = nt_load16(src + 256 * i);
    dst[i] = make_float4(bitcast<float>(u.x), bitcast<float>(u.y), bitcast<float>(u.z), bitcast<float>(u.w));
  }
}

MI_DEVICE float f4_at(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

MI_DEVICE f32x4 mma_f32(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

template <int D, bool PREFILL>
__global__ __launch_bounds__(256) void attend_f32_kernel(DecodeParams p, F32Tiles pt) {
  constexpr int VW = D / 16;      // output dim tiles; floats per lane of a key row
  constexpr int NV = VW / 4;      // float4 per lane of a key row
  constexpr int KQ = D / 4;       // S MFMA steps; floats of a lane's Q / K operand run
  constexpr int KRS = D * 4 + 16;  // LDS row stride of the K staging buffer (bytes): rows 4 banks apart
  constexpr int RUN = lane_run(D, 4);  // consecutive floats per lane (dim_of)
  constexpr float kNegInf = -__builtin_inff();
  constexpr int kStageBytes = 4 * 16 * KRS;
  constexpr int kMergeBytes = 4 * (4 * NV * 64 * 16);
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes];
  __shared__ float lds_m[4][kRows], lds_l[4][kRows];

  const int lane = lane_id();
  const int wave = uniform((int)threadIdx.x >> 6);
  const int nkv = p.num_kv_heads;
  const int G = p.group;
  const int ps = p.page_size;
  int b, h, row0, kidx = 0, nitems_b = 1, pg_end;
  if constexpr (PREFILL) {
    const int bpt = pt.tile_rows / kRows;  // 16-row blocks per tile
    const int x = (int)blockIdx.x;
    const int j = x % bpt, rest = x / bpt;
    h = uniform(rest % nkv);
    const int t = rest / nkv;
    if (t >= pt.hdr[0]) return;  // uniform
    const int2 tile = pt.tiles[t];
    b = uniform(tile.x);
    row0 = uniform(tile.y + kRows * j);
  } else {
    // the decode kernel's XCD-aware mapping: the kv-heads of an item share an XCD
    const int gsz = 8 * nkv;
    const int gi = uniform((int)blockIdx.x / gsz);
    const int gr = (int)blockIdx.x - gi * gsz;
    h = uniform(gr >> 3);
    const int item = uniform(gi * 8 + (gr & 7));
    if (item >= p.hdr[kHdrChunks]) return;
    const int4 wk = p.work[item];
    b = uniform(wk.x);
    kidx = uniform(wk.y);
    nitems_b = uniform(wk.w);
    row0 = 0;
    pg_end = uniform(wk.z);
  }
  const int page_base = p.kv_indptr[b];
  const int np = p.kv_indptr[b + 1] - page_base;
  const int kv_len = (np - 1) * ps + p.last_page_len[b];
  int qo_start = b, qo_len = 1;
  if (p.qo_indptr) {
    qo_start = p.qo_indptr[b];
    qo_len = p.qo_indptr[b + 1] - qo_start;
  }
  const int rows = min(qo_len * G - row0, kRows);  // rows of this block
  if (rows <= 0) return;                           // uniform: past the request's last row
  const int first_qtok = row0 / G, last_qtok = (row0 + rows - 1) / G;
  int tok0, tok1;  // key range of the unit
  if constexpr (PREFILL) {
    pg_end = np;
    tok0 = 0;
    tok1 = p.causal ? min(kv_len, kv_len - qo_len + last_qtok + 1) : kv_len;
  } else {
    tok0 = kidx * p.hdr[kHdrChunkPages] * ps;
    tok1 = min(pg_end * ps, kv_len);
  }
  const int unit_tiles = tok1 > tok0 ? (tok1 - tok0 + 15) >> 4 : 0;
  const int tq = unit_tiles >> 2, trem = unit_tiles & 3;
  const int my_t0 = wave * tq + min(wave, trem);
  const int ntiles = tq + (wave < trem ? 1 : 0);
  const int tok_begin = tok0 + 16 * my_t0;

  const int col = lane & 15;  // MFMA column = row of the block
  const int grp = lane >> 4;
  const int row = row0 + col;
  const int qtok = row / G;
  const int g = row - qtok * G;
  const bool row_valid = col < rows;
  int lim = p.causal ? (kv_len - qo_len + qtok) : (kv_len - 1);
  lim = min(lim, kv_len - 1);
  const int mask_from = p.causal ? (kv_len - qo_len + first_qtok + 1) : kv_len;  // keys >= this need a row check

  // Q as the B operand of S^T = K Q^T: lane holds Q[row][KQ*grp, +KQ)
  float4 qf[KQ / 4];
  {
    const float* qrow = (const float*)p.q + (int64_t)(qo_start + qtok) * p.q_stride_tok +
                        (int64_t)(h * G + g) * p.q_stride_head + KQ * grp;
#pragma unroll
    for (int i = 0; i < KQ / 4; ++i) qf[i] = row_valid ? *(const float4*)(qrow + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float sl2 = p.scale_log2;

  const uint8_t* kv = (const uint8_t*)p.kv;
  const int64_t head_off = (int64_t)h * p.head_stride * 4;
  const uint32_t voff0 = (uint32_t)((4 * grp) * p.token_stride + RUN * col) * 4;
  const uint32_t vrow = (uint32_t)(p.token_stride * 4);
  const int64_t kvhalf = p.kv_stride * 4;
  auto tile_base = [&](int page, int r0) -> const uint8_t* {
    return kv + (int64_t)page * p.page_stride * 4 + (int64_t)r0 * p.token_stride * 4 + head_off;
  };
  auto load_tile = [&](F32Regs<D>& t, const uint8_t* base) {
    const uint8_t* kb = base + voff0;
#pragma unroll
    for (int r = 0; r < 4; ++r) load_f4(t.k[r], kb + r * vrow);
    const uint8_t* vb = kb + kvhalf;
#pragma unroll
    for (int r = 0; r < 4; ++r) load_f4(t.v[r], vb + r * vrow);
  };
  uint8_t* kst = &lds[wave * 16 * KRS];

  f32x4 acc[VW];
#pragma unroll
  for (int m = 0; m < VW; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  auto compute_tile = [&](F32Regs<D>& t, int ti) {
    const int tb = tok_begin + 16 * ti;
    // K rows -> LDS (row 4*grp + r, dims [VW*col, +VW)) -> A operand runs
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = (float*)(kst + (4 * grp + r) * KRS);  // row in natural dim order
#pragma unroll
      for (int i = 0; i < NV; ++i) *(float4*)(dst + dim_of(RUN, col, 4 * i)) = t.k[r][i];
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    const float4* krun = (const float4*)(kst + col * KRS + KQ * grp * 4);
#pragma unroll
    for (int i = 0; i < KQ / 4; ++i) {
      const float4 a = krun[i];
      s = mma_f32(a.x, qf[i].x, s);
      s = mma_f32(a.y, qf[i].y, s);
      s = mma_f32(a.z, qf[i].z, s);
      s = mma_f32(a.w, qf[i].w, s);
    }
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sv[r] = s[r] * sl2;
    if (tb + 16 > mask_from) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = tb + 4 * grp + r;
        if (key > lim) sv[r] = kNegInf;
        if (key >= kv_len) {  // slots past the end hold stale data: keep NaN/Inf out of P.V
#pragma unroll
          for (int i = 0; i < NV; ++i) t.v[r][i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
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
      for (int m = 0; m < VW; ++m) acc[m] *= alpha;
    }
    m_run = m_new;
#pragma unroll
    for (int m = 0; m < VW; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[m] = mma_f32(f4_at(t.v[r][m >> 2], m & 3), pr[r], acc[m]);
  };

  // Tile loop in windows of 64 pages: the window's page ids sit in one VGPR
  // (lane i: page i of the window) and v_readlane hands each tile's page to
  // the scalar unit; loads run one tile ahead of the MFMA work.
  for (int w0 = 0; w0 < ntiles;) {
    const int wtok = tok_begin + 16 * w0;
    const int first = wtok / ps;
    const int wt = min(ntiles - w0, ((first + 64) * ps - wtok) >> 4);
    const int pwin = first + lane < pg_end ? p.kv_indices[page_base + first + lane] : 0;
    auto tile_ptr = [&](int t) -> const uint8_t* {
      const int tok = wtok + 16 * t;
      return tile_base(__builtin_amdgcn_readlane(pwin, tok / ps - first), tok % ps);
    };
    F32Regs<D> A, B;
    load_tile(A, tile_ptr(0));
    int t = 0;
    for (; t + 2 < wt; t += 2) {  // every load in range: exact vmcnt waits
      load_tile(B, tile_ptr(t + 1));
      compute_tile(A, w0 + t);
      load_tile(A, tile_ptr(t + 2));
      compute_tile(B, w0 + t + 1);
    }
    if (t + 1 < wt) {
      load_tile(B, tile_ptr(t + 1));
      compute_tile(A, w0 + t);
      compute_tile(B, w0 + t + 1);
    } else {
      compute_tile(A, w0 + t);
    }
    w0 += wt;
  }

  // Merge the 4 wavefronts' states in LDS (same register layout in every
  // wavefront: lane -> row col, dims VW*(4*grp + r) + m); wavefront w
  // finishes the dims with r == w.
  __syncthreads();
  {
    const float l_row = rows4_sum(l_run);
    if (grp == 0) {
      lds_m[wave][col] = m_run;
      lds_l[wave][col] = l_row;
    }
    float4* st = (float4*)lds + (size_t)wave * 4 * NV * 64 + lane;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < VW; m += 4)
        st[(r * NV + m / 4) * 64] = make_float4(acc[m][r], acc[m + 1][r], acc[m + 2][r], acc[m + 3][r]);
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, lds_m[w][col]);
  const float M_use = M == kNegInf ? 0.f : M;
  float sc[4], L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    sc[w] = fast_exp2(lds_m[w][col] - M_use);
    L += sc[w] * lds_l[w][col];
  }
  float4 o[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) o[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4* src = (const float4*)lds + (size_t)w * 4 * NV * 64 + (size_t)wave * NV * 64 + lane;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float4 v = src[i * 64];
      o[i].x += sc[w] * v.x;
      o[i].y += sc[w] * v.y;
      o[i].z += sc[w] * v.z;
      o[i].w += sc[w] * v.w;
    }
  }
  const float inv = L > 0.f ? 1.f / L : (L == 0.f ? 0.f : __builtin_nanf(""));  // NaN L: keep the row NaN
  if (!row_valid) return;
  if (nitems_b == 1) {  // dims dim_of(RUN, 4*grp + wave, j) of row col
    float* dst = (float*)p.out + (int64_t)(qo_start + qtok) * p.out_stride_tok +
                 (int64_t)(h * G + g) * p.out_stride_head;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      *(float4*)(dst + dim_of(RUN, 4 * grp + wave, 4 * i)) = make_float4(o[i].x * inv, o[i].y * inv, o[i].z * inv, o[i].w * inv);
  } else {  // partial (o, lse) in the split-KV layout of the decode kernel
    const int64_t unit_idx = (int64_t)(p.chunk_indptr[b] + kidx) * nkv + h;
    float* ob = p.o_part + unit_idx * kRows * D + 4 * lane;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      *(float4*)(ob + 256 * (wave * NV + i)) = make_float4(o[i].x * inv, o[i].y * inv, o[i].z * inv, o[i].w * inv);
    if (wave == 0 && grp == 0)  // -inf: empty partial; NaN: the row met a NaN or +inf score
      p.lse_part[unit_idx * kRows + col] = L > 0.f ? M + fast_log2(L) : (L == 0.f ? kNegInf : __builtin_nanf(""));
  }
}

template <int D, bool PREFILL>
static void launch_f32(const DecodeParams& dp, const F32Tiles& pt, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((attend_f32_kernel<D, PREFILL>), dim3(grid), dim3(256), 0, stream, dp, pt);
}

template <bool PREFILL>
static int dispatch_f32(const DecodeParams& dp, const F32Tiles& pt, int head_dim, int grid, hipStream_t stream) {
  switch (head_dim) {
    case 64: launch_f32<64, PREFILL>(dp, pt, grid, stream); break;
    case 128: launch_f32<128, PREFILL>(dp, pt, grid, stream); break;
    case 256: launch_f32<256, PREFILL>(dp, pt, grid, stream); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

int f32_attend_launch(const DecodeParams& dp, int head_dim, int grid, hipStream_t stream) {
  if (grid <= 0) return MI_OK;
  return dispatch_f32<false>(dp, F32Tiles{nullptr, nullptr, 0}, head_dim, grid, stream);
}

int f32_prefill_launch(const DecodeParams& dp, const int32_t* tile_hdr, const int2* tiles, int max_tiles,
                       int tile_rows, int head_dim, hipStream_t stream) {
  if (tile_rows <= 0 || tile_rows % kRows) return MI_ERR_INVALID;
  const int64_t grid = (int64_t)max_tiles * dp.num_kv_heads * (tile_rows / kRows);
  if (grid <= 0) return MI_OK;
  if (grid > 0x7fffffff) return MI_ERR_UNSUPPORTED;
  return dispatch_f32<true>(dp, F32Tiles{tile_hdr, tiles, tile_rows}, head_dim, (int)grid, stream);
}

}  // namespace mi
