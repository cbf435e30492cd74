// Ragged paged prefill (P3 + P7) for MI355X (gfx950).
//
// Replaces FlashInferPrefillWrapper.plan/run (mstar/utils/flashinfer_utils.py:162-269).
//
// plan:  token_map_kernel writes the per-new-token (page, slot) map of
//        flashinfer_utils.py:211-256; prefill_plan_kernel lists the
//        128-row tiles of every long-query request; short-query requests
//        (qo_len * group <= 16, e.g. the decode rows of a mixed batch) get a
//        split-KV plan for the decode kernel in the same workspace.
// run:   decode kernel + merge for the short-query requests, then
//        prefill_kernel for the tiles.
//
// prefill_kernel: one workgroup = 4 wavefronts = 128 (query token, q-head)
// rows of one request and one kv-head (GQA rows packed token-major, so K/V
// are read once per group of q-heads).  Each wavefront owns 2 groups of 16
// rows.  K/V tiles of 64 keys (32 for head_dim 256) are gathered from the
// paged cache with 128-bit loads into registers one tile ahead, then stored
// to LDS (rows padded by 16 bytes against bank conflicts) and shared by the
// 4 wavefronts:
//   S^T[16 keys x 16 rows] = K . Q^T    (v_mfma_f32_16x16x32, K from LDS)
//   online softmax in fp32 (exp2 domain), causal mask aligned to the end of the KV
//   O^T[D x 16 rows]      += V^T . P^T  (v_mfma_f32_16x16x16, V transposed in registers)
// fp8 K/V are converted to the MFMA type when a tile is stored to LDS; the
// per-head scales multiply the scores and the output.
// Workgroups are mapped XCD-aware: the 8 XCDs each take a contiguous range of
// (kv-head, tile) units, so the tiles of one request and head share an L2.
#include "mi_common.h"
#include "mi_internal.h"

namespace mi {

constexpr int kTileRows = 128;  // rows per workgroup
constexpr int kShortRows = 16;  // qo_len * group <= 16 -> decode kernel

struct PrefillLayout {
  int64_t hdr, tiles, split;
  int32_t max_tiles;
};

static PrefillLayout prefill_layout(int32_t batch, int32_t max_qo_tokens, int32_t group) {
  PrefillLayout L;
  const int64_t rows = (int64_t)max_qo_tokens * group;
  int64_t mt = (rows + kTileRows - 1) / kTileRows + batch;
  if (mt > (1 << 28)) mt = 1 << 28;
  L.max_tiles = (int32_t)mt;
  L.hdr = 0;
  L.tiles = 256;
  L.split = mi_align_up(L.tiles + 8LL * L.max_tiles, 256);
  return L;
}

// ------------------------------------------------------------ token map
__global__ __launch_bounds__(256) void token_map_kernel(const int32_t* qo_indptr, const int32_t* kv_indptr,
                                                        const int32_t* kv_indices, const int32_t* last_page_len,
                                                        int32_t batch, int32_t page_size, int64_t* t2p,
                                                        int64_t* t2c, int32_t map_len) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= map_len) return;
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
__global__ __launch_bounds__(1024) void prefill_plan_kernel(const int32_t* qo_indptr, int32_t batch,
                                                            int32_t group, int32_t max_tiles, int32_t* hdr,
                                                            int2* tiles) {
  __shared__ int smem[16];
  int carry = 0;
  for (int base = 0; base < batch; base += 1024) {
    const int b = base + (int)threadIdx.x;
    int n = 0;
    if (b < batch) {
      const int rows = (qo_indptr[b + 1] - qo_indptr[b]) * group;
      n = rows > kShortRows ? (rows + kTileRows - 1) / kTileRows : 0;
    }
    int total;
    const int first = block_exclusive_scan_1024(n, total, smem) + carry;
    for (int i = 0; i < n && first + i < max_tiles; ++i)
      tiles[first + i] = make_int2(b, (n - 1 - i) * kTileRows);  // causal: heaviest tile first
    carry += total;
  }
  if (threadIdx.x == 0) hdr[0] = min(carry, max_tiles);
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
  void* out;
  int64_t out_stride_tok, out_stride_head;
  int32_t num_kv_heads, group, page_size, causal;
  float scale_log2;
};

template <typename MT, bool FP8, int D>
struct PrefillCfg {
  static constexpr int KEYS = D > 128 ? 32 : 64;          // keys per LDS tile
  static constexpr int RS = D * 2 + 16;                   // LDS row stride (bytes, 16-bit elements)
  static constexpr int ESZ = FP8 ? 1 : 2;                 // cache element size
  static constexpr int CPR = D * ESZ / 16;                // 16-byte chunks per cached row
  static constexpr int RPP = 256 / CPR;                   // rows per loader pass
  static constexpr int NP = KEYS / RPP;                   // loader passes per tile
  static_assert(KEYS % RPP == 0, "loader mapping");
};

template <typename MT, bool FP8, int D>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p) {
  using C = PrefillCfg<MT, FP8, D>;
  constexpr int KS = D / 32, VW = D / 16, KEYS = C::KEYS, RS = C::RS, ESZ = C::ESZ;
  constexpr int NSUB = KEYS / 16;
  constexpr float kNegInf = -__builtin_inff();
  __shared__ __attribute__((aligned(16))) uint8_t lds_k[KEYS * RS];
  __shared__ __attribute__((aligned(16))) uint8_t lds_v[KEYS * RS];

  // ---- XCD-aware unit: XCD x = blockIdx % 8 takes units [x*per, (x+1)*per)
  const int nkv = p.num_kv_heads;
  const int n_tiles = p.hdr[0];
  const int n_units = n_tiles * nkv;
  const int per_xcd = (n_units + 7) >> 3;
  const int j = (int)blockIdx.x >> 3;
  const int unit = ((int)blockIdx.x & 7) * per_xcd + j;
  if (j >= per_xcd || unit >= n_units) return;
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

  // ---- this lane's two query rows (one per 16-row group)
  uint4 qf[2][KS];
  int lim[2];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
    const int n = row0 + 32 * wave + 16 * rg + col;
    const int tok = n / G, g = n - tok * G;
    const bool valid = n < rows_total;
    int l = p.causal ? (kv_len - qo_len + tok) : (kv_len - 1);
    lim[rg] = min(l, kv_len - 1);
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(qo_start + tok) * p.q_stride_tok +
                           (int64_t)(h * G + g) * p.q_stride_head;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[rg][s] = valid ? *(const uint4*)(qrow + 32 * s + 8 * grp) : make_uint4(0, 0, 0, 0);
  }
  // ---- keys this workgroup needs, and where per-row masking starts
  const int last_row = min(row0 + kTileRows, rows_total) - 1;
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

  // ---- cooperative tile loader: thread -> (row tid / CPR + pass*RPP, chunk tid % CPR)
  const uint8_t* kvb = (const uint8_t*)p.kv + (int64_t)h * p.head_stride * ESZ;
  const int lrow = tid / C::CPR, lchunk = tid - lrow * C::CPR;
  uint4 kreg[C::NP], vreg[C::NP];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < C::NP; ++i) {
      const int key = kt * KEYS + i * C::RPP + lrow;
      if (key < kv_end) {
        const int page = p.kv_indices[page_base + key / ps];
        const uint8_t* src = kvb + ((int64_t)page * p.page_stride + (int64_t)(key % ps) * p.token_stride) * ESZ +
                             16 * lchunk;
        kreg[i] = *(const uint4*)src;
        vreg[i] = *(const uint4*)(src + p.kv_stride * ESZ);
      } else {
        kreg[i] = make_uint4(0, 0, 0, 0);
        vreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < C::NP; ++i) {
      const int r = i * C::RPP + lrow;
      if constexpr (FP8) {  // 16 fp8 -> 16 MFMA-type elements (32 bytes)
        const uint32_t kw[4] = {kreg[i].x, kreg[i].y, kreg[i].z, kreg[i].w};
        const uint32_t vw[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
        uint32_t ko[8], vo[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          ko[2 * w] = fp8x2_to_mt<MT>(kw[w], false);
          ko[2 * w + 1] = fp8x2_to_mt<MT>(kw[w], true);
          vo[2 * w] = fp8x2_to_mt<MT>(vw[w], false);
          vo[2 * w + 1] = fp8x2_to_mt<MT>(vw[w], true);
        }
        uint8_t* kd = lds_k + r * RS + 32 * lchunk;
        uint8_t* vd = lds_v + r * RS + 32 * lchunk;
        *(uint4*)kd = make_uint4(ko[0], ko[1], ko[2], ko[3]);
        *(uint4*)(kd + 16) = make_uint4(ko[4], ko[5], ko[6], ko[7]);
        *(uint4*)vd = make_uint4(vo[0], vo[1], vo[2], vo[3]);
        *(uint4*)(vd + 16) = make_uint4(vo[4], vo[5], vo[6], vo[7]);
      } else {
        *(uint4*)(lds_k + r * RS + 16 * lchunk) = kreg[i];
        *(uint4*)(lds_v + r * RS + 16 * lchunk) = vreg[i];
      }
    }
  };

  f32x4 acc[2][VW];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int jj = 0; jj < VW; ++jj) acc[rg][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {kNegInf, kNegInf}, l_run[2] = {0.f, 0.f};

  auto compute = [&](int kt) {
    const int kb = kt * KEYS;
    // S^T for both row groups, NSUB sub-tiles of 16 keys
    f32x4 s[2][NSUB];
#pragma unroll
    for (int js = 0; js < NSUB; ++js) {
      s[0][js] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[1][js] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const uint4 a = *(const uint4*)(lds_k + (16 * js + col) * RS + (8 * grp + 32 * st) * 2);
        s[0][js] = MT::mma_16x16x32(a, qf[0][st], s[0][js]);
        s[1][js] = MT::mma_16x16x32(a, qf[1][st], s[1][js]);
      }
    }
    const bool need_mask = kb + KEYS > mask_from;
    uint2 pb[2][NSUB];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) {
      float sv[NSUB][4];
      float mt = kNegInf;
#pragma unroll
      for (int js = 0; js < NSUB; ++js)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = s[rg][js][r] * sl2;
          if (need_mask && kb + 16 * js + 4 * grp + r > lim[rg]) x = kNegInf;
          sv[js][r] = x;
          mt = fmaxf(mt, x);
        }
      mt = rows4_max(mt);
      const float m_new = fmaxf(m_run[rg], mt);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[rg] - m_use);
      float psum = 0.f;
#pragma unroll
      for (int js = 0; js < NSUB; ++js) {
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pr[r] = fast_exp2(sv[js][r] - m_use);
          psum += pr[r];
        }
        pb[rg][js] = make_uint2(MT::pack2(pr[0], pr[1]), MT::pack2(pr[2], pr[3]));
      }
      l_run[rg] = l_run[rg] * alpha + psum;
      if (__builtin_amdgcn_ballot_w64(m_new > m_run[rg])) {
#pragma unroll
        for (int jj = 0; jj < VW; ++jj) acc[rg][jj] *= alpha;
      }
      m_run[rg] = m_new;
    }
    // O^T += V^T P^T; lane reads rows 16js+4grp+r, elements [VW*col, VW*col+VW)
#pragma unroll
    for (int js = 0; js < NSUB; ++js) {
      uint32_t vv[4][VW / 2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint8_t* src = lds_v + (16 * js + 4 * grp + r) * RS + VW * col * 2;
        if constexpr (VW == 4) {
          const uint2 t = *(const uint2*)src;
          vv[r][0] = t.x;
          vv[r][1] = t.y;
        } else {
#pragma unroll
          for (int i = 0; i < VW / 2; i += 4) {
            const uint4 t = *(const uint4*)(src + 4 * i);
            vv[r][i] = t.x;
            vv[r][i + 1] = t.y;
            vv[r][i + 2] = t.z;
            vv[r][i + 3] = t.w;
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < VW; ++jj) {
        uint2 a;
        if (jj & 1) {
          a.x = pack_hi16(vv[0][jj >> 1], vv[1][jj >> 1]);
          a.y = pack_hi16(vv[2][jj >> 1], vv[3][jj >> 1]);
        } else {
          a.x = pack_lo16(vv[0][jj >> 1], vv[1][jj >> 1]);
          a.y = pack_lo16(vv[2][jj >> 1], vv[3][jj >> 1]);
        }
        acc[0][jj] = MT::mma_16x16x16(a, pb[0][js], acc[0][jj]);
        acc[1][jj] = MT::mma_16x16x16(a, pb[1][js], acc[1][jj]);
      }
    }
  };

  if (n_kt > 0) {
    load_tile(0);
    store_tile();
    __syncthreads();
    for (int kt = 0; kt < n_kt; ++kt) {
      if (kt + 1 < n_kt) load_tile(kt + 1);  // global loads in flight during compute
      compute(kt);
      __syncthreads();
      if (kt + 1 < n_kt) {
        store_tile();
        __syncthreads();
      }
    }
  }

  // ---- epilogue
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
    const float l_tot = rows4_sum(l_run[rg]);
    const float inv = l_tot > 0.f ? vscale / l_tot : 0.f;
    const int n = row0 + 32 * wave + 16 * rg + col;
    if (n >= rows_total) continue;
    const int tok = n / G, g = n - tok * G;
    uint16_t* orow = (uint16_t*)p.out + (int64_t)(qo_start + tok) * p.out_stride_tok +
                     (int64_t)(h * G + g) * p.out_stride_head;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t w[VW / 2];
#pragma unroll
      for (int i = 0; i < VW / 2; ++i) w[i] = MT::pack2(acc[rg][2 * i][r] * inv, acc[rg][2 * i + 1][r] * inv);
      uint16_t* dst = orow + VW * (4 * grp + r);
      if constexpr (VW == 4) {
        *(uint2*)dst = make_uint2(w[0], w[1]);
      } else {
#pragma unroll
        for (int i = 0; i < VW / 2; i += 4) *(uint4*)(dst + 2 * i) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
      }
    }
  }
}

template <typename MT, bool FP8>
static int launch_prefill(const PrefillParams& pp, int head_dim, int grid, hipStream_t stream) {
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 64>), dim3(grid), dim3(256), 0, stream, pp); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 128>), dim3(grid), dim3(256), 0, stream, pp); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<MT, FP8, 256>), dim3(grid), dim3(256), 0, stream, pp); break;
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
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, num_qo_heads / num_kv_heads);
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
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, G);
  if (workspace_bytes < L.split) return MI_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  if (token_map_len > 0) {
    hipLaunchKernelGGL(token_map_kernel, dim3((token_map_len + 255) / 256), dim3(256), 0, s, qo_indptr, kv_indptr,
                       kv_indices, last_page_len, batch, page_size, token_to_page, token_to_cache, token_map_len);
  }
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(1024), 0, s, qo_indptr, batch, G, L.max_tiles,
                     (int32_t*)(ws + L.hdr), (int2*)(ws + L.tiles));
  MI_CHECK_LAUNCH();
  return decode_plan_impl(qo_indptr, kv_indptr, kv_indices, last_page_len, batch, page_size, num_qo_heads,
                          num_kv_heads, head_dim, nullptr, workspace, workspace_bytes, L.split, s);
}

extern "C" int mi_prefill_run(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                              const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                              int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, float sm_scale,
                              void* workspace, int64_t workspace_bytes, void* out, int64_t out_stride_token,
                              int64_t out_stride_head, void* stream) {
  using namespace mi;
  if (!kv || batch < 0 || max_qo_tokens < 0 || !workspace) return MI_ERR_INVALID;
  if (batch == 0) return MI_OK;
  if (!q || !out || !kv->data || !qo_indptr || !kv_indptr || !kv_indices || !last_page_len) return MI_ERR_INVALID;
  const int nkv = kv->num_kv_heads, D = kv->head_dim;
  if (nkv <= 0 || num_qo_heads <= 0 || num_qo_heads % nkv) return MI_ERR_INVALID;
  const int G = num_qo_heads / nkv;
  if (G > kShortRows || kv->page_size % 16 || !ok_head_dim(D)) return MI_ERR_UNSUPPORTED;
  const bool fp8 = kv->dtype == MI_FP8_E4M3;
  if (q_dtype != MI_BF16 && q_dtype != MI_F16) return MI_ERR_UNSUPPORTED;
  if (!fp8 && kv->dtype != q_dtype) return MI_ERR_UNSUPPORTED;
  if (fp8 && (!kv->k_scale || !kv->v_scale)) return MI_ERR_INVALID;
  const PrefillLayout L = prefill_layout(batch, max_qo_tokens, G);
  if (workspace_bytes < L.split) return MI_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  // short-query requests: split-KV decode kernel + merge
  int st = decode_run_impl(q, q_dtype, q_stride_token, q_stride_head, kv, qo_indptr, kv_indptr, kv_indices,
                           last_page_len, batch, num_qo_heads, causal, sm_scale, workspace, workspace_bytes,
                           L.split, out, out_stride_token, out_stride_head, kPhaseAttend | kPhaseMerge, s);
  if (st != MI_OK) return st;
  // long-query requests: MFMA prefill tiles
  const uint8_t* ws = (const uint8_t*)workspace;
  PrefillParams pp;
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
  pp.out = out;
  pp.out_stride_tok = out_stride_token;
  pp.out_stride_head = out_stride_head;
  pp.num_kv_heads = nkv;
  pp.group = G;
  pp.page_size = kv->page_size;
  pp.causal = causal ? 1 : 0;
  pp.scale_log2 = sm_scale * 1.4426950408889634f;
  const int64_t units = (int64_t)L.max_tiles * nkv;
  const int grid = (int)((units + 7) / 8 * 8);
  if (q_dtype == MI_BF16)
    st = fp8 ? launch_prefill<BF16, true>(pp, D, grid, s) : launch_prefill<BF16, false>(pp, D, grid, s);
  else
    st = fp8 ? launch_prefill<F16, true>(pp, D, grid, s) : launch_prefill<F16, false>(pp, D, grid, s);
  if (st != MI_OK) return st;
  MI_CHECK_LAUNCH();
  return MI_OK;
}
