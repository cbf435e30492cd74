// The persistent ragged prefill kernel (prefill_kernel, head_dim 64 and 128)
// and its parameters, shared by mi_prefill.hip (plan, launch, head_dim 64),
// mi_prefill_d128.hip (the head_dim 128 instantiations, compiled with their
// own scheduler setting) and mi_prefill_rs.h (the head_dim 256 kernel).  The
// kernels' description heads mi_prefill.hip.
#pragma once

#include "mi_common.h"
#include "mi_internal.h"
#include "mi_plan.h"

namespace mi {


// Eight wavefronts per prefill workgroup (two per SIMD).  Up to head_dim 128
// (prefill_kernel) each wavefront owns two 16-row groups: 256-row tiles.  At
// head_dim 256 (prefill_rs_kernel, mi_prefill_rs.h) a pair of wavefronts owns
// two 16-row groups, split by role: 128-row tiles.
constexpr int pf_waves(int) { return 8; }
constexpr int pf_rg(int head_dim) { return head_dim > 128 ? 1 : 2; }  // 16-row groups per wavefront (per pair at 256)
constexpr int pf_rows(int head_dim) { return 16 * pf_rg(head_dim) * pf_waves(head_dim); }  // (token, q-head) rows per workgroup
constexpr int kPfKeys = 32;                // keys per K/V tile
constexpr int kPfTileCap = 1024;           // tiles whose row-group addresses are staged in LDS at a time
constexpr int kCtrStride = 32;  // one 128-byte line per XCD counter

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
  static_assert(D <= 128, "head_dim 256 runs prefill_rs_kernel");
  using C = PrefillCfg<MT, FP8, D>;
  constexpr int KS = D / 32, VW = D / 16, KEYS = C::KEYS, RSK = C::RSK, RSV = C::RSV, ESZ = C::ESZ, CPR = C::CPR;
  constexpr int THREADS = C::THREADS, NL = C::NL, HALF = C::HALF, STAGE = C::STAGE;
  constexpr int RG = pf_rg(D), WROWS = 16 * RG;  // 16-row groups and rows per wavefront
  constexpr int LCH = FP8 ? 32 : 16;  // LDS bytes per loaded chunk
  constexpr float kNegInf = -__builtin_inff();
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * STAGE];
  // byte offset (from the head's base) of the first row of each 16-row group of the staged tiles
  __shared__ int64_t lds_toff[2 * kPfTileCap];

  __shared__ int s_unit;
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
  const int64_t page_bytes = p.page_stride * ESZ;
  int c0 = 0;  // first tile of the tile addresses staged in LDS
  // NB register buffers: tile X is loaded into buffer (X - t0) % NB, NB steps
  // before the step that stores it to LDS.  Two: with three (loads one step
  // further ahead) the c4 batch ran 1.5-2.5% slower at head_dim 128 (225 vs
  // 217 VGPRs).  The step loop is unrolled over lcm(3 LDS stages, NB) steps.
  constexpr int NB = 2;
  constexpr int UNR = 6;
  uint4 rr[NB][NL];
  // A tile's loads in two parts: the row-group addresses (LDS reads of the
  // table staged per unit) and the global loads, so a step can read the
  // addresses early and issue the loads later with no address arithmetic
  // beyond one add.
  auto tile_pages = [&](int t, int64_t (&pg)[NL]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) pg[i] = lds_toff[2 * (t - c0) + (l_grp[i] >> 4)];
  };
  auto load_tile_at = [&](const int64_t (&pg)[NL], uint4 (&r)[NL]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (2 * HALF % THREADS == 0 || tid + i * THREADS < 2 * HALF) {
        const uint8_t* base = kvb + uniform64(pg[i]);
        r[i] = *(const uint4*)(base + l_off[i]);
      }
    }
  };
  auto load_tile = [&](int t, uint4 (&r)[NL]) {
    int64_t pg[NL];
    tile_pages(t, pg);
    load_tile_at(pg, r);
  };
  // TAIL: the tile may reach past kv_len (only the request's last tile can),
  // so its V rows past the end are overwritten with zeros
  auto store_tile_impl = [&](int t, const uint4 (&r)[NL], int stage, auto tail) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * THREADS;
      if (2 * HALF % THREADS == 0 || c < 2 * HALF) {
        const int half = c / HALF, rem = c - half * HALF;
        const int row = rem / CPR, ch = rem - row * CPR;
        const uint4 v = r[i];
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
        // V rows past the KV end may hold anything (unwritten slots of the last page)
        if constexpr (decltype(tail)::value) {
          if (l_v[i] && t * KEYS + l_row[i] >= kv_len) {
            *(uint4*)dst = make_uint4(0, 0, 0, 0);
            if constexpr (FP8) *(uint4*)(dst + 16) = make_uint4(0, 0, 0, 0);
          }
        }
      }
    }
  };
  // Tiles before the request's last one hold no row past kv_len (kv_end <=
  // kv_len): their stores skip the tail test, chosen by a wave-uniform branch.
  auto store_tile = [&](int t, const uint4 (&r)[NL], int stage) {
    if (t * KEYS + KEYS > kv_len)
      store_tile_impl(t, r, stage, std::true_type{});
    else
      store_tile_impl(t, r, stage, std::false_type{});
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
  float moff[RG];  // -m_run * sl2 (0 while m_run is -inf): the exponent offset, changed only with m_run
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    m_run[rg] = kNegInf;
    l_run[rg] = 0.f;
    thr[rg] = kNegInf;
    moff[rg] = 0.f;
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
    // K fragment reads KLA slices ahead of the MFMAs that use them: at head_dim
    // 128 three of the four (c4 tiles 534-561 -> 522-554 us against one slice
    // ahead, 550-556 with all four first), at head_dim 64 one of the two.
    constexpr int KLA = KS >= 4 ? 3 : 1;
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * KLA, 0);
#pragma unroll
    for (int st = KLA; st < KS; ++st) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * RG, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * RG * KLA, 0);
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
          moff[rg] = mt == kNegInf ? 0.f : -mt * sl2;
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

      float pr[2][4];
#pragma unroll
      for (int js = 0; js < 2; ++js)
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[js][r] = fast_exp2(fmaf(s[rg][js][r], sl2, moff[rg]));
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
  };
  // Ping-pong: the two wavefronts that share a SIMD (one of waves {0,2,5,7},
  // one of {1,3,4,6}, for either round-robin or paired wave placement) put
  // their softmax on opposite sides of their MFMA work, so one's vector
  // work runs under the other's matrix work.  Group A finishes tile T-1's
  // softmax at the start of step T, group B finishes tile T's at its end.
  const bool grp_a = ((wave ^ (wave >> 2)) & 1) == 0;

  // ---- tile chunks (one for contexts up to kPfTileCap tiles).  Per chunk,
  // the byte offset of every tile's two 16-row key groups (page offset plus
  // slot offset; a group past the request's last page re-reads its last
  // group, masked and with V zeroed) is staged in LDS, so the step loop does
  // no page or slot arithmetic.  Loads past the last tile repeat the last
  // tile, so the steady loop has no conditional loads and the compiler's
  // vmcnt waits stay exact.
  for (c0 = 0; c0 * KEYS < kv_end; c0 += kPfTileCap) {
    const int t0 = c0;
    const int t1 = min(n_kt, c0 + kPfTileCap);
    __syncthreads();
    for (int e = tid; e < 2 * (t1 - t0); e += THREADS) {
      const int key = min((t0 + (e >> 1)) * KEYS + 16 * (e & 1), key_cap);
      const int pidx = (int)((unsigned)key / (unsigned)ps);
      const int slot = key - pidx * ps;
      lds_toff[e] = (int64_t)p.kv_indices[page_base + pidx] * page_bytes + (int64_t)slot * tok_bytes;
    }
    __syncthreads();
    const int tl = t1 - 1;
    // Three-stage LDS ring: in step T both groups read V of tile T-1 (P.V)
    // and K of tile T (scores), and tile T+1 is stored into the stage tile
    // T-2 used; the register buffer it came from then takes tile T+1+NB.
    const int n = t1 - t0;
#pragma unroll
    for (int u = 0; u < NB; ++u) load_tile(min(t0 + u, tl), rr[u]);
    store_tile(t0, rr[0], 0);
    load_tile(min(t0 + NB, tl), rr[0]);
    __syncthreads();
    f32x4 sc[RG][2];
    uint4 pbk[RG];
    uint4 va[VW];
    // step 0: scores and V^T fragments of tile t0; group B also its softmax
    qk(0, sc);
    vfrag(0, va);
    if (!grp_a) {
      sm_max(t0, sc);
      sm_exp(sc, pbk);
    }
    store_tile(min(t0 + 1, tl), rr[1], 1);
    load_tile(min(t0 + 1 + NB, tl), rr[1]);
    __syncthreads();
    // steps 1 .. n-1
    for (int i = 1; i < n; i += UNR) {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int ii = i + u;
        if (ii >= n) break;
        const int T = t0 + ii;
        // Tile T+1 goes into the stage tile T-2 used, which no wave reads in
        // this step; each group stores it (and issues the loads of tile T+1+NB)
        // in its vector half, under the other group's MFMA work.
        int64_t pg4[NL];
        tile_pages(min(T + 1 + NB, tl), pg4);
        // Each group's vector half runs at raised wave priority, so its softmax
        // issues ahead of the partner's MFMA stream on the shared SIMD
        // (c4 583 -> 580 us).
        if (grp_a) {
          __builtin_amdgcn_s_setprio(1);
          store_tile(min(T + 1, tl), rr[(u + 2) % NB], (u + 2) % 3);
          sm_max(T - 1, sc);
          sm_exp(sc, pbk);
          load_tile_at(pg4, rr[(u + 2) % NB]);
          __builtin_amdgcn_s_setprio(0);
        }
        // scores of tile T first (group B's softmax waits on them), then P.V of
        // tile T-1; V^T fragments of tile T replace those of T-1 after it
        qk((u + 1) % 3, sc);       // stage of tile T = ii % 3
        pv(va, pbk);               // tile T-1
        vfrag((u + 1) % 3, va);
        if (!grp_a) {
          __builtin_amdgcn_s_setprio(1);
          store_tile(min(T + 1, tl), rr[(u + 2) % NB], (u + 2) % 3);
          load_tile_at(pg4, rr[(u + 2) % NB]);
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
    pv(va, pbk);
  }

  // ---- epilogue: lane holds dims 16*jj + 4*grp + r of its row
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const float l_tot = rows4_sum(l_run[rg]);
    const float inv = l_tot > 0.f ? vscale / l_tot : (l_tot == 0.f ? 0.f : __builtin_nanf(""));  // NaN: row stays NaN
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

// head_dim 128 launches, defined in mi_prefill_d128.hip
int prefill_d128_launch(const PrefillParams& pp, bool f16, bool fp8, int grid, hipStream_t stream);

}  // namespace mi
