// Role-split ragged prefill (prefill_rs_kernel), the head_dim 256 kernel.
//
// Same units as prefill_kernel (128-row tiles of one request and kv-head at
// head_dim 256, the plan's per-XCD queues) and page-offset table, but the 8
// wavefronts form 4 pairs, each pair owning PROWS rows (RGP 16-row groups: 32
// rows at head_dim 256), and the two wavefronts of a pair split the work by
// role:
//   S-role (waves 0, 2, 5, 7): S^T = K.Q^T for the pair's rows, the online
//     softmax and the probabilities P(T) of tile T, written to LDS (2 KB per
//     pair at head_dim 256) together with each row's rescale factor;
//   O-role (waves 1, 3, 4, 6): one step behind, O^T += V^T.P^T(T-1) over all
//     dims of the pair's rows, and the rows' probability sums (the 128
//     accumulator registers hold what an S-role wavefront holds as Q).
// Every K and V^T fragment read from LDS then feeds RGP MFMAs, where 16 rows
// per wavefront read each fragment for one: at head_dim 256 those fragment
// reads, not the MFMAs, set the step time.  Each SIMD holds one wavefront of
// each role for round-robin (SIMD = wave % 4) and paired (SIMD = wave / 2)
// placement alike, so the S-role softmax runs under the O-role MFMAs.
// Tiles of a 16-bit cache go from memory straight into LDS (global_load_lds,
// 16 bytes per lane, issued at the end of step T for tile T+2): the tile bytes
// then pass through no registers and no ds_write, which had cost ~16% of the
// kernel's cycles.  fp8 tiles are widened in registers on the way, as in
// prefill_kernel.  The fp8 path also builds at head_dim 128 (pairs of 64 rows,
// four row groups), which measured slower than prefill_kernel there and is not
// launched.
#pragma once

#include "mi_prefill_kernel.h"

namespace mi {

template <typename MT, bool FP8, int D>
__global__ __launch_bounds__(512) void prefill_rs_kernel(PrefillParams p) {
  using C = PrefillCfg<MT, FP8, D>;
  // 16-row groups per pair: the O-role's accumulators (RGP x D/16 f32x4) fill
  // 128 registers at either head_dim; C::ROWS = 4 pairs x 16 x RGP
  constexpr int RGP = D > 128 ? 2 : 4, PROWS = 16 * RGP;
  static_assert(C::ROWS == 4 * PROWS, "tile rows = four pairs");
  constexpr int KS = D / 32, VW = D / 16, KEYS = C::KEYS, RSK = C::RSK, RSV = C::RSV, ESZ = C::ESZ, CPR = C::CPR;
  constexpr int THREADS = C::THREADS, NL = C::NL, HALF = C::HALF;
  constexpr int LCH = FP8 ? 32 : 16;  // LDS bytes per loaded chunk
  constexpr float kNegInf = -__builtin_inff();
  static_assert(THREADS == 512, "four wavefront pairs");
  static_assert(RSK == RSV, "one LDS row stride for K and V");
  // 16-bit caches: direct loads into 4-stage K and V rings of unpadded rows
  // whose 16-byte chunks are XOR-swizzled (K: chunk ^ (row & 15); V: 32-byte
  // segment ^ (row & 7)), so the fragment reads stay free of bank conflicts;
  // the page-offset table holds half as many tiles to leave LDS for the rings.
  // fp8 caches: a 3-stage ring of padded rows, stored from registers.
  constexpr bool DMA = !FP8;
  constexpr int RS = DMA ? D * 2 : RSK;  // LDS row stride
  constexpr int KSZ = KEYS * RS, VSZ = KEYS * RS, NKS = DMA ? 4 : 3, NVS = DMA ? 4 : 3, VOFF = NKS * KSZ;
  constexpr int CAP = DMA ? kPfTileCap / 2 : kPfTileCap;  // tiles whose page offsets are staged at a time
  static_assert(!DMA || (KEYS == 32 && D * 2 == 512 && THREADS == 512), "direct loads: 4 per thread and tile");
  __shared__ __attribute__((aligned(16))) uint8_t lds[NKS * KSZ + NVS * VSZ];
  __shared__ int64_t lds_toff[2 * CAP];
  // probabilities of the step (B operand layout: per pair, row group and lane
  // one uint4) and each row's rescale factor, double-buffered by step parity
  __shared__ uint4 lds_p[2][4][RGP][64];
  __shared__ float lds_alpha[2][4][RGP][64];
  __shared__ int s_unit;

  const int n_tiles = p.hdr[0];
  const int xcd = (int)blockIdx.x & 7;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const bool role_s = ((wave ^ (wave >> 2)) & 1) == 0;
  const int pr = wave >> 1;  // pair: rows PROWS*pr .. PROWS*(pr+1)-1 of the tile
  const int ps = p.page_size, G = p.group;

  // Each role runs its own copy of the unit loop (the role is a compile-time
  // constant there), so a wavefront's registers hold only its role's state:
  // the S-role's Q fragments or the O-role's accumulators.  Both copies pass
  // the same sequence of workgroup barriers.
  auto run = [&](auto role) {
    constexpr bool S = decltype(role)::value;
    for (;;) {
      if (tid == 0) {
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
      const int2 te = p.tiles[unit - h * n_tiles];
      const int b = te.x, row0 = te.y;
      const int qo_start = p.qo_indptr[b];
      const int qo_len = p.qo_indptr[b + 1] - qo_start;
      const int page_base = p.kv_indptr[b];
      const int np = p.kv_indptr[b + 1] - page_base;
      const int kv_len = (np - 1) * ps + p.last_page_len[b];
      const int rows_total = qo_len * G;

      // R: the S-role's Q fragments (R[rg][s] for s < KS), the O-role's accumulators
      f32x4 R[RGP][VW];
      int lim[RGP];
#pragma unroll
      for (int rg = 0; rg < RGP; ++rg) {
        const int n = row0 + PROWS * pr + 16 * rg + col;
        const int tok = n / G, g = n - tok * G;
        const int l = p.causal ? (kv_len - qo_len + tok) : (kv_len - 1);
        lim[rg] = min(l, kv_len - 1);
        if constexpr (S) {
          const bool valid = n < rows_total;
          const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(qo_start + tok) * p.q_stride_tok +
                                 (int64_t)(h * G + g) * p.q_stride_head;
#pragma unroll
          for (int s = 0; s < KS; ++s)
            R[rg][s] = bitcast<f32x4>(valid ? *(const uint4*)(qrow + 32 * s + 8 * grp) : make_uint4(0, 0, 0, 0));
        } else {
#pragma unroll
          for (int jj = 0; jj < VW; ++jj) R[rg][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
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

      // ---- loader (as prefill_kernel): chunk c = tid + i*THREADS -> (half, row, 16-byte column)
      const uint8_t* kvb = (const uint8_t*)p.kv + (int64_t)h * p.head_stride * ESZ;
      const int64_t tok_bytes = p.token_stride * ESZ;
      uint32_t l_off[NL];
      int l_grp[NL];
      int l_row[NL];
      bool l_v[NL];
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
      const int key_cap = np * ps - 16;
      const int64_t page_bytes = p.page_stride * ESZ;
      int c0 = 0;
      constexpr int NB = 2;
      constexpr int UNR = 6;
      uint4 rr[NB][NL];
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
      auto store_tile_impl = [&](int t, const uint4 (&r)[NL], int stage, auto tail) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          const int c = tid + i * THREADS;
          if (2 * HALF % THREADS == 0 || c < 2 * HALF) {
            const int half = c / HALF, rem = c - half * HALF;
            const int row = rem / CPR, ch = rem - row * CPR;
            const uint4 v = r[i];
            uint8_t* dst = lds + (half ? VOFF + stage * VSZ : stage * KSZ) + row * RS + LCH * ch;
            if constexpr (FP8) {
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
            if constexpr (decltype(tail)::value) {
              if (l_v[i] && t * KEYS + l_row[i] >= kv_len) {
                *(uint4*)dst = make_uint4(0, 0, 0, 0);
                if constexpr (FP8) *(uint4*)(dst + 16) = make_uint4(0, 0, 0, 0);
              }
            }
          }
        }
      };
      auto store_tile = [&](int t, const uint4 (&r)[NL], int stage) {
        if (t * KEYS + KEYS > kv_len)
          store_tile_impl(t, r, stage, std::true_type{});
        else
          store_tile_impl(t, r, stage, std::false_type{});
      };
      // Direct loads: load i of wave w fills rows 2*rp, 2*rp+1 (rp = 8*(i&1) + w,
      // both in 16-row group i&1) of the tile's K (i < 2) or V (i >= 2) half;
      // lane l writes LDS chunk l%32 of row 2*rp + l/32 with the cached chunk
      // the swizzle puts there.
      uint32_t d_off[4];
      if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int hv = i >> 1, rp = 8 * (i & 1) + wave, r = 2 * rp + (lane >> 5), pch = lane & 31;
          const int c = hv ? (pch ^ (2 * (r & 7))) : (pch ^ (r & 15));
          d_off[i] = (uint32_t)((int64_t)hv * p.kv_stride * ESZ + (int64_t)(r & 15) * tok_bytes + 16 * c);
        }
      }
      const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
      // The load's LDS address is M0 (one s_nop after writing it, as the ISA
      // requires before an LDS-DMA load).  hipcc warns that m0 is a reserved
      // register on the clobber list: the compiler emits no M0 use of its own
      // in this kernel (no LDS-DMA builtin, s_sendmsg, movrel or interpolation),
      // so nothing of its lives in M0 across these statements.
      auto dma_tile = [&](int t, int kst, int vst) {
        // both 16-row groups' page offsets first, then the four loads (scalar
        // base + 32-bit lane offset)
        const uint8_t* gb[2] = {kvb + uniform64(lds_toff[2 * (t - c0)]), kvb + uniform64(lds_toff[2 * (t - c0) + 1])};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rp = 8 * (i & 1) + wave;
          const uint32_t m0 = lds_base + (i >= 2 ? VOFF + vst * VSZ : kst * KSZ) + rp * 1024;
          asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(d_off[i]), "s"(gb[i & 1])
                       : "memory", "m0");
        }
      };
      // End of a step: this wave's loads of K of the next tile and of V of the
      // current one have landed (`newer` loads may stay in flight: 6 = V of the
      // next tile and both halves of the one after it), and V rows of tile t
      // past kv_len are zeroed.
      auto dma_wait = [&](int t, int vst, int newer) {
        if (newer == 6)
          asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else if (newer == 2)
          asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (t * KEYS + KEYS > kv_len) {
#pragma unroll
          for (int i = 2; i < 4; ++i) {
            const int rp = 8 * (i & 1) + wave;
            if (t * KEYS + 2 * rp + (lane >> 5) >= kv_len)
              *(uint4*)(lds + VOFF + vst * VSZ + rp * 1024 + 16 * lane) = make_uint4(0, 0, 0, 0);
          }
        }
      };

      // softmax state: the S-role's lazy running max (as prefill_kernel), the
      // O-role's row sums of the probabilities it accumulates
      constexpr float kLazy = 8.f;
      const float lazy_raw = kLazy / sl2;
      float m_run[RGP], l_run[RGP], thr[RGP], moff[RGP];
#pragma unroll
      for (int rg = 0; rg < RGP; ++rg) {
        m_run[rg] = kNegInf;
        l_run[rg] = 0.f;
        thr[rg] = kNegInf;
        moff[rg] = 0.f;
      }
      const int t_mask = mask_from > 0 ? mask_from / KEYS : 0;

      // swizzled K fragment offsets (direct-load rings): 32-dim slice s of key
      // row 16*js + col sits at kbo[s & 3] + 256*(s >> 2) + 8192*js
      uint32_t kbo[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) kbo[m] = col * 512 + 16 * (grp ^ (col & 3)) + 64 * (m ^ (col >> 2));
      // S-role: scores, softmax and probabilities of tile t (K in LDS stage
      // `stage`), published in the exchange buffers of parity t & 1.
      auto s_step = [&](int t, int stage) {
        const uint8_t* sk = lds + stage * KSZ;
        f32x4 s[RGP][2];
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg)
#pragma unroll
          for (int js = 0; js < 2; ++js) s[rg][js] = f32x4{0.f, 0.f, 0.f, 0.f};
        // K fragments in chunks of KC 32-dim slices (both 16-key halves), one
        // chunk read ahead of its MFMAs; the empty asm with a memory clobber
        // keeps the compiler from hoisting every read (64 registers).
        constexpr int KC = 2;
        uint4 ka[2][KC][2];
        auto kread = [&](int c, uint4 (&a)[KC][2]) {
#pragma unroll
          for (int k = 0; k < KC; ++k)
#pragma unroll
            for (int js = 0; js < 2; ++js)
              a[k][js] = DMA ? *(const uint4*)(sk + kbo[(KC * c + k) & 3] + 256 * ((KC * c + k) >> 2) + 8192 * js)
                             : *(const uint4*)(sk + (16 * js + col) * RS + (8 * grp + 32 * (KC * c + k)) * 2);
        };
        kread(0, ka[0]);
#pragma unroll
        for (int c = 0; c < KS / KC; ++c) {
          if (c + 1 < KS / KC) kread(c + 1, ka[(c + 1) & 1]);
          asm volatile("" ::: "memory");
#pragma unroll
          for (int k = 0; k < KC; ++k)
#pragma unroll
            for (int rg = 0; rg < RGP; ++rg)
#pragma unroll
              for (int js = 0; js < 2; ++js)
                s[rg][js] = MT::mma_16x16x32(ka[c & 1][k][js], bitcast<uint4>(R[rg][KC * c + k]), s[rg][js]);
        }
        const int kb = t * KEYS;
        if (t >= t_mask) {
#pragma unroll
          for (int rg = 0; rg < RGP; ++rg)
#pragma unroll
            for (int js = 0; js < 2; ++js)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (kb + 16 * js + 4 * grp + r > lim[rg]) s[rg][js][r] = kNegInf;
        }
        float ml[RGP], alpha[RGP];
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) alpha[rg] = 1.f;
        bool any_need = false;
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) {
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
          for (int rg = 0; rg < RGP; ++rg) {
            const float mt = rows4_max(ml[rg]);
            const bool grow = mt > thr[rg];
            alpha[rg] = grow ? fast_exp2((m_run[rg] - mt) * sl2) : 1.f;
            if (grow) {
              m_run[rg] = mt;
              thr[rg] = mt + lazy_raw;
              moff[rg] = mt == kNegInf ? 0.f : -mt * sl2;
            }
          }
        }
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) {
          float q[2][4];
#pragma unroll
          for (int js = 0; js < 2; ++js)
#pragma unroll
            for (int r = 0; r < 4; ++r) q[js][r] = fast_exp2(fmaf(s[rg][js][r], sl2, moff[rg]));
          const uint4 pb = make_uint4(MT::pack2(q[0][0], q[0][1]), MT::pack2(q[0][2], q[0][3]),
                                      MT::pack2(q[1][0], q[1][1]), MT::pack2(q[1][2], q[1][3]));
          lds_p[t & 1][pr][rg][lane] = pb;
          lds_alpha[t & 1][pr][rg][lane] = alpha[rg];
        }
      };
      // swizzled V^T fragment offsets (direct-load rings): 32-byte segment jj of
      // key row R sits at vbo[jj & 7] + 256*(jj >> 3)
      uint32_t vbo[8];
      {
        const int R = 4 * grp + ((lane & 15) >> 2);
#pragma unroll
        for (int m = 0; m < 8; ++m) vbo[m] = R * 512 + 8 * (lane & 3) + 32 * (m ^ (R & 7));
      }
      // O-role: O^T += V^T.P^T of tile t (V in LDS stage `stage`), after the
      // rescale the S-role found for that tile.
      auto o_step = [&](int t, int stage) {
        uint4 pb[RGP];
        float alpha[RGP];
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) {
          pb[rg] = lds_p[t & 1][pr][rg][lane];
          alpha[rg] = lds_alpha[t & 1][pr][rg][lane];
        }
        bool rescale = false;
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) rescale |= alpha[rg] != 1.f;
        if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
          for (int rg = 0; rg < RGP; ++rg)
#pragma unroll
            for (int jj = 0; jj < VW; ++jj) R[rg][jj] *= alpha[rg];
#pragma unroll
          for (int rg = 0; rg < RGP; ++rg) l_run[rg] *= alpha[rg];
        }
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg)
          l_run[rg] = MT::sum2(pb[rg].w, MT::sum2(pb[rg].z, MT::sum2(pb[rg].y, MT::sum2(pb[rg].x, l_run[rg]))));
        const uint8_t* vt = lds + VOFF + stage * VSZ;
        const uint8_t* vt0 = vt + (4 * grp + ((lane & 15) >> 2)) * RS + 8 * (lane & 3);
        // V^T fragments in chunks of VC output tiles, one chunk read ahead of
        // the MFMAs that use it: the empty asm with a memory clobber keeps the
        // compiler from hoisting every read (64 registers) above the MFMAs.
        constexpr int VC = 4;
        uint4 va[2][VC];
        auto vread = [&](int c, uint4 (&a)[VC]) {
#pragma unroll
          for (int k = 0; k < VC; ++k) {
            const int jj = VC * c + k;
            const uint8_t* a0p = DMA ? vt + vbo[jj & 7] + 256 * (jj >> 3) : vt0 + 32 * jj;
            const v4i16 x0 = ds_read_tr16(a0p);
            const v4i16 x1 = ds_read_tr16(a0p + 16 * RS);
            const uint2 a0 = bitcast<uint2>(x0), a1 = bitcast<uint2>(x1);
            a[k] = make_uint4(a0.x, a0.y, a1.x, a1.y);
          }
        };
        vread(0, va[0]);
#pragma unroll
        for (int c = 0; c < VW / VC; ++c) {
          if (c + 1 < VW / VC) vread(c + 1, va[(c + 1) & 1]);
          asm volatile("" ::: "memory");
#pragma unroll
          for (int k = 0; k < VC; ++k)
#pragma unroll
            for (int rg = 0; rg < RGP; ++rg)
              R[rg][VC * c + k] = MT::mma_16x16x32(va[c & 1][k], pb[rg], R[rg][VC * c + k]);
        }
      };

      // ---- tile chunks.  The S-role reads K of tile T, the O-role V of tile T-1.
      if constexpr (DMA) {
        // Step ii of a chunk: the S-role's scores of tile ii, the O-role's P.V
        // of tile ii-1, then every wave's direct loads of tile ii+2 (ring stage
        // (ii+2) % 4); before the barrier each wave's loads of K of tile ii+1
        // and V of tile ii have landed (and are visible to all after it).
        for (c0 = 0; c0 * KEYS < kv_end; c0 += CAP) {
          const int t0 = c0;
          const int t1 = min(n_kt, c0 + CAP);
          __syncthreads();
          for (int e = tid; e < 2 * (t1 - t0); e += THREADS) {
            const int key = min((t0 + (e >> 1)) * KEYS + 16 * (e & 1), key_cap);
            const int pidx = (int)((unsigned)key / (unsigned)ps);
            const int slot = key - pidx * ps;
            lds_toff[e] = (int64_t)p.kv_indices[page_base + pidx] * page_bytes + (int64_t)slot * tok_bytes;
          }
          __syncthreads();
          const int tl = t1 - 1;
          const int n = t1 - t0;
          // the compiler's own loads (Q fragments, metadata) complete here, so
          // it has no load of its own to wait for inside the step loop (a wait
          // there would also drain the direct loads in flight)
          __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
          dma_tile(t0, 0, 0);
          dma_tile(min(t0 + 1, tl), 1, 1);
          asm volatile("s_waitcnt vmcnt(6)" ::: "memory");  // K of tile t0
          __syncthreads();
          // step 0
          if (n >= 3) dma_tile(t0 + 2, 2, 2);
          if constexpr (S) s_step(t0, 0);
          dma_wait(t0, 0, n >= 3 ? 6 : (n >= 2 ? 2 : 0));
          __syncthreads();
          // steps 1 .. n-3 (each loads tile ii+2): ring stage of tile ii = ii % 4 = (u + 1) % 4
          for (int i = 1; i <= n - 3; i += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int ii = i + u;
              if (ii > n - 3) break;
              const int T = t0 + ii;
              if constexpr (S)
                s_step(T, (u + 1) & 3);
              else
                o_step(T - 1, u);
              dma_tile(T + 2, (u + 3) & 3, (u + 3) & 3);
              dma_wait(T, (u + 1) & 3, 6);
              __syncthreads();
            }
          }
          // the last two steps load nothing
          for (int ii = max(1, n - 2); ii < n; ++ii) {
            const int T = t0 + ii;
            if constexpr (S)
              s_step(T, ii & 3);
            else
              o_step(T - 1, (ii - 1) & 3);
            dma_wait(T, ii & 3, T + 1 <= tl ? 2 : 0);
            __syncthreads();
          }
          if constexpr (!S) o_step(tl, (n - 1) & 3);
        }
      } else {
        // as prefill_kernel: step T stores tile T+1 into the stage tile T-2 used
        // and loads tile T+1+NB into registers
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
          const int n = t1 - t0;
#pragma unroll
          for (int u = 0; u < NB; ++u) load_tile(min(t0 + u, tl), rr[u]);
          store_tile(t0, rr[0], 0);
          load_tile(min(t0 + NB, tl), rr[0]);
          __syncthreads();
          // step 0: scores of tile t0
          if constexpr (S) s_step(t0, 0);
          store_tile(min(t0 + 1, tl), rr[1 % NB], 1);
          load_tile(min(t0 + 1 + NB, tl), rr[1 % NB]);
          __syncthreads();
          for (int i = 1; i < n; i += UNR) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
              const int ii = i + u;
              if (ii >= n) break;
              const int T = t0 + ii;
              if constexpr (S) {
                s_step(T, (u + 1) % 3);  // stage of tile T = ii % 3
                store_tile(min(T + 1, tl), rr[(u + 2) % NB], (u + 2) % 3);
                load_tile(min(T + 1 + NB, tl), rr[(u + 2) % NB]);
              } else {
                store_tile(min(T + 1, tl), rr[(u + 2) % NB], (u + 2) % 3);
                load_tile(min(T + 1 + NB, tl), rr[(u + 2) % NB]);
                o_step(T - 1, u % 3);  // stage of tile T-1 = (ii-1) % 3
              }
              __syncthreads();
            }
          }
          // last step: P.V of tile t1-1
          if constexpr (!S) o_step(t1 - 1, (n - 1) % 3);
        }
      }

      // ---- epilogue: the S-role publishes its row sums, the O-role writes the rows
      if constexpr (!S) {
#pragma unroll
        for (int rg = 0; rg < RGP; ++rg) {
          const float l_tot = rows4_sum(l_run[rg]);
          const float inv = l_tot > 0.f ? vscale / l_tot : (l_tot == 0.f ? 0.f : __builtin_nanf(""));
          const int nrow = row0 + PROWS * pr + 16 * rg + col;
          if (nrow >= rows_total) continue;
          const int tok = nrow / G, g = nrow - tok * G;
          uint16_t* orow = (uint16_t*)p.out + (int64_t)(qo_start + tok) * p.out_stride_tok +
                           (int64_t)(h * G + g) * p.out_stride_head;
#pragma unroll
          for (int jj = 0; jj < VW; ++jj) {
            const f32x4 o = R[rg][jj];
            *(uint2*)(orow + 16 * jj + 4 * grp) =
                make_uint2(MT::pack2(o[0] * inv, o[1] * inv), MT::pack2(o[2] * inv, o[3] * inv));
          }
        }
      }
    }  // unit loop
  };
  if (role_s)
    run(std::true_type{});
  else
    run(std::false_type{});
  if (tid == 0) {
    __threadfence();
    if (atomicAdd(p.ctr + 8 * kCtrStride, 1) == (int)gridDim.x - 1) {
#pragma unroll
      for (int y = 0; y < 9; ++y) __hip_atomic_store(p.ctr + y * kCtrStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace mi
