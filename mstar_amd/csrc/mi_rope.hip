// Rotary position embedding on the packed batch, and its position ids.
//
// mi_rope_positions replaces the position list of
// BatchedCacheManager._plan_rope_impl (mstar/engine/cache_manager.py:480-492):
//   pos[t] = position_id_start[r] + (t - qo_indptr[r]) for token t of request r.
// mi_rope_apply replaces the FlashInfer call of BatchedCacheManager.apply_rope
// (cache_manager.py:702-760: apply_rope_pos_ids_inplace /
// apply_llama31_rope_pos_ids_inplace): q [tokens, Hq, D] and k [tokens, Hkv, D]
// are rotated in place, dims [0, rotary_dim) in pairs (i, i + rotary_dim/2)
// or, interleaved, (2i, 2i+1); pair i turns by pos * f_i with
//   g_i = 1 / theta^(2i/rotary_dim),  f_i = g_i / rope_scale,
// or, with Llama-3.1 smoothing, f_i = (1 - s) g_i / rope_scale + s g_i,
//   s = clamp(g_i * smooth_a + smooth_b, 0, 1).
// All arithmetic is fp32 (fp32 angle pos * f_i, accurate sincosf); results
// are rounded to the tensor dtype (round to nearest even).
//
// One thread owns 4 consecutive pairs of one token for 4 heads: it computes
// the 4 (cos, sin) once, loads the 4 heads' elements together, then rotates
// and stores them, so the transcendental work is shared by 4 heads and every
// thread has independent loads in flight.
#include "mi_common.h"

namespace mi {

struct RopeParams {
  void* q;
  void* k;
  int64_t q_stride_tok, q_stride_head, k_stride_tok, k_stride_head;
  const void* pos;
  int32_t pos_is_64, num_tokens, num_qo_heads, num_kv_heads, rotary_dim, interleave, llama31;
  float theta, rope_scale, smooth_a, smooth_b;
};

constexpr int kRopeHeads = 4;  // heads per thread (one (cos, sin) set, independent loads)

template <typename MT>
MI_DEVICE void rot_pair(uint32_t& wa, uint32_t& wb, float c0, float s0, float c1, float s1) {
  // wa = (a0, a1), wb = (b0, b1): pairs (a_e, b_e) turn by angle e
  const float a0 = MT::to_f32((uint16_t)(wa & 0xffffu)), a1 = MT::to_f32((uint16_t)(wa >> 16));
  const float b0 = MT::to_f32((uint16_t)(wb & 0xffffu)), b1 = MT::to_f32((uint16_t)(wb >> 16));
  wa = MT::pack2(a0 * c0 - b0 * s0, a1 * c1 - b1 * s1);
  wb = MT::pack2(b0 * c0 + a0 * s0, b1 * c1 + a1 * s1);
}

// Interleaved pair (a, b) in one 32-bit word turns by one angle.
template <typename MT>
MI_DEVICE uint32_t rot_word(uint32_t w, float c, float s) {
  const float a = MT::to_f32((uint16_t)(w & 0xffffu)), b = MT::to_f32((uint16_t)(w >> 16));
  return MT::pack2(a * c - b * s, b * c + a * s);
}

// cos/sin of pairs i0 .. i0+3 of token t (fp32 angle pos * f_i).
MI_DEVICE void rope_cos_sin(const RopeParams& p, int64_t t, int i0, float (&c)[4], float (&s)[4]) {
  const float pos = p.pos_is_64 ? (float)((const int64_t*)p.pos)[t] : (float)((const int32_t*)p.pos)[t];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g = 1.0f / powf(p.theta, (float)(2 * (i0 + j)) / (float)p.rotary_dim);
    float f = g / p.rope_scale;
    if (p.llama31) {
      const float sm = fminf(fmaxf(g * p.smooth_a + p.smooth_b, 0.f), 1.f);
      f = (1.0f - sm) * f + sm * g;
    }
    sincosf(pos * f, &s[j], &c[j]);
  }
}

// One thread: 4 consecutive pairs of one token for kRopeHeads heads (q heads
// first, then k heads).  Consecutive threads take consecutive pair groups of
// the same heads, so a wavefront's accesses are contiguous runs of each row.
template <typename MT, bool INTERLEAVE>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  const int half = p.rotary_dim >> 1;
  const int groups = half >> 2;
  const int nh = p.num_qo_heads + p.num_kv_heads;
  const int chunks = (nh + kRopeHeads - 1) / kRopeHeads;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t t = gid / (groups * chunks);
  if (t >= p.num_tokens) return;
  const int rem = (int)(gid - t * groups * chunks);
  const int chunk = rem / groups, i0 = (rem - chunk * groups) * 4;
  float c[4], s[4];
  rope_cos_sin(p, t, i0, c, s);
  uint16_t* rows[kRopeHeads];
  bool live[kRopeHeads];
#pragma unroll
  for (int j = 0; j < kRopeHeads; ++j) {
    const int hh = chunk * kRopeHeads + j;
    live[j] = hh < nh;
    rows[j] = hh < p.num_qo_heads
                  ? (uint16_t*)p.q + t * p.q_stride_tok + (int64_t)hh * p.q_stride_head
                  : (uint16_t*)p.k + t * p.k_stride_tok + (int64_t)(hh - p.num_qo_heads) * p.k_stride_head;
  }
  if constexpr (INTERLEAVE) {  // pairs (2i, 2i+1): 8 consecutive elements
    uint4 u[kRopeHeads];
#pragma unroll
    for (int j = 0; j < kRopeHeads; ++j)
      if (live[j]) u[j] = *(const uint4*)(rows[j] + 2 * i0);
#pragma unroll
    for (int j = 0; j < kRopeHeads; ++j) {
      if (!live[j]) continue;
      uint32_t w[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = rot_word<MT>(w[e], c[e], s[e]);
      *(uint4*)(rows[j] + 2 * i0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {  // pairs (i, i + half)
    uint2 ua[kRopeHeads], ub[kRopeHeads];
#pragma unroll
    for (int j = 0; j < kRopeHeads; ++j)
      if (live[j]) {
        ua[j] = *(const uint2*)(rows[j] + i0);
        ub[j] = *(const uint2*)(rows[j] + half + i0);
      }
#pragma unroll
    for (int j = 0; j < kRopeHeads; ++j) {
      if (!live[j]) continue;
      rot_pair<MT>(ua[j].x, ub[j].x, c[0], s[0], c[1], s[1]);
      rot_pair<MT>(ua[j].y, ub[j].y, c[2], s[2], c[3], s[3]);
      *(uint2*)(rows[j] + i0) = ua[j];
      *(uint2*)(rows[j] + half + i0) = ub[j];
    }
  }
}

// ------------------------------------------------------------ RoPE + append
// mi_rope_append: the rotation above and the paged KV append in one pass.
// q is rotated in place; k is rotated (in place too when keep_k), and the
// rotated k together with v is written to its cache slot, converted exactly
// as the separate append kernel converts (copy, round-to-nearest-even, or
// e4m3fn(clamp(x / scale, +-448))).  Rotated values are rounded to the q/k
// dtype before the cache conversion, so the cache holds what
// rope-then-append writes, bit for bit.
struct RopeAppendParams {
  RopeParams r{};
  const void* v;
  int64_t v_stride_tok, v_stride_head;
  void* cache;
  int64_t page_stride, kv_stride, token_stride, head_stride, max_pages;
  const float* k_scale;
  const float* v_scale;
  const int64_t* page_idx;
  const int64_t* slot_idx;
  int64_t idx_stride;
  const int32_t* num_tokens_device;
  int32_t num_append, head_dim, page_size, keep_k;
};

// NW 32-bit words of MT elements (2 per word) -> cache elements at dst.
template <typename MT, int DST, int NW>
MI_DEVICE void cache_store(uint8_t* dst, const uint32_t* w, float inv_scale) {
  if constexpr (DST == MI_F32) {  // exact widening of the rounded q/k-dtype values
    float o[2 * NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      o[2 * i] = MT::to_f32((uint16_t)(w[i] & 0xffffu));
      o[2 * i + 1] = MT::to_f32((uint16_t)(w[i] >> 16));
    }
#pragma unroll
    for (int i = 0; i < NW / 2; ++i) ((float4*)dst)[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  } else if constexpr (DST == MT::kDtype) {
    if constexpr (NW == 2) *(uint2*)dst = make_uint2(w[0], w[1]);
    else *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
  } else if constexpr (DST == MI_FP8_E4M3) {
    uint32_t o[NW / 2] = {};
#pragma unroll
    for (int i = 0; i < 2 * NW; ++i) {
      float y = MT::to_f32((uint16_t)(w[i >> 1] >> (16 * (i & 1)))) * inv_scale;
      if (y == y) y = fminf(fmaxf(y, -448.f), 448.f);  // NaN stays NaN
      o[i >> 2] |= (uint32_t)f32_to_e4m3fn(y) << (8 * (i & 3));
    }
    if constexpr (NW == 2) *(uint32_t*)dst = o[0];
    else *(uint2*)dst = make_uint2(o[0], o[1]);
  } else {
    uint32_t o[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const float a = MT::to_f32((uint16_t)(w[i] & 0xffffu)), b = MT::to_f32((uint16_t)(w[i] >> 16));
      const uint32_t lo = DST == MI_BF16 ? f32_to_bf16_rne(a) : f32_to_f16_rne(a);
      const uint32_t hi = DST == MI_BF16 ? f32_to_bf16_rne(b) : f32_to_f16_rne(b);
      o[i] = lo | (hi << 16);
    }
    if constexpr (NW == 2) *(uint2*)dst = make_uint2(o[0], o[1]);
    else *(uint4*)dst = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One thread: one 8-element group g of one token for kRopeHeads q heads, or
// for one k or one v head (the cache conversion, fp8 above all, is the long
// part of a thread; one head each spreads it over more threads).  Groups g < rotary_dim/8 hold 4 pairs
// (elements 4g.. and rotary_dim/2 + 4g.., or 8g.. interleaved); the others,
// and every v group, are elements 8g .. 8g+7, copied unrotated.
template <typename MT, int DST, bool INTERLEAVE>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendParams a) {
  constexpr int ESZ = DST == MI_FP8_E4M3 ? 1 : DST == MI_F32 ? 4 : 2;
  const RopeParams& p = a.r;
  const int groups = a.head_dim >> 3, rgroups = p.rotary_dim >> 3, half = p.rotary_dim >> 1;
  const int hq = p.num_qo_heads, hkv = p.num_kv_heads;
  const int qchunks = (hq + kRopeHeads - 1) / kRopeHeads, chunks = qchunks + 2 * hkv;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t t = gid / (groups * chunks);
  if (t >= p.num_tokens) return;
  const int rem = (int)(gid - t * groups * chunks);
  const int chunk = rem / groups, g = rem - chunk * groups;
  const bool kvc = chunk >= qchunks;  // a k or v head: the one head hq + chunk - qchunks
  const int h0 = kvc ? hq + chunk - qchunks : chunk * kRopeHeads;
  const int hend = kvc ? h0 + 1 : min(h0 + kRopeHeads, hq);
  const bool rot = g < rgroups;
  // The token's cache row (K half, head 0), or null when it is not written.
  // (The index entries exist for t < num_append; the device count, read in
  // parallel, only trims that range.)
  uint8_t* crow = nullptr;
  if (t < a.num_append && kvc) {
    const bool real = !a.num_tokens_device || t < *a.num_tokens_device;
    const int64_t page = a.page_idx[t * a.idx_stride], slot = a.slot_idx[t * a.idx_stride];
    if (real && page >= 0 && page < a.max_pages && slot >= 0 && slot < a.page_size)
      crow = (uint8_t*)a.cache + (page * a.page_stride + slot * a.token_stride) * ESZ;
  }
  // Element offsets of the group's two 4-element halves within a row.
  const int e0 = rot && !INTERLEAVE ? 4 * g : 8 * g;
  const int e1 = rot && !INTERLEAVE ? half + 4 * g : 8 * g + 4;
  // Loads do not wait for the page lookup: k and v rows exist for every
  // token t < num_tokens, so only the cache stores depend on it.
  uint16_t* src[kRopeHeads];
  bool live[kRopeHeads];
#pragma unroll
  for (int j = 0; j < kRopeHeads; ++j) {
    const int hh = h0 + j;
    if (hh >= hend) {
      live[j] = false;
      src[j] = nullptr;
    } else if (hh < hq) {
      live[j] = rot;
      src[j] = (uint16_t*)p.q + t * p.q_stride_tok + (int64_t)hh * p.q_stride_head;
    } else if (hh < hq + hkv) {
      live[j] = true;
      src[j] = (uint16_t*)p.k + t * p.k_stride_tok + (int64_t)(hh - hq) * p.k_stride_head;
    } else {
      live[j] = true;
      src[j] = (uint16_t*)a.v + t * a.v_stride_tok + (int64_t)(hh - hq - hkv) * a.v_stride_head;
    }
  }
  // fp8 cache: the heads' reciprocal scales, loaded beside the rows (every
  // k and v head has a scale, whatever the page lookup finds).
  float isc[kRopeHeads];
#pragma unroll
  for (int j = 0; j < kRopeHeads; ++j) {
    const int hh = h0 + j;
    isc[j] = 1.f;
    if (DST == MI_FP8_E4M3 && hh >= hq && hh < hend)
      isc[j] = 1.0f / (hh < hq + hkv ? a.k_scale[hh - hq] : a.v_scale[hh - hq - hkv]);
  }
  float c[4] = {}, s[4] = {};
  if (rot && h0 < hq + hkv) rope_cos_sin(p, t, 4 * g, c, s);
  uint32_t w[kRopeHeads][4];
#pragma unroll
  for (int j = 0; j < kRopeHeads; ++j)
    if (live[j]) {
      if (h0 + j >= hq + hkv || !rot || INTERLEAVE) {
        const uint4 u = *(const uint4*)(src[j] + 8 * g);
        w[j][0] = u.x; w[j][1] = u.y; w[j][2] = u.z; w[j][3] = u.w;
      } else {
        const uint2 ua = *(const uint2*)(src[j] + e0), ub = *(const uint2*)(src[j] + e1);
        w[j][0] = ua.x; w[j][1] = ua.y; w[j][2] = ub.x; w[j][3] = ub.y;
      }
    }
#pragma unroll
  for (int j = 0; j < kRopeHeads; ++j) {
    if (!live[j]) continue;
    const int hh = h0 + j;
    if (hh >= hq + hkv) {  // v head: unrotated, 8 elements
      if (!crow) continue;
      const int vh = hh - hq - hkv;
      cache_store<MT, DST, 4>(crow + (a.kv_stride + vh * a.head_stride + 8 * g) * ESZ, w[j], isc[j]);
      continue;
    }
    const bool is_k = hh >= hq;
    if (rot) {
      if constexpr (INTERLEAVE) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[j][e] = rot_word<MT>(w[j][e], c[e], s[e]);
      } else {
        rot_pair<MT>(w[j][0], w[j][2], c[0], s[0], c[1], s[1]);
        rot_pair<MT>(w[j][1], w[j][3], c[2], s[2], c[3], s[3]);
      }
      if (!is_k || a.keep_k) {
        if (INTERLEAVE) {
          *(uint4*)(src[j] + e0) = make_uint4(w[j][0], w[j][1], w[j][2], w[j][3]);
        } else {
          *(uint2*)(src[j] + e0) = make_uint2(w[j][0], w[j][1]);
          *(uint2*)(src[j] + e1) = make_uint2(w[j][2], w[j][3]);
        }
      }
    }
    if (is_k && crow) {
      const int kh = hh - hq;
      uint8_t* row = crow + (int64_t)kh * a.head_stride * ESZ;
      cache_store<MT, DST, 2>(row + e0 * ESZ, w[j], isc[j]);
      cache_store<MT, DST, 2>(row + e1 * ESZ, w[j] + 2, isc[j]);
    }
  }
}

__global__ __launch_bounds__(256) void rope_positions_kernel(const int32_t* qo_indptr, const int32_t* start,
                                                             int32_t batch, int64_t* pos, int32_t n) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= n || batch <= 0) return;
  int lo = 0, hi = batch - 1;  // last request r with qo_indptr[r] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qo_indptr[mid] <= t) lo = mid; else hi = mid - 1;
  }
  pos[t] = (int64_t)start[lo] + (t - qo_indptr[lo]);
}

// Llama-3.1 blend s = clamp(g * smooth_a + smooth_b, 0, 1); false on bad factors.
static bool set_smoothing(RopeParams& p, int32_t llama31, float low, float high, float old_context_len) {
  p.llama31 = llama31 ? 1 : 0;
  p.smooth_a = 0.f;
  p.smooth_b = 0.f;
  if (!llama31) return true;
  if (!(high > low) || !(low > 0.f)) return false;
  const double two_pi = 6.283185307179586;
  p.smooth_a = (float)((double)old_context_len / (two_pi * ((double)high - low)));
  p.smooth_b = (float)(-(double)low / ((double)high - low));
  return true;
}

template <typename MT, int DST>
static void launch_rope_append(const RopeAppendParams& a, int grid, hipStream_t s) {
  if (a.r.interleave) hipLaunchKernelGGL((rope_append_kernel<MT, DST, true>), dim3(grid), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((rope_append_kernel<MT, DST, false>), dim3(grid), dim3(256), 0, s, a);
}

template <typename MT>
static int launch_rope_append_src(const RopeAppendParams& a, int dst, int grid, hipStream_t s) {
  switch (dst) {
    case MI_BF16: launch_rope_append<MT, MI_BF16>(a, grid, s); break;
    case MI_F16: launch_rope_append<MT, MI_F16>(a, grid, s); break;
    case MI_FP8_E4M3: launch_rope_append<MT, MI_FP8_E4M3>(a, grid, s); break;
    case MI_F32: launch_rope_append<MT, MI_F32>(a, grid, s); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

}  // namespace mi

extern "C" int mi_rope_positions(const int32_t* qo_indptr, const int32_t* position_id_start, int32_t batch,
                                 int64_t* pos_ids, int32_t num_tokens, void* stream) {
  using namespace mi;
  if (batch < 0 || num_tokens < 0) return MI_ERR_INVALID;
  if (num_tokens == 0) return MI_OK;
  if (batch == 0 || !qo_indptr || !position_id_start || !pos_ids) return MI_ERR_INVALID;
  hipLaunchKernelGGL(rope_positions_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     qo_indptr, position_id_start, batch, pos_ids, num_tokens);
  MI_CHECK_LAUNCH();
  return MI_OK;
}

extern "C" int mi_rope_apply(void* q, int64_t q_stride_token, int64_t q_stride_head, int32_t num_qo_heads, void* k,
                             int64_t k_stride_token, int64_t k_stride_head, int32_t num_kv_heads, int32_t dtype,
                             int32_t head_dim, int32_t rotary_dim, const void* pos_ids, int32_t pos_dtype,
                             int32_t num_tokens, int32_t interleave, float rope_scale, float rope_theta,
                             int32_t llama31, float low_freq_factor, float high_freq_factor,
                             float old_context_len, void* stream) {
  using namespace mi;
  if (num_tokens < 0 || num_qo_heads < 0 || num_kv_heads < 0) return MI_ERR_INVALID;
  if (num_tokens == 0 || num_qo_heads + num_kv_heads == 0) return MI_OK;
  if (!pos_ids || (num_qo_heads > 0 && !q) || (num_kv_heads > 0 && !k)) return MI_ERR_INVALID;
  if (dtype != MI_BF16 && dtype != MI_F16) return MI_ERR_UNSUPPORTED;
  if (pos_dtype != MI_I32 && pos_dtype != MI_I64) return MI_ERR_UNSUPPORTED;
  if (rotary_dim <= 0 || rotary_dim > head_dim || rotary_dim % 8 || head_dim % 8) return MI_ERR_UNSUPPORTED;
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f)) return MI_ERR_INVALID;
  // 8-byte (half split) / 16-byte (interleaved) element groups
  const int64_t align = interleave ? 8 : 4;
  if ((num_qo_heads > 0 && ((uintptr_t)q % (2 * align) || q_stride_token % align || q_stride_head % align)) ||
      (num_kv_heads > 0 && ((uintptr_t)k % (2 * align) || k_stride_token % align || k_stride_head % align)))
    return MI_ERR_INVALID;
  RopeParams p{};
  p.q = q;
  p.k = k;
  p.q_stride_tok = q_stride_token;
  p.q_stride_head = q_stride_head;
  p.k_stride_tok = k_stride_token;
  p.k_stride_head = k_stride_head;
  p.pos = pos_ids;
  p.pos_is_64 = pos_dtype == MI_I64;
  p.num_tokens = num_tokens;
  p.num_qo_heads = num_qo_heads;
  p.num_kv_heads = num_kv_heads;
  p.rotary_dim = rotary_dim;
  p.interleave = interleave ? 1 : 0;
  p.theta = rope_theta;
  p.rope_scale = rope_scale;
  if (!set_smoothing(p, llama31, low_freq_factor, high_freq_factor, old_context_len)) return MI_ERR_INVALID;
  const int64_t chunks = (num_qo_heads + num_kv_heads + kRopeHeads - 1) / kRopeHeads;
  const int64_t threads = (int64_t)num_tokens * (rotary_dim / 8) * chunks;
  const int grid = (int)((threads + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MI_BF16) {
    if (interleave) hipLaunchKernelGGL((rope_kernel<BF16, true>), dim3(grid), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((rope_kernel<BF16, false>), dim3(grid), dim3(256), 0, s, p);
  } else {
    if (interleave) hipLaunchKernelGGL((rope_kernel<F16, true>), dim3(grid), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((rope_kernel<F16, false>), dim3(grid), dim3(256), 0, s, p);
  }
  MI_CHECK_LAUNCH();
  return MI_OK;
}

extern "C" int mi_rope_append(void* q, int64_t q_stride_token, int64_t q_stride_head, int32_t num_qo_heads, void* k,
                              int64_t k_stride_token, int64_t k_stride_head, const void* v, int64_t v_stride_token,
                              int64_t v_stride_head, int32_t dtype, int32_t keep_k, const mi_paged_kv* kv,
                              const int64_t* page_idx, const int64_t* slot_idx, int64_t idx_stride,
                              int32_t num_append_tokens, const int32_t* num_tokens_device, int32_t rotary_dim, const void* pos_ids,
                              int32_t pos_dtype, int32_t num_tokens, int32_t interleave, float rope_scale,
                              float rope_theta, int32_t llama31, float low_freq_factor, float high_freq_factor,
                              float old_context_len, void* stream) {
  using namespace mi;
  if (!kv || num_tokens < 0 || num_append_tokens < 0 || num_qo_heads < 0) return MI_ERR_INVALID;
  if (num_tokens == 0) return MI_OK;
  if (!kv->data || !k || !v || !pos_ids || !page_idx || !slot_idx || idx_stride <= 0) return MI_ERR_INVALID;
  if (num_qo_heads > 0 && !q) return MI_ERR_INVALID;
  const int hkv = kv->num_kv_heads, d = kv->head_dim;
  if (hkv <= 0 || d <= 0 || kv->page_size <= 0) return MI_ERR_INVALID;
  if (dtype != MI_BF16 && dtype != MI_F16) return MI_ERR_UNSUPPORTED;
  if (pos_dtype != MI_I32 && pos_dtype != MI_I64) return MI_ERR_UNSUPPORTED;
  if (rotary_dim <= 0 || rotary_dim > d || rotary_dim % 8 || d % 8) return MI_ERR_UNSUPPORTED;
  const int dst = kv->dtype;
  if (dst != MI_BF16 && dst != MI_F16 && dst != MI_FP8_E4M3 && dst != MI_F32) return MI_ERR_UNSUPPORTED;
  if (dst == MI_FP8_E4M3 && (!kv->k_scale || !kv->v_scale)) return MI_ERR_INVALID;
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f)) return MI_ERR_INVALID;
  // q: 4-element groups (8 elements interleaved); k, v and cache rows: 8-element groups.
  const int64_t qalign = interleave ? 8 : 4;
  if (num_qo_heads > 0 && ((uintptr_t)q % (2 * qalign) || q_stride_token % qalign || q_stride_head % qalign))
    return MI_ERR_INVALID;
  if ((k_stride_token | k_stride_head | v_stride_token | v_stride_head) % 8) return MI_ERR_INVALID;
  if ((uintptr_t)k % 16 || (uintptr_t)v % 16) return MI_ERR_INVALID;
  const int desz = dst == MI_FP8_E4M3 ? 1 : dst == MI_F32 ? 4 : 2;
  if ((kv->page_stride | kv->kv_stride | kv->token_stride | kv->head_stride) % 8) return MI_ERR_INVALID;
  if ((uintptr_t)kv->data % (8 * desz)) return MI_ERR_INVALID;
  RopeAppendParams a{};
  RopeParams& p = a.r;
  p.q = q;
  p.k = k;
  p.q_stride_tok = q_stride_token;
  p.q_stride_head = q_stride_head;
  p.k_stride_tok = k_stride_token;
  p.k_stride_head = k_stride_head;
  p.pos = pos_ids;
  p.pos_is_64 = pos_dtype == MI_I64;
  p.num_tokens = num_tokens;
  p.num_qo_heads = num_qo_heads;
  p.num_kv_heads = hkv;
  p.rotary_dim = rotary_dim;
  p.interleave = interleave ? 1 : 0;
  p.theta = rope_theta;
  p.rope_scale = rope_scale;
  if (!set_smoothing(p, llama31, low_freq_factor, high_freq_factor, old_context_len)) return MI_ERR_INVALID;
  a.v = v;
  a.v_stride_tok = v_stride_token;
  a.v_stride_head = v_stride_head;
  a.cache = kv->data;
  a.page_stride = kv->page_stride;
  a.kv_stride = kv->kv_stride;
  a.token_stride = kv->token_stride;
  a.head_stride = kv->head_stride;
  a.max_pages = kv->max_pages;
  a.k_scale = kv->k_scale;
  a.v_scale = kv->v_scale;
  a.page_idx = page_idx;
  a.slot_idx = slot_idx;
  a.idx_stride = idx_stride;
  a.num_tokens_device = num_tokens_device;
  a.num_append = num_append_tokens;
  a.head_dim = d;
  a.page_size = kv->page_size;
  a.keep_k = keep_k ? 1 : 0;
  const int64_t chunks = (num_qo_heads + kRopeHeads - 1) / kRopeHeads + 2 * hkv;
  const int64_t threads = (int64_t)num_tokens * chunks * (d / 8);
  if ((threads + 255) / 256 > INT32_MAX) return MI_ERR_INVALID;
  const int grid = (int)((threads + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  const int st = dtype == MI_BF16 ? launch_rope_append_src<BF16>(a, dst, grid, s)
                                  : launch_rope_append_src<F16>(a, dst, grid, s);
  if (st != MI_OK) return st;
  MI_CHECK_LAUNCH();
  return MI_OK;
}
