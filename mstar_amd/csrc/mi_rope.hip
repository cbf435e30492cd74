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
  const float pos = p.pos_is_64 ? (float)((const int64_t*)p.pos)[t] : (float)((const int32_t*)p.pos)[t];
  float c[4], s[4];
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
      for (int e = 0; e < 4; ++e) {
        const float a = MT::to_f32((uint16_t)(w[e] & 0xffffu)), b = MT::to_f32((uint16_t)(w[e] >> 16));
        w[e] = MT::pack2(a * c[e] - b * s[e], b * c[e] + a * s[e]);
      }
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
  RopeParams p;
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
  p.llama31 = llama31 ? 1 : 0;
  p.smooth_a = 0.f;
  p.smooth_b = 0.f;
  if (llama31) {
    if (!(high_freq_factor > low_freq_factor) || !(low_freq_factor > 0.f)) return MI_ERR_INVALID;
    const double two_pi = 6.283185307179586;
    p.smooth_a = (float)((double)old_context_len / (two_pi * ((double)high_freq_factor - low_freq_factor)));
    p.smooth_b = (float)(-(double)low_freq_factor / ((double)high_freq_factor - low_freq_factor));
  }
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
