// Paged KV append (P5) for MI355X.
//
// Replaces the two torch index_put launches per layer of
// FlashInferPrefillWrapper.set_kv_cache / FlashInferDecodeWrapper.set_kv_cache
// (mstar/utils/flashinfer_utils.py:284-288, 480-484) with one kernel that
// writes K and V together.  One thread moves 8 consecutive head_dim
// elements of one (token, kv-head) for both K and V: 128-bit loads and
// stores for 16-bit caches, 64-bit stores for fp8.
//
// Conversions are bit-exact with torch's CPU casts:
//   bf16 -> bf16, f16 -> f16 : copy
//   any  -> bf16            : via fp32, round-to-nearest-even (NaN -> 0x7FC0)
//   any  -> f16             : via fp32, round-to-nearest-even
//   any  -> fp8 e4m3fn      : q = e4m3fn_RNE(clamp(x * (1/scale[h]), -448, 448))
//   f32 -> f32               : copy;  bf16/f16 -> f32 : exact widening
#include "mi_common.h"

namespace mi {

struct AppendParams {
  const void* k;
  const void* v;
  int64_t k_stride_tok, k_stride_head, v_stride_tok, v_stride_head;
  void* cache;
  int64_t page_stride, kv_stride, token_stride, head_stride, max_pages;
  const float* k_scale;
  const float* v_scale;
  const int64_t* page_idx;
  const int64_t* slot_idx;
  int64_t idx_stride;
  const int32_t* num_tokens_device;
  int32_t num_tokens, num_kv_heads, head_dim, page_size;
};

template <int SRC>
MI_DEVICE void load8(const void* base, int64_t off, float (&x)[8]) {
  if constexpr (SRC == MI_F32) {
    const float4 a = *(const float4*)((const float*)base + off);
    const float4 b = *(const float4*)((const float*)base + off + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const uint4 u = *(const uint4*)((const uint16_t*)base + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
      x[2 * i] = SRC == MI_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      x[2 * i + 1] = SRC == MI_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}

template <int SRC, int DST>
MI_DEVICE void move8(const void* src, int64_t soff, uint8_t* dst_row, float inv_scale) {
  if constexpr (SRC == DST && DST == MI_F32) {  // exact copy, bit patterns kept
    const uint4* s4 = (const uint4*)((const float*)src + soff);
    ((uint4*)dst_row)[0] = s4[0];
    ((uint4*)dst_row)[1] = s4[1];
  } else if constexpr (SRC == DST && DST != MI_FP8_E4M3) {
    *(uint4*)dst_row = *(const uint4*)((const uint16_t*)src + soff);  // exact copy
  } else if constexpr (DST == MI_F32) {  // 16-bit source widened exactly
    float x[8];
    load8<SRC>(src, soff, x);
    ((float4*)dst_row)[0] = make_float4(x[0], x[1], x[2], x[3]);
    ((float4*)dst_row)[1] = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    float x[8];
    load8<SRC>(src, soff, x);
    if constexpr (DST == MI_FP8_E4M3) {
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float y = x[i] * inv_scale;
        if (y == y) y = fminf(fmaxf(y, -448.f), 448.f);  // NaN stays NaN
        w[i >> 2] |= (uint32_t)f32_to_e4m3fn(y) << (8 * (i & 3));
      }
      *(uint2*)dst_row = make_uint2(w[0], w[1]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = DST == MI_BF16 ? f32_to_bf16_rne(x[2 * i]) : f32_to_f16_rne(x[2 * i]);
        const uint32_t hi = DST == MI_BF16 ? f32_to_bf16_rne(x[2 * i + 1]) : f32_to_f16_rne(x[2 * i + 1]);
        w[i] = lo | (hi << 16);
      }
      *(uint4*)dst_row = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void append_kernel(AppendParams p) {
  constexpr int ESZ = DST == MI_FP8_E4M3 ? 1 : DST == MI_F32 ? 4 : 2;
  const int per_token = p.num_kv_heads * (p.head_dim >> 3);
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(gid / per_token);
  int n = p.num_tokens;
  if (p.num_tokens_device) n = min(n, *p.num_tokens_device);
  if (i >= n) return;
  const int rem = (int)(gid - (int64_t)i * per_token);
  const int hh = rem / (p.head_dim >> 3);
  const int d0 = (rem - hh * (p.head_dim >> 3)) << 3;
  const int64_t page = p.page_idx[(int64_t)i * p.idx_stride];
  const int64_t slot = p.slot_idx[(int64_t)i * p.idx_stride];
  if (page < 0 || page >= p.max_pages || slot < 0 || slot >= p.page_size) return;
  uint8_t* row = (uint8_t*)p.cache +
                 (page * p.page_stride + slot * p.token_stride + hh * p.head_stride + d0) * ESZ;
  float ik = 1.f, iv = 1.f;
  if constexpr (DST == MI_FP8_E4M3) {
    ik = 1.0f / p.k_scale[hh];
    iv = 1.0f / p.v_scale[hh];
  }
  move8<SRC, DST>(p.k, (int64_t)i * p.k_stride_tok + (int64_t)hh * p.k_stride_head + d0, row, ik);
  move8<SRC, DST>(p.v, (int64_t)i * p.v_stride_tok + (int64_t)hh * p.v_stride_head + d0,
                  row + p.kv_stride * ESZ, iv);
}

template <int SRC>
static int launch_append_src(const AppendParams& ap, int dst, int grid, hipStream_t stream) {
  switch (dst) {
    case MI_BF16: hipLaunchKernelGGL((append_kernel<SRC, MI_BF16>), dim3(grid), dim3(256), 0, stream, ap); break;
    case MI_F16: hipLaunchKernelGGL((append_kernel<SRC, MI_F16>), dim3(grid), dim3(256), 0, stream, ap); break;
    case MI_FP8_E4M3: hipLaunchKernelGGL((append_kernel<SRC, MI_FP8_E4M3>), dim3(grid), dim3(256), 0, stream, ap); break;
    case MI_F32: hipLaunchKernelGGL((append_kernel<SRC, MI_F32>), dim3(grid), dim3(256), 0, stream, ap); break;
    default: return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

static bool aligned(const void* ptr, int bytes) { return ((uintptr_t)ptr % (uintptr_t)bytes) == 0; }

}  // namespace mi

extern "C" int mi_kv_append(const mi_paged_kv* kv, const void* k, const void* v, int32_t src_dtype,
                            int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_token,
                            int64_t v_stride_head, const int64_t* page_idx, const int64_t* slot_idx,
                            int64_t idx_stride, int32_t num_tokens, const int32_t* num_tokens_device,
                            void* stream) {
  using namespace mi;
  if (!kv || num_tokens < 0) return MI_ERR_INVALID;
  if (num_tokens == 0) return MI_OK;
  if (!kv->data || !k || !v || !page_idx || !slot_idx || idx_stride <= 0) return MI_ERR_INVALID;
  if (kv->num_kv_heads <= 0 || kv->head_dim <= 0 || kv->page_size <= 0) return MI_ERR_INVALID;
  if (kv->head_dim % 8) return MI_ERR_UNSUPPORTED;
  const int dst = kv->dtype;
  if (dst != MI_BF16 && dst != MI_F16 && dst != MI_FP8_E4M3 && dst != MI_F32) return MI_ERR_UNSUPPORTED;
  if (src_dtype != MI_BF16 && src_dtype != MI_F16 && src_dtype != MI_F32) return MI_ERR_UNSUPPORTED;
  if (dst == MI_FP8_E4M3 && (!kv->k_scale || !kv->v_scale)) return MI_ERR_INVALID;
  // 8-element vector moves need 8-element aligned rows on both sides.
  const int sesz = src_dtype == MI_F32 ? 4 : 2, desz = dst == MI_FP8_E4M3 ? 1 : dst == MI_F32 ? 4 : 2;
  if ((k_stride_token | k_stride_head | v_stride_token | v_stride_head) % 8) return MI_ERR_INVALID;
  if ((kv->page_stride | kv->kv_stride | kv->token_stride | kv->head_stride) % 8) return MI_ERR_INVALID;
  if (!aligned(k, 8 * sesz) || !aligned(v, 8 * sesz) || !aligned(kv->data, 8 * desz)) return MI_ERR_INVALID;
  AppendParams ap{};
  ap.k = k;
  ap.v = v;
  ap.k_stride_tok = k_stride_token;
  ap.k_stride_head = k_stride_head;
  ap.v_stride_tok = v_stride_token;
  ap.v_stride_head = v_stride_head;
  ap.cache = kv->data;
  ap.page_stride = kv->page_stride;
  ap.kv_stride = kv->kv_stride;
  ap.token_stride = kv->token_stride;
  ap.head_stride = kv->head_stride;
  ap.max_pages = kv->max_pages;
  ap.k_scale = kv->k_scale;
  ap.v_scale = kv->v_scale;
  ap.page_idx = page_idx;
  ap.slot_idx = slot_idx;
  ap.idx_stride = idx_stride;
  ap.num_tokens_device = num_tokens_device;
  ap.num_tokens = num_tokens;
  ap.num_kv_heads = kv->num_kv_heads;
  ap.head_dim = kv->head_dim;
  ap.page_size = kv->page_size;
  const int64_t threads = (int64_t)num_tokens * kv->num_kv_heads * (kv->head_dim / 8);
  const int grid = (int)((threads + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  int st;
  switch (src_dtype) {
    case MI_BF16: st = launch_append_src<MI_BF16>(ap, dst, grid, s); break;
    case MI_F16: st = launch_append_src<MI_F16>(ap, dst, grid, s); break;
    default: st = launch_append_src<MI_F32>(ap, dst, grid, s); break;
  }
  if (st != MI_OK) return st;
  MI_CHECK_LAUNCH();
  return MI_OK;
}
