// Internal interfaces shared between the decode and prefill translation units.
#pragma once

#include "mi_common.h"

namespace mi {

// Workspace layout of a split-KV plan (decode kernel + merge).
struct SplitLayout {
  int64_t hdr, chunk_indptr, work, lse, opart, total;
  int32_t max_chunks;
};
// ws_avail: bytes the caller's workspace offers from the layout's start (-1:
// unbounded, giving the recommended size); the chunk budget shrinks to fit.
// pair: the plan is for paired kv-heads (see pair_heads); it only sets the
// chunk target, the buffers are sized for nkv heads of head_dim either way.
SplitLayout split_layout(int32_t batch, int32_t nkv, int32_t head_dim, int64_t ws_avail, bool pair = false);

// Decode over head_dim 128 with at most 8 query heads per kv-head reads two
// adjacent kv-heads as one 256-element row (512 contiguous bytes of a token
// row instead of 256): each query row takes the 128 elements of its own head
// and zeros in the other half, the score MFMAs accumulate the two halves in
// separate registers and each row keeps its own head's (so its scores see
// only its head, non-finite keys of the other head included), and it keeps
// only its half of the output.  Decided from the call's shapes alone, so a
// plan and the run that consumes it agree; decode calls only (no qo_indptr),
// and batches of at least kPairMinBatch requests, whose items are long enough
// for the one-workgroup-per-CU head_dim 256 kernel (c3, B=256: 542 -> 515 us;
// c2, B=64, min-chunk items: 57 -> 60 us).  The run uses the paired kernel
// for 16-bit caches only (fp8 pairs are 256-byte rows: c5 400 -> 410 us).
// A ragged batch (qo_indptr given) pairs only on the prefill path (`ragged`),
// where a request that does not fit a paired row block has somewhere else to
// go: there the short-query threshold halves (pair_short_rows) and the MFMA
// tiles take the requests between the two thresholds.
constexpr int32_t kPairMinBatch = 128;
inline bool pair_heads(const int32_t* qo_indptr, int32_t batch, int32_t num_kv_heads, int32_t group,
                       int32_t head_dim, bool ragged = false) {
  return (!qo_indptr || ragged) && batch >= kPairMinBatch && head_dim == 128 && num_kv_heads % 2 == 0 &&
         group >= 1 && 2 * group <= 16;
}
// Short-query requests of a ragged batch (qo_len * group <= this many rows)
// run on the split-KV decode kernels, longer ones on the MFMA prefill tiles.
// 16 rows (one MFMA column block); 8 for a paired plan, whose column block
// holds a request's rows of both heads of a pair.
constexpr int32_t kShortRowsMax = 16;
inline int32_t pair_short_rows(bool pair) { return pair ? kShortRowsMax / 2 : kShortRowsMax; }

int decode_plan_impl(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                     const int32_t* last_page_len, int32_t batch, int32_t page_size,
                     int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                     int64_t* kv_locations, void* workspace, int64_t workspace_bytes,
                     int64_t ws_offset, hipStream_t stream);

// Checks the arguments and fills the plan kernel's parameters (no launch).
struct PlanParams;
int decode_plan_params(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
                       const int32_t* last_page_len, int32_t batch, int32_t page_size,
                       int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                       int64_t* kv_locations, void* workspace, int64_t workspace_bytes,
                       int64_t ws_offset, PlanParams* out, bool ragged_pair = false);

enum : int { kPhaseAttend = 1, kPhaseMerge = 2 };

// The attention kernels move q / out rows and KV rows in 16-byte pieces: a
// tensor qualifies when its base is 16-byte aligned and each element stride
// spans a whole number of 16-byte pieces.
inline bool rows_aligned16(const void* base, int64_t stride_a, int64_t stride_b, int elem_bytes) {
  return ((uintptr_t)base & 15) == 0 && (stride_a * elem_bytes) % 16 == 0 && (stride_b * elem_bytes) % 16 == 0;
}
inline bool kv_aligned16(const mi_paged_kv* kv) {
  const int esz = kv->dtype == MI_FP8_E4M3 ? 1 : kv->dtype == MI_F32 ? 4 : 2;
  return rows_aligned16(kv->data, kv->page_stride, kv->kv_stride, esz) &&
         rows_aligned16(kv->data, kv->token_stride, kv->head_stride, esz);
}

// Arguments of the split-KV decode kernels (decode, merge, and their fp32
// variants): q/out rows, the KV layer, the packed batch and the plan in the
// workspace.
struct DecodeParams {
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
  const int4* work;
  const int32_t* chunk_indptr;
  float* lse_part;
  float* o_part;
  void* out;
  int64_t out_stride_tok, out_stride_head;
  int32_t num_kv_heads, group, page_size, causal;
  float scale_log2;
  int32_t short_rows = kShortRowsMax;  // ragged batches: requests with qo_len * group above this are not ours
};

// fp32 KV (q, cache and output in fp32): the attend phase of a split-KV plan
// (mi_f32.hip), and the merge with fp32 output (mi_decode.hip).
int f32_attend_launch(const DecodeParams& dp, int head_dim, int grid, hipStream_t stream);
int merge_launch(const DecodeParams& dp, int head_dim, int out_dtype, int batch, hipStream_t stream);
// fp32 ragged prefill over the prefill plan's tile list: one workgroup per
// (tile, kv-head, 16-row block).
int f32_prefill_launch(const DecodeParams& dp, const int32_t* tile_hdr, const int2* tiles, int max_tiles,
                       int tile_rows, int head_dim, hipStream_t stream);

int decode_run_impl(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                    const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                    const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                    int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                    int64_t workspace_bytes, int64_t ws_offset, void* out,
                    int64_t out_stride_token, int64_t out_stride_head, int phases, hipStream_t stream,
                    bool ragged_pair = false);

// Exclusive prefix sum over a 1024-thread block; `smem` holds >= 16 ints.
__device__ __forceinline__ int block_exclusive_scan_1024(int v, int& total, int* smem) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) smem[w] = x;
  __syncthreads();
  if (w == 0) {
    int t = lane < 16 ? smem[lane] : 0;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(t, o, 64);
      if (lane >= o) t += y;
    }
    if (lane < 16) smem[lane] = t;
  }
  __syncthreads();
  const int before = w ? smem[w - 1] : 0;
  total = smem[15];
  __syncthreads();
  return before + x - v;
}

// Sum and max of v over a 1024-thread workgroup, returned to every thread
// (smem: 16 ints, free again on return).
__device__ __forceinline__ int block_sum_1024(int v, int* smem) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) smem[w] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += smem[i];
  __syncthreads();
  return t;
}

__device__ __forceinline__ int block_max_1024(int v, int* smem) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  if (lane == 0) smem[w] = v;
  __syncthreads();
  int t = smem[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) t = max(t, smem[i]);
  __syncthreads();
  return t;
}

}  // namespace mi
