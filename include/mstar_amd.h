/*
 * mstar_amd.h — C ABI of the MI355X (gfx950) ragged paged-attention library.
 *
 * This is the drop-in boundary for M*'s continuous-batch attention path:
 * per-step batch packing, paged KV-cache append and paged attention.  Every
 * entry point takes raw device pointers, explicit sizes and a hipStream_t
 * (passed as void*), launches asynchronously on that stream, allocates no
 * memory and returns an int status (MI_OK == 0, negative on error).  No C++
 * exception crosses this boundary.  Buffers belong to the caller: the KV
 * pool, the per-wrapper workspace, index tensors and outputs.
 *
 * Layout of one KV layer (M*'s "NHD" layout, kv_cache_engine.py:132-136):
 *   [max_pages, 2 (K,V), page_size, num_kv_heads, head_dim]
 * described by mi_paged_kv with explicit element strides.
 *
 * Threading: plan and run of different workspaces may run concurrently on
 * different streams.  Library-wide state: a per-device cache of the CU count
 * (written once per device on first use; it feeds the split-KV partition of
 * small decode jobs) and, for mi_decode_noalloc only, one static device
 * scratch array per GPU with its address cached per device (see that entry
 * point: calls that overlap on one GPU race there).  Everything else a call
 * uses comes in through its arguments.
 */
#ifndef MSTAR_AMD_H
#define MSTAR_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type codes */
#define MI_BF16 0
#define MI_F16 1
#define MI_F32 2
#define MI_FP8_E4M3 3 /* OCP e4m3fn (gfx950 native), max 448, per-head fp32 scales */
#define MI_I32 4       /* index / position dtypes */
#define MI_I64 5

/* status codes */
#define MI_OK 0
#define MI_ERR_INVALID (-1)     /* bad argument (null pointer, size, stride) */
#define MI_ERR_UNSUPPORTED (-2) /* valid but not implemented (dtype, head_dim, page_size) */
#define MI_ERR_WORKSPACE (-3)   /* workspace too small or not planned for this call */
#define MI_ERR_LAUNCH (-4)      /* HIP launch error */

#define MI_ABI_VERSION 4

/* One layer of the paged KV cache. Strides are in elements. */
typedef struct mi_paged_kv {
  void* data;           /* element (page 0, K, slot 0, head 0, dim 0) */
  int32_t dtype;        /* MI_BF16, MI_F16, MI_F32 or MI_FP8_E4M3 */
  int32_t page_size;    /* tokens per page */
  int32_t num_kv_heads;
  int32_t head_dim;     /* 64, 128 or 256 */
  int64_t max_pages;    /* pages in the pool; page ids outside [0, max_pages) are skipped by append */
  int64_t page_stride;  /* between consecutive pages */
  int64_t kv_stride;    /* from the K half of a page to its V half */
  int64_t token_stride; /* between slots of a page */
  int64_t head_stride;  /* between kv heads of a slot (head_dim elements must be contiguous) */
  const float* k_scale; /* MI_FP8_E4M3 only: [num_kv_heads] dequantisation scales, else NULL */
  const float* v_scale;
} mi_paged_kv;

/* Human-readable text for a status code (static storage). */
const char* mi_status_string(int status);

/* MI_ABI_VERSION of the loaded library. */
int mi_abi_version(void);

/* ------------------------------------------------------------------------
 * P1 — per-step batch packing on the GPU.
 * Replaces the Python packing loop of BatchedCacheManager._plan_attention_impl
 * (mstar/engine/cache_manager.py:272-322).  Pages must already be allocated
 * (host FIFO allocator, mstar/engine/kv_store.py:463-482).  Request r's page
 * list is its block-table row: the first table_pages[r] entries are already
 * in the table, the remaining num_pages[r] - table_pages[r] follow in
 * new_pages (all requests' new pages concatenated in batch order) and are
 * written into the row by this call (table_pages == NULL: all pages are in
 * the table, new_pages unused).  For request r (batch order):
 *   T_r             = seq_len[r] + new_len[r]
 *   qo_indptr[r+1]  = qo_indptr[r] + new_len[r]
 *   kv_indptr[r+1]  = kv_indptr[r] + num_pages[r]
 *   kv_indices[kv_indptr[r] + p] = page p of request r's list
 *   last_page_len[r]= T_r % page_size, or page_size when that is 0
 *   kv_locations[r] = (last page of the request's list, last_page_len[r] - 1) when
 *                     new_len[r] == 1 (cache_manager.py:293-294), (-1, -1) if the list
 *                     is empty; only if kv_locations != NULL (int64 [batch, 2]); rows
 *                     with new_len != 1 are left untouched
 * grid_blocks: number of workgroups to launch (>= 1); every workgroup
 * recomputes the prefix sums, so no inter-block synchronisation is needed.
 * ------------------------------------------------------------------------ */
int mi_pack(const int32_t* req_slot, const int32_t* seq_len, const int32_t* new_len,
            const int32_t* num_pages, int32_t batch, int32_t* block_table,
            int64_t block_table_stride, const int32_t* table_pages, const int32_t* new_pages,
            int32_t page_size, int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
            int32_t* last_page_len, int64_t* kv_locations, int32_t grid_blocks, void* stream);

/* mi_pack followed by mi_decode_plan(NULL, kv_indptr, kv_indices, last_page_len, batch,
 * page_size, num_qo_heads, num_kv_heads, head_dim, NULL, workspace, workspace_bytes) in
 * one launch, for decode steps (new_len[r] == 1 for every request; kv_locations as in
 * mi_pack).  The plan workgroup reads the per-request page counts num_pages directly, so
 * it runs beside the packing workgroups; the packed arrays and the plan in the workspace
 * are those of the two separate calls.  Replaces the pair of calls BatchedCacheManager
 * makes per decode step (cache_manager.py:399-415 -> FlashInferDecodeWrapper.plan,
 * flashinfer_utils.py:369-453). */
int mi_pack_plan(const int32_t* req_slot, const int32_t* seq_len, const int32_t* new_len,
                 const int32_t* num_pages, int32_t batch, int32_t* block_table,
                 int64_t block_table_stride, const int32_t* table_pages, const int32_t* new_pages,
                 int32_t page_size, int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
                 int32_t* last_page_len, int64_t* kv_locations, int32_t grid_blocks,
                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* mi_pack_plan (workspace != NULL) or mi_pack (workspace == NULL) with the step's
 * metadata in HOST memory, handed to the kernel as its launch argument instead of being
 * copied to the device first: meta holds meta_len int32 values,
 * [req_slot | seq_len | new_len | num_pages | table_pages] (batch values each, in that
 * order) followed by the new pages (as many as the num_pages - table_pages differences
 * add up to, else MI_ERR_INVALID); the buffer may be reused once the call returns.
 * meta_len <= MI_PACK_HOST_META is always accepted.  Up to MI_PACK_HOST_META_MAX values
 * are accepted when the step fits the argument in a compact form (every req_slot,
 * new_len, num_pages and table_pages below 65536, two of them per int32, and
 * 3 * batch + new pages <= MI_PACK_HOST_ARGS); otherwise the call returns
 * MI_ERR_UNSUPPORTED without launching anything and the caller uses mi_pack_plan.
 * Same outputs as the device-pointer entry points.  Extension for small steps (no
 * counterpart in the reference): it saves the host-to-device copy of the metadata. */
#define MI_PACK_HOST_META 768
#define MI_PACK_HOST_META_MAX 4096
#define MI_PACK_HOST_ARGS 896
int mi_pack_plan_host(const int32_t* meta, int32_t meta_len, int32_t batch, int32_t* block_table,
                      int64_t block_table_stride, int32_t page_size, int32_t* qo_indptr,
                      int32_t* kv_indptr, int32_t* kv_indices, int32_t* last_page_len,
                      int64_t* kv_locations, int32_t grid_blocks, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t head_dim, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* Incremental device block-table update: block_table[slot[i]*stride + pos[i]] = page[i]
 * for i < n.  Keeps the device copy of each request's page list in step with the
 * host allocator (mstar/engine/kv_store.py:463-482) without re-sending whole lists. */
int mi_block_table_update(int32_t* block_table, int64_t stride, const int32_t* slot,
                          const int32_t* pos, const int32_t* page, int32_t n, void* stream);

/* ------------------------------------------------------------------------
 * P4 — decode plan: split-KV work partition built on the GPU.
 * Replaces FlashInfer's BatchDecodeWithPagedKVCacheWrapper.plan as called from
 * FlashInferDecodeWrapper.plan (mstar/utils/flashinfer_utils.py:369-453),
 * including the write locations of flashinfer_utils.py:433-436.
 * qo_indptr == NULL means one query token per request (decode); otherwise
 * request r has qo_indptr[r+1]-qo_indptr[r] query tokens and
 * (query tokens) * (num_qo_heads/num_kv_heads) must be <= 16 for every request.
 * kv_locations (nullable, int64 [batch, 2]) receives
 * (kv_indices[kv_indptr[r+1]-1], last_page_len[r]-1), or (-1, -1) when the
 * request holds no page.
 * mi_decode_workspace_bytes gives the recommended workspace size; a smaller
 * workspace makes the plan use fewer, longer KV chunks (MI_ERR_WORKSPACE only
 * when not even batch+1 chunks fit).  The plan is stored in the workspace and
 * read by mi_decode_run, which must get the same workspace size.
 * ------------------------------------------------------------------------ */
int64_t mi_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim);
int mi_decode_plan(const int32_t* qo_indptr, const int32_t* kv_indptr,
                   const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                   int32_t page_size, int32_t num_qo_heads, int32_t num_kv_heads,
                   int32_t head_dim, int64_t* kv_locations, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * P6 — paged GQA decode attention (+ split-KV merge).
 * Replaces FlashInferDecodeWrapper.run (mstar/utils/flashinfer_utils.py:455-465).
 *   out[t, h, :] = softmax(sm_scale * q[t,h,:] . K_r[:, h / G, :]) V_r[:, h / G, :]
 * over the request's kv_len = (npages-1)*page_size + last_page_len tokens
 * (causal alignment to the end of the KV when a request has several query
 * tokens and causal != 0).  q and out: [tokens, num_qo_heads, head_dim] with
 * the given element strides (head_dim contiguous), dtype q_dtype: bf16 or
 * fp16 (the cache's dtype, or an fp8 cache), or fp32 with an fp32 cache
 * (attention computed in fp32 throughout).  Requests without KV produce zeros.
 * q, out and the KV layer are moved in 16-byte pieces: their bases must be
 * 16-byte aligned and every element stride a whole number of 16-byte pieces
 * (MI_ERR_INVALID otherwise; mi_prefill_run checks the same).
 * mi_decode_run = mi_decode_attend (one wavefront per (KV chunk, kv-head):
 * finished rows of unsplit requests, partial (o, lse) of split ones) followed
 * by mi_decode_merge (log-sum-exp merge of the partials); the two halves take
 * the same arguments and may be called separately on the same stream.
 * ------------------------------------------------------------------------ */
int mi_decode_run(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                  const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                  const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                  int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                  int64_t workspace_bytes, void* out, int64_t out_stride_token,
                  int64_t out_stride_head, void* stream);
int mi_decode_attend(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                     const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                     int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                     int64_t workspace_bytes, void* out, int64_t out_stride_token,
                     int64_t out_stride_head, void* stream);
int mi_decode_merge(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                    const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                    const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                    int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                    int64_t workspace_bytes, void* out, int64_t out_stride_token,
                    int64_t out_stride_head, void* stream);

/* ------------------------------------------------------------------------
 * Decode without a caller workspace.  No counterpart in the reference: this
 * entry point is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * mi_decode_noalloc = mi_decode_plan(qo_indptr, kv_indptr, kv_indices,
 * last_page_len, batch, kv->page_size, num_qo_heads, kv->num_kv_heads,
 * kv->head_dim, kv_locations, ...) followed by mi_decode_run on the same
 * stream, with the plan and the split-KV partials kept in a static device
 * buffer the library holds on every GPU it runs on (MI_NOALLOC_SCRATCH_BYTES
 * per device, until the process ends) instead of a workspace.  Outputs and
 * kv_locations equal those of the two calls given a workspace of
 * MI_NOALLOC_SCRATCH_BYTES bytes.  Limit: the buffer must hold batch + 1
 * split-KV items of partials (4 * num_kv_heads * 16 * (head_dim + 1) bytes
 * each, plus the plan's header and offsets; for 4 kv heads and head_dim 128
 * a batch of up to about 2000 requests); a larger batch returns
 * MI_ERR_WORKSPACE before anything is launched.  The stream must belong to
 * the current device.  All calls on one GPU share its buffer, so calls that
 * overlap on one GPU (two streams, or two threads without ordering between
 * them) race.  Allocates nothing.
 * ------------------------------------------------------------------------ */
#define MI_NOALLOC_SCRATCH_BYTES (64LL << 20)
int mi_decode_noalloc(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                      const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                      const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                      int32_t num_qo_heads, int32_t causal, float sm_scale, void* out,
                      int64_t out_stride_token, int64_t out_stride_head, int64_t* kv_locations,
                      void* stream);

/* ------------------------------------------------------------------------
 * P5 — paged KV append.
 * Replaces FlashInferPrefillWrapper.set_kv_cache / FlashInferDecodeWrapper.set_kv_cache
 * (mstar/utils/flashinfer_utils.py:271-288, 467-484):
 *   cache[page[i], K, slot[i]] = k[i];  cache[page[i], V, slot[i]] = v[i]
 * cast to the cache dtype (RNE; fp8: x * (1/scale) clamped to +-448, then RNE).
 * page[i] = page_idx[i * idx_stride], slot[i] = slot_idx[i * idx_stride]
 * (idx_stride 1 for token_to_page/token_to_cache, 2 for kv_cache_locations
 * [B, 2] with slot_idx = page_idx + 1).  Tokens whose page id is outside
 * [0, max_pages) or slot outside [0, page_size) are skipped.  When
 * num_tokens_device != NULL only the first min(num_tokens, *num_tokens_device)
 * tokens are written (graph-replay padding is dropped).
 * k, v: [num_tokens, num_kv_heads, head_dim], element strides given, dtype src_dtype.
 * ------------------------------------------------------------------------ */
int mi_kv_append(const mi_paged_kv* kv, const void* k, const void* v, int32_t src_dtype,
                 int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_token,
                 int64_t v_stride_head, const int64_t* page_idx, const int64_t* slot_idx,
                 int64_t idx_stride, int32_t num_tokens, const int32_t* num_tokens_device,
                 void* stream);

/* ------------------------------------------------------------------------
 * P3 + P7 — ragged prefill plan and attention.
 * mi_prefill_plan replaces FlashInferPrefillWrapper.plan
 * (mstar/utils/flashinfer_utils.py:162-256): it writes the per-token page map
 *   token_to_page[t]  = kv_indices[kv_indptr[r] + g / page_size]
 *   token_to_cache[t] = g % page_size,  g = kv_len_r - qo_len_r + (t - qo_indptr[r])
 * for t < qo_indptr[batch] (entries in [qo_indptr[batch], token_map_len) are set
 * to 0, like the graph-mode tail fill of flashinfer_utils.py:251-253), and the
 * work partition for mi_prefill_run into the workspace.  Requests whose
 * qo_len * (num_qo_heads/num_kv_heads) <= mi_prefill_short_rows(...) (16, or 8
 * for a plan over kv-head pairs) go to the split-KV decode kernel, longer
 * ones to the MFMA prefill kernel.
 * max_qo_tokens bounds qo_indptr[batch] (grid sizing without a host sync);
 * mi_prefill_run must get the same batch, max_qo_tokens and workspace.
 * mi_prefill_run replaces FlashInferPrefillWrapper.run (:258-269):
 *   out[t, h] = softmax(sm_scale * q[t,h] . K_r^T) V_r over the request's keys
 *   i <= kv_len - qo_len + j for query j (causal) or all kv_len keys.
 * q/out dtypes as for mi_decode_run (fp32 with an fp32 cache included).
 * The KV layer's K-to-V offset plus page_size token rows must stay below
 * 2^31 bytes (MI_ERR_UNSUPPORTED otherwise; M*'s page layout is far below).
 * mi_prefill_run = mi_prefill_short (the short-query requests, through the
 * split-KV decode kernel and merge) followed by mi_prefill_tiles (the MFMA
 * tiles of the long-query requests).  The halves take the same arguments and
 * write disjoint output rows; after the plan they may run in either order or
 * on two streams.  They have no separate counterpart in the reference.
 * ------------------------------------------------------------------------ */
int64_t mi_prefill_workspace_bytes(int32_t batch, int32_t max_qo_tokens, int32_t num_qo_heads,
                                   int32_t num_kv_heads, int32_t head_dim);
/* Which requests of a plan of this shape are short-query requests (run by
 * mi_prefill_short): those with qo_len * (num_qo_heads / num_kv_heads) at most
 * the returned number of rows; the others are mi_prefill_tiles' work.  16, or
 * 8 when the plan reads kv-head pairs as one row (batch >= 128, head_dim 128,
 * at most 8 q-heads per kv-head, an even number of kv-heads).  For a caller
 * that skips a launch with no work; negative on invalid arguments.  Helper
 * of this library's split of FlashInferPrefillWrapper.run, no counterpart in
 * the reference. */
int32_t mi_prefill_short_rows(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim);
int mi_prefill_plan(const int32_t* qo_indptr, const int32_t* kv_indptr,
                    const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                    int32_t max_qo_tokens, int32_t page_size, int32_t num_qo_heads,
                    int32_t num_kv_heads, int32_t head_dim, int64_t* token_to_page,
                    int64_t* token_to_cache, int32_t token_map_len, void* workspace,
                    int64_t workspace_bytes, void* stream);
int mi_prefill_run(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                   const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                   const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                   int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, float sm_scale, void* workspace,
                   int64_t workspace_bytes, void* out, int64_t out_stride_token,
                   int64_t out_stride_head, void* stream);
int mi_prefill_short(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                     const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                     int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, float sm_scale,
                     void* workspace, int64_t workspace_bytes, void* out, int64_t out_stride_token,
                     int64_t out_stride_head, void* stream);
int mi_prefill_tiles(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                     const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                     int32_t max_qo_tokens, int32_t num_qo_heads, int32_t causal, float sm_scale,
                     void* workspace, int64_t workspace_bytes, void* out, int64_t out_stride_token,
                     int64_t out_stride_head, void* stream);

/* ------------------------------------------------------------------------
 * RoPE on the packed batch (the path's next row: the rotation every layer
 * applies to q and k right before the append and the attention).
 * mi_rope_positions replaces the position list of
 * BatchedCacheManager._plan_rope_impl (mstar/engine/cache_manager.py:480-492):
 *   pos_ids[t] = position_id_start[r] + (t - qo_indptr[r]),  t < num_tokens.
 * mi_rope_apply replaces the FlashInfer call of BatchedCacheManager.apply_rope
 * (cache_manager.py:702-760; flashinfer.rope.apply_rope_pos_ids_inplace and
 * apply_llama31_rope_pos_ids_inplace): q [num_tokens, num_qo_heads, head_dim]
 * and k [num_tokens, num_kv_heads, head_dim] (bf16 or f16, element strides,
 * head_dim contiguous) are rotated in place.  Dims [0, rotary_dim) turn in
 * pairs (i, i + rotary_dim/2), or (2i, 2i+1) when interleave != 0, by the
 * fp32 angle pos * f_i, f_i = theta^(-2i/rotary_dim) / rope_scale; with
 * llama31 != 0 the frequency is blended towards theta^(-2i/rotary_dim) by
 * clamp(old_context_len * g / (2 pi (high - low)) - low / (high - low), 0, 1).
 * rotary_dim and head_dim must be multiples of 8; pos_dtype MI_I32 or MI_I64.
 * ------------------------------------------------------------------------ */
int mi_rope_positions(const int32_t* qo_indptr, const int32_t* position_id_start, int32_t batch,
                      int64_t* pos_ids, int32_t num_tokens, void* stream);
int mi_rope_apply(void* q, int64_t q_stride_token, int64_t q_stride_head, int32_t num_qo_heads, void* k,
                  int64_t k_stride_token, int64_t k_stride_head, int32_t num_kv_heads, int32_t dtype,
                  int32_t head_dim, int32_t rotary_dim, const void* pos_ids, int32_t pos_dtype,
                  int32_t num_tokens, int32_t interleave, float rope_scale, float rope_theta,
                  int32_t llama31, float low_freq_factor, float high_freq_factor, float old_context_len,
                  void* stream);
/* mi_rope_append fuses BatchedCacheManager.apply_rope (cache_manager.py:702-760)
 * with the K/V append of run_attention (cache_manager.py:653-701 ->
 * FlashInfer*Wrapper.set_kv_cache, flashinfer_utils.py:271-288, 467-484):
 * one pass that rotates q in place (as mi_rope_apply), rotates k (in place
 * when keep_k != 0), and writes the rotated k and v [num_tokens,
 * kv->num_kv_heads, kv->head_dim] of tokens t < min(num_append_tokens,
 * *num_tokens_device) to their cache slots (as mi_kv_append with num_tokens =
 * num_append_tokens, and the same page_idx/slot_idx/idx_stride meaning; k and
 * v in `dtype`, 16-byte aligned rows).  All num_tokens tokens of q and k are
 * rotated.  The cache contents, q and (with keep_k) k are bit-identical to
 * mi_rope_apply followed by mi_kv_append.
 * ------------------------------------------------------------------------ */
int mi_rope_append(void* q, int64_t q_stride_token, int64_t q_stride_head, int32_t num_qo_heads, void* k,
                   int64_t k_stride_token, int64_t k_stride_head, const void* v, int64_t v_stride_token,
                   int64_t v_stride_head, int32_t dtype, int32_t keep_k, const mi_paged_kv* kv,
                   const int64_t* page_idx, const int64_t* slot_idx, int64_t idx_stride,
                   int32_t num_append_tokens, const int32_t* num_tokens_device, int32_t rotary_dim,
                   const void* pos_ids, int32_t pos_dtype, int32_t num_tokens, int32_t interleave,
                   float rope_scale, float rope_theta, int32_t llama31, float low_freq_factor,
                   float high_freq_factor, float old_context_len, void* stream);

/* ------------------------------------------------------------------------
 * Page snapshot copies (multi-label / CFG planning).
 * mi_copy_pages replaces the per-page copies of BatchedCacheManager.snapshot_all
 * (mstar/engine/cache_manager.py:840-870): for i < num_pairs and every layer l,
 *   page dst_pages[i] of layer l := page src_pages[i] of layer l
 * in a pool laid out as [num_layers][max_pages][page_bytes...] with the given
 * byte strides (16-byte aligned).  No destination may also be a source in
 * the same call.  Pairs with ids outside [0, max_pages) are skipped.
 * ------------------------------------------------------------------------ */
int mi_copy_pages(void* pool, int64_t layer_stride_bytes, int32_t num_layers, int64_t page_stride_bytes,
                  int64_t page_bytes, int64_t max_pages, const int32_t* src_pages, const int32_t* dst_pages,
                  int32_t num_pairs, void* stream);

/* ------------------------------------------------------------------------
 * KV page transfer: remote reads, CPU offload/reload, wire format.
 *
 * A whole KV pool, all layers: [num_layers][num_pages][2 (K,V)][page_size]
 * token rows of token_stride bytes (num_kv_heads * head_dim elements, the
 * layout of kv_cache_engine.py:132-136), byte strides, 16-byte aligned.
 * `data` must be HIP device memory or HIP-allocated pinned host memory
 * (torch pin_memory); anything else is MI_ERR_INVALID.
 *
 * A record i names a page and a token range [token_start[i], token_end[i])
 * (NULL arrays: whole pages) and stands for the K rows and the V rows of
 * that range in every layer of [layer_begin, layer_end).  Records with page
 * ids outside [0, num_pages) or an empty or out-of-page range are skipped.
 * No destination row may be written by two records or read by another
 * record of the same call.
 * ------------------------------------------------------------------------ */
typedef struct mi_kv_pool {
  void* data;           /* (layer 0, page 0, K, token 0) */
  int64_t layer_stride; /* bytes */
  int64_t page_stride;  /* bytes */
  int64_t kv_stride;    /* bytes from a page's K half to its V half */
  int64_t token_stride; /* bytes of one token row; rows of a half are contiguous */
  int64_t num_pages;
  int32_t num_layers;
  int32_t page_size;
} mi_kv_pool;

/* Pool-to-pool token copies: dst page dst_pages[i] rows [ts, te) := src page
 * src_pages[i] rows [ts, te), K and V, every layer of the range.  src and
 * dst may be the same pool (then sources and destinations must not overlap)
 * and either may live in pinned host memory.  Replaces
 *   - CudaIpcKVTransferEngine._do_read (mstar/engine/kv_store.py:330-380) and
 *     MooncakeKVTransferEngine.read_batched_async + _get_ptr_nbytes
 *     (kv_store.py:233-285): one KVReadInfo per (layer, page), one transfer
 *     or torch copy per record;
 *   - CPUPagePool.offload_pages / reload_pages
 *     (mstar/engine/cpu_page_pool.py:63-124): one torch copy per page.
 * src and dst must agree in token_stride and page_size. */
int mi_kv_copy_tokens(const mi_kv_pool* src, const mi_kv_pool* dst, const int32_t* src_pages,
                      const int32_t* dst_pages, const int32_t* token_start, const int32_t* token_end,
                      int32_t num_records, int32_t layer_begin, int32_t layer_end, void* stream);

/* Wire format: the records' rows in one contiguous buffer, layer-major.  With
 * rows_i = token_end[i] - token_start[i], R = sum rows_i and row_offset the
 * exclusive prefix sum of rows (num_records + 1 entries, device memory;
 * NULL allowed only with NULL token ranges, meaning i * page_size), record
 * i's K rows for layer l start at token row
 *   2*R*(l - layer_begin) + 2*row_offset[i]
 * followed by its V rows; the buffer holds
 * 2*R*(layer_end - layer_begin)*token_stride bytes.  Segments that would fall
 * outside [0, wire_bytes) or whose row_offset entries disagree with the
 * ranges are skipped.  No counterpart in the reference, which moves each
 * (layer, page, K|V) segment separately (kv_store.py:261-285); a transport
 * sends one buffer instead. */
int mi_kv_wire_pack(const mi_kv_pool* pool, const int32_t* pages, const int32_t* token_start,
                    const int32_t* token_end, const int64_t* row_offset, int32_t num_records,
                    int32_t layer_begin, int32_t layer_end, void* wire, int64_t wire_bytes, void* stream);
int mi_kv_wire_unpack(const void* wire, int64_t wire_bytes, const mi_kv_pool* pool, const int32_t* pages,
                      const int32_t* token_start, const int32_t* token_end, const int64_t* row_offset,
                      int32_t num_records, int32_t layer_begin, int32_t layer_end, void* stream);

/* Measurement only (no counterpart in the reference): reads `bytes` (a
 * multiple of 16, `data` 16-byte aligned) of device memory with the decode
 * kernels' 16-byte non-temporal loads, `grid` workgroups of 256 threads, and
 * writes one folded word per wavefront to sink[0 .. 4*grid).  Its rate over a
 * KV pool is the box's plain HBM read ceiling, which the benchmark reports
 * beside the decode kernel's achieved bandwidth. */
int mi_hbm_read(const void* data, int64_t bytes, uint32_t* sink, int32_t grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSTAR_AMD_H */
