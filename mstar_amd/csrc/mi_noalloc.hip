// Decode plan + attention for callers that cannot allocate device memory.
//
// mi_decode_noalloc runs what mi_decode_plan followed by mi_decode_run do,
// with the split-KV plan and the partial (o, lse) results kept in a
// library-owned static device buffer (`scratch`, MI_NOALLOC_SCRATCH_BYTES per
// device) instead of a caller workspace.  The kernels are the decode
// translation unit's; this file only owns the buffer and resolves its device
// address once per device.
//
// `scratch` names a host-side shadow in host code.  Its device address comes
// from hipGetSymbolAddress with the device current, is kept per device and is
// the only form of it that host code passes on.
#include <mutex>

#include "mi_internal.h"

namespace mi {

constexpr int64_t kScratchBytes = MI_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size must keep 256-byte alignment of the plan layout");

// Every GPU holds its own copy for the life of the process.  Nothing in it
// has to start at zero: the plan kernel writes the header, item offsets and
// work list before the decode kernel reads them, and the decode kernel writes
// every partial the merge reads.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device id

// Device address of `scratch` on `device`, which must be the current device.
static int scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return MI_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) return MI_ERR_LAUNCH;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return MI_OK;
}

}  // namespace mi

extern "C" int mi_decode_noalloc(const void* q, int32_t q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                                 const mi_paged_kv* kv, const int32_t* qo_indptr, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* last_page_len, int32_t batch,
                                 int32_t num_qo_heads, int32_t causal, float sm_scale, void* out,
                                 int64_t out_stride_token, int64_t out_stride_head, int64_t* kv_locations,
                                 void* stream) {
  if (!kv || batch < 0) return MI_ERR_INVALID;
  if (batch == 0) return MI_OK;
  if (kv->num_kv_heads <= 0 || num_qo_heads <= 0) return MI_ERR_INVALID;
  // Host-side size check against the fixed buffer: the plan needs at least
  // batch + 1 items of partials beside its header and item offsets.
  const mi::SplitLayout L = mi::split_layout(batch, kv->num_kv_heads, kv->head_dim, mi::kScratchBytes);
  if (L.max_chunks <= batch || L.total > mi::kScratchBytes) return MI_ERR_WORKSPACE;
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess) return MI_ERR_LAUNCH;
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess) return MI_ERR_INVALID;
    if (sdev != device) return MI_ERR_INVALID;  // the buffer of the current device only
  }
  void* ws = nullptr;
  int st = mi::scratch_address(device, &ws);
  if (st != MI_OK) return st;
  st = mi::decode_plan_impl(qo_indptr, kv_indptr, kv_indices, last_page_len, batch, kv->page_size, num_qo_heads,
                            kv->num_kv_heads, kv->head_dim, kv_locations, ws, mi::kScratchBytes, 0,
                            (hipStream_t)stream);
  if (st != MI_OK) return st;
  return mi::decode_run_impl(q, q_dtype, q_stride_token, q_stride_head, kv, qo_indptr, kv_indptr, kv_indices,
                             last_page_len, batch, num_qo_heads, causal, sm_scale, ws, mi::kScratchBytes, 0, out,
                             out_stride_token, out_stride_head, mi::kPhaseAttend | mi::kPhaseMerge,
                             (hipStream_t)stream);
}
