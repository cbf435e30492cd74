"""plan()/run()/set_kv_cache() wrappers over the gfx950 kernels.

Drop-in replacements for M*'s ``FlashInferPrefillWrapper`` and
``FlashInferDecodeWrapper`` (``mstar/utils/flashinfer_utils.py:70-484``): same
constructor arguments, same ``plan``/``run``/``set_kv_cache`` signatures and the
same attributes that M*'s cache manager and CUDA-graph runner read
(``_qo_indptr_buf``, ``token_to_page``, ``token_to_cache``, ``_total_tokens``,
``kv_cache_locations``, ``_n_req``, the ``_paged_kv_*_buf`` static buffers).
The reference names are exported as aliases.

KV layer layout: ``[max_pages, 2, page_size, num_kv_heads, head_dim]`` (NHD).

Differences from the reference, all deliberate:

* No FlashInfer: planning runs on the GPU (``mi_decode_plan`` /
  ``mi_prefill_plan``) and never reads device memory back on the host.
  ``plan()`` accepts CPU or device index tensors; CPU tensors go through one
  pinned, asynchronous host->device copy.
* ``set_kv_cache`` writes K and V in one kernel and, in CUDA-graph mode, skips
  the padding tokens beyond the planned count (the reference maps them to
  page 0 slot 0, ``flashinfer_utils.py:251-253``).
* Optional fp8-e4m3 KV caches (``torch.float8_e4m3fn``) with per-head fp32
  ``k_scale``/``v_scale`` passed to ``set_kv_cache`` and ``run``.
* ``rope_set_kv_cache`` (no reference counterpart) fuses the RoPE call that
  precedes ``set_kv_cache`` in every layer with the append itself.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .trace import trace_range

__all__ = [
    "PagedPrefillWrapper",
    "PagedDecodeWrapper",
    "FlashInferPrefillWrapper",
    "FlashInferDecodeWrapper",
]

_MAX_GROUP = 16  # q heads per kv head handled by one MFMA tile


def _check_heads(num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int) -> None:
    if num_kv_heads <= 0 or num_qo_heads % num_kv_heads:
        raise ValueError(f"num_qo_heads={num_qo_heads} must be a multiple of num_kv_heads={num_kv_heads}")
    if num_qo_heads // num_kv_heads > _MAX_GROUP:
        raise ValueError(f"GQA group {num_qo_heads // num_kv_heads} > {_MAX_GROUP} is not supported")
    if head_dim not in (64, 128, 256):
        raise ValueError(f"head_dim {head_dim} not supported (64, 128, 256)")
    if page_size <= 0 or page_size % 16:
        raise ValueError(f"page_size {page_size} must be a positive multiple of 16")


class _Staging:
    """Pinned host buffers for asynchronous index uploads, reused across plans.

    Two buffers alternate, and each upload is one copy on a side stream of
    its own, issued as soon as plan() is called: it runs beside whatever the
    launch stream is still executing (the previous step's attention), and
    the launch stream waits for it (an event) before the plan kernel.  On
    one stream the copy would sit between the previous step's last kernel
    and this step's plan kernel (about 20 us for c4's 166 KB of indices).
    """

    def __init__(self):
        self.bufs: list = [None, None]
        self.events: list = [None, None]
        self.i = 0
        self.stream: torch.cuda.Stream | None = None

    def upload(self, parts: list[torch.Tensor], device: torch.device,
               dests: list[torch.Tensor | None]) -> list[torch.Tensor]:
        """Copy CPU int tensors to the device in one transfer.

        ``dests[i]`` (a device tensor of at least ``parts[i].numel()``
        elements, same dtype) receives part ``i`` in place; ``None`` allocates.
        """
        flat = [p.reshape(-1).view(torch.int32) if p.dtype == torch.int64 else p.reshape(-1) for p in parts]
        sizes = [f.numel() for f in flat]
        total = sum(sizes)
        i = self.i
        self.i ^= 1
        if self.events[i] is not None:
            self.events[i].synchronize()  # the copy that last read buffer i is done
        buf = self.bufs[i]
        if buf is None or buf.numel() < total:
            buf = self.bufs[i] = torch.empty(max(total, 1 << 16), dtype=torch.int32, pin_memory=True)
        # numpy copies on the calling thread: torch's CPU copy_ of a part above
        # its grain size wakes the intra-op thread pool, which cost 0.1-0.7 ms
        # per plan on a box whose pool had been resized
        host = buf.numpy()
        off = 0
        for f, n in zip(flat, sizes):
            host[off:off + n] = f.numpy()
            off += n
        cur = torch.cuda.current_stream(device)
        if torch.cuda.is_current_stream_capturing():  # a captured plan keeps the copy on its own stream
            staged = torch.empty(total, dtype=torch.int32, device=device)
            staged.copy_(buf[:total], non_blocking=True)
            ev = self.events[i] = torch.cuda.Event()
            ev.record(cur)
        else:
            if self.stream is None or self.stream.device != cur.device:
                self.stream = torch.cuda.Stream(device=device)
            with torch.cuda.stream(self.stream):
                staged = torch.empty(total, dtype=torch.int32, device=device)
                staged.copy_(buf[:total], non_blocking=True)
                ev = self.events[i] = torch.cuda.Event()
                ev.record(self.stream)
            cur.wait_event(ev)
            staged.record_stream(cur)  # read on the launch stream from here on
        outs = []
        off = 0
        for p, f, n, d in zip(parts, flat, sizes, dests):
            piece = staged[off:off + n]
            if p.dtype == torch.int64:
                piece = piece.view(torch.int64)
            piece = piece.view(p.shape)
            off += n
            if d is not None:
                d.view(-1)[: piece.numel()].copy_(piece.reshape(-1))
                outs.append(d)
            else:
                outs.append(piece)
        return outs


def _as_device_int(t: torch.Tensor, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if t.dtype != dtype:
        t = t.to(dtype)
    if t.device != device:
        t = t.to(device, non_blocking=True)
    return t.contiguous()


def _q_strides(q: torch.Tensor, name: str) -> tuple[int, int]:
    if q.dim() != 3 or q.stride(2) != 1:
        raise ValueError(f"{name} must be [tokens, heads, head_dim] with contiguous head_dim")
    if q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        raise ValueError(f"{name}: rows must be 16-byte aligned")
    return q.stride(0), q.stride(1)


def _kv_src(k: torch.Tensor, name: str) -> torch.Tensor:
    if k.dim() != 3:
        raise ValueError(f"{name} must be [tokens, num_kv_heads, head_dim]")
    if k.stride(2) != 1 or k.stride(0) % 8 or k.stride(1) % 8 or k.data_ptr() % (8 * k.element_size()):
        k = k.contiguous()
    return k


def _append(kv_cache_layer: torch.Tensor, k: torch.Tensor, v: torch.Tensor, page_idx: torch.Tensor,
            slot_idx_ptr: int, idx_stride: int, n: int, n_dev_ptr: int | None,
            k_scale: torch.Tensor | None, v_scale: torch.Tensor | None) -> None:
    if n == 0:
        return
    desc = _lib.paged_kv_desc(kv_cache_layer, k_scale, v_scale)
    if k.shape[1:] != (desc.num_kv_heads, desc.head_dim) or v.shape[1:] != k.shape[1:]:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match the cache heads/head_dim")
    if k.shape[0] < n or v.shape[0] < n:
        raise ValueError(f"k/v hold {k.shape[0]} tokens, {n} planned")
    src_dt = _lib.TORCH_TO_MI.get(k.dtype)
    if src_dt is None or src_dt == _lib.MI_FP8_E4M3:
        raise ValueError(f"unsupported k/v dtype {k.dtype}")
    if v.dtype != k.dtype:
        v = v.to(k.dtype)
    k = _kv_src(k, "k")
    v = _kv_src(v, "v")
    _lib.check(
        _lib.lib().mi_kv_append(
            desc, k.data_ptr(), v.data_ptr(), src_dt, k.stride(0), k.stride(1), v.stride(0), v.stride(1),
            page_idx.data_ptr(), slot_idx_ptr, idx_stride, n, n_dev_ptr, _lib.stream_ptr(kv_cache_layer.device),
        ),
        "mi_kv_append",
    )


def _rope_set_kv_cache(wrapper, kv_cache_layer, q, k, v, pos_ids, rotary_dim, interleave, rope_scale, rope_theta,
                       k_scale, v_scale, keep_k, llama31) -> None:
    from .rope import rope_append

    page_idx, slot_ptr, idx_stride, n, n_dev = wrapper._append_target()
    rope_append(q, k, v, kv_cache_layer, pos_ids, page_idx, slot_ptr, idx_stride, n, n_dev,
                rotary_dim=rotary_dim, interleave=interleave, rope_scale=rope_scale, rope_theta=rope_theta,
                k_scale=k_scale, v_scale=v_scale, keep_k=keep_k, llama31=llama31)


class _FusedRopeAppend:
    """``rope_set_kv_cache``: RoPE on q/k fused with ``set_kv_cache`` (one launch)."""

    def rope_set_kv_cache(self, kv_cache_layer: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          pos_ids: torch.Tensor, rotary_dim: int | None = None, interleave: bool = False,
                          rope_scale: float = 1, rope_theta: float = 1e4, k_scale: torch.Tensor | None = None,
                          v_scale: torch.Tensor | None = None, keep_k: bool = True,
                          llama31: dict | None = None) -> None:
        """``apply_rope_pos_ids_inplace(q, k, pos_ids, ...)`` then ``set_kv_cache(kv_cache_layer, k, v)``.

        Same results bit for bit, in one kernel (``mi_rope_append``).  ``llama31``
        holds ``low_freq_factor``/``high_freq_factor``/``old_context_len`` for
        the Llama-3.1 frequencies.  q, k and v share one dtype (bf16 or fp16);
        k and v rows must be 16-byte aligned.
        """
        _rope_set_kv_cache(self, kv_cache_layer, q, k, v, pos_ids, rotary_dim, interleave, rope_scale, rope_theta,
                           k_scale, v_scale, keep_k, llama31)


class PagedDecodeWrapper(_FusedRopeAppend):
    """Batched paged decode attention (``flashinfer_utils.py:291-484``)."""

    def __init__(
        self,
        workspace_buffer: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        batch_size: int | None = None,
        max_num_pages: int | None = None,
        device: torch.device = torch.device("cuda"),
        use_cuda_graph: bool = False,
        enable_nvtx: bool = False,
    ):
        _check_heads(num_qo_heads, num_kv_heads, head_dim, page_size)
        _lib.lib()
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.use_cuda_graph = use_cuda_graph
        self.enable_nvtx = enable_nvtx
        self.batch_size = batch_size
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.dtype = None
        self._workspace = workspace_buffer
        self._staging = _Staging()
        self._n_req = 0
        if use_cuda_graph:
            assert batch_size is not None, "batch_size required for CUDA graph mode"
            assert max_num_pages is not None, "max_num_pages required for CUDA graph mode"
            self._paged_kv_indptr_buf = torch.zeros(batch_size + 1, dtype=torch.int32, device=self.device)
            self._paged_kv_indices_buf = torch.zeros(max_num_pages, dtype=torch.int32, device=self.device)
            self._paged_kv_last_page_len_buf = torch.ones(batch_size, dtype=torch.int32, device=self.device)
            self.kv_cache_locations = torch.zeros(batch_size, 2, dtype=torch.long, device=self.device)
        else:
            self.kv_cache_locations = None

    # -------------------------------------------------------------- plan
    def plan(
        self,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        kv_cache_locations: torch.Tensor | None = None,
        dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        """Build the split-KV plan on the GPU (``flashinfer_utils.py:369-453``)."""
        n_req = paged_kv_indptr.shape[0] - 1
        if paged_kv_last_page_len.shape[0] != n_req:
            raise ValueError("paged_kv_last_page_len must have one entry per request")
        dev = self.device
        if self.use_cuda_graph:
            if n_req != self.batch_size:  # captured launches bake the batch in
                raise ValueError(f"CUDA-graph mode plans a fixed batch of {self.batch_size}, got {n_req}")
            if paged_kv_indices.shape[0] > self._paged_kv_indices_buf.shape[0]:
                raise ValueError("paged_kv_indices exceeds max_num_pages")
            dests = [self._paged_kv_indptr_buf, self._paged_kv_indices_buf, self._paged_kv_last_page_len_buf]
        else:
            dests = [None, None, None]
        srcs = [paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len]
        nv = self.enable_nvtx
        with trace_range(nv, "flashinfer.decode.metadata_h2d"):
            if all(t.device.type == "cpu" for t in srcs):
                srcs = [t.to(torch.int32) for t in srcs]
                indptr, indices, last = self._staging.upload(srcs, dev, dests)
            else:
                indptr, indices, last = [_as_device_int(t, torch.int32, dev) for t in srcs]
                if self.use_cuda_graph:
                    for d, s in zip(dests, (indptr, indices, last)):
                        if d.data_ptr() != s.data_ptr():
                            d[: s.shape[0]].copy_(s)
                    indptr, indices, last = dests

        if kv_cache_locations is not None:
            with trace_range(nv, "flashinfer.decode.kv_location_h2d"):
                loc = kv_cache_locations.to(dev, torch.long, non_blocking=True)
            if self.use_cuda_graph:
                with trace_range(nv, "flashinfer.decode.kv_location_copy"):
                    self.kv_cache_locations[:n_req].copy_(loc)
            else:
                self.kv_cache_locations = loc
            loc_out = None
        else:
            if not self.use_cuda_graph:
                self.kv_cache_locations = torch.empty(n_req, 2, dtype=torch.long, device=dev)
            loc_out = self.kv_cache_locations
        # the split-KV plan; the write locations (the reference's kv_location_compute) come out of the same launch
        with trace_range(nv, "flashinfer.decode.plan_inner"):
            _lib.check(
                _lib.lib().mi_decode_plan(
                    None, indptr.data_ptr(), indices.data_ptr(), last.data_ptr(), n_req, self.page_size,
                    self.num_qo_heads, self.num_kv_heads, self.head_dim,
                    loc_out.data_ptr() if loc_out is not None else None,
                    self._workspace.data_ptr(), self._workspace.numel() * self._workspace.element_size(),
                    _lib.stream_ptr(dev),
                ),
                "mi_decode_plan",
            )
        self._indptr, self._indices, self._last = indptr, indices, last
        self._n_req = n_req
        self.dtype = dtype

    def _adopt_plan(self, kv_indptr: torch.Tensor, kv_indices: torch.Tensor, last: torch.Tensor,
                    kv_cache_locations: torch.Tensor, dtype: torch.dtype) -> None:
        """Take a plan the caller already wrote into this wrapper's workspace
        (``mi_pack_plan``: the packed device arrays and the split-KV plan of
        one decode step), as if :meth:`plan` had been called with them."""
        n_req = kv_indptr.shape[0] - 1
        if self.use_cuda_graph:
            if n_req != self.batch_size:
                raise ValueError(f"CUDA-graph mode plans a fixed batch of {self.batch_size}, got {n_req}")
            statics = (self._paged_kv_indptr_buf, self._paged_kv_indices_buf, self._paged_kv_last_page_len_buf)
            if any(d.data_ptr() != t.data_ptr() for d, t in zip(statics, (kv_indptr, kv_indices, last))):
                raise ValueError("a graph-mode plan must be packed into the wrapper's static buffers")
            if kv_cache_locations.data_ptr() != self.kv_cache_locations.data_ptr():
                self.kv_cache_locations[:n_req].copy_(kv_cache_locations)
            kv_indptr, kv_indices, last = statics
        else:
            self.kv_cache_locations = kv_cache_locations
        self._indptr, self._indices, self._last = kv_indptr, kv_indices, last
        self._n_req = n_req
        self.dtype = dtype

    # --------------------------------------------------------------- run
    def run(self, q: torch.Tensor, kv_cache_layer: torch.Tensor, k_scale: torch.Tensor | None = None,
            v_scale: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Paged decode attention (``flashinfer_utils.py:455-465``): q ``[n_req, Hq, D]`` -> o."""
        if self.dtype is None:
            raise RuntimeError("plan() must be called before run()")
        if q.dtype != self.dtype:
            q = q.to(self.dtype)
        n = self._n_req
        if q.dim() != 3 or q.shape[0] < n or q.shape[1] != self.num_qo_heads or q.shape[2] != self.head_dim:
            raise ValueError(f"q shape {tuple(q.shape)} does not match the plan")
        if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
            q = q.contiguous()
        desc = _lib.paged_kv_desc(kv_cache_layer, k_scale, v_scale)
        if desc.num_kv_heads != self.num_kv_heads or desc.head_dim != self.head_dim or desc.page_size != self.page_size:
            raise ValueError("kv_cache_layer geometry does not match the wrapper")
        if out is None:
            out = torch.empty(q.shape[0], self.num_qo_heads, self.head_dim, dtype=q.dtype, device=q.device)
        qs = _q_strides(q, "q")
        os_ = _q_strides(out, "out")
        batch = n
        _lib.check(
            _lib.lib().mi_decode_run(
                q.data_ptr(), _lib.TORCH_TO_MI[q.dtype], qs[0], qs[1], desc, None, self._indptr.data_ptr(),
                self._indices.data_ptr(), self._last.data_ptr(), batch, self.num_qo_heads, 0,
                1.0 / math.sqrt(self.head_dim), self._workspace.data_ptr(),
                self._workspace.numel() * self._workspace.element_size(), out.data_ptr(), os_[0], os_[1],
                _lib.stream_ptr(q.device),
            ),
            "mi_decode_run",
        )
        return out

    def set_kv_cache(self, kv_cache_layer: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
        """Write one new token per request (``flashinfer_utils.py:467-484``)."""
        _append(kv_cache_layer, k, v, *self._append_target(), k_scale, v_scale)

    def _append_target(self):
        """(page ids, slot ids pointer, index stride, tokens, device token count) of this step's append."""
        loc = self.kv_cache_locations
        return loc, loc.data_ptr() + 8, 2, self._n_req, None


class PagedPrefillWrapper(_FusedRopeAppend):
    """Batched ragged paged prefill attention (``flashinfer_utils.py:70-288``)."""

    def __init__(
        self,
        workspace_buffer: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        batch_size: int | None = None,
        max_total_tokens: int | None = None,
        max_num_pages: int | None = None,
        device: torch.device = torch.device("cuda"),
        use_cuda_graph: bool = False,
        enable_nvtx: bool = False,
    ):
        _check_heads(num_qo_heads, num_kv_heads, head_dim, page_size)
        _lib.lib()
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.use_cuda_graph = use_cuda_graph
        self.enable_nvtx = enable_nvtx
        self.batch_size = batch_size
        self.max_total_tokens = max_total_tokens
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.dtype = None
        self.causal = True
        self._workspace = workspace_buffer
        self._staging = _Staging()
        # Side stream of run(): made here so that a run() under graph capture
        # only records the fork/join on it (creating a stream is not capturable).
        self._side = torch.cuda.Stream(device=self.device)
        self._n_req = 0
        if use_cuda_graph:
            assert batch_size is not None, "batch_size required for CUDA graph mode"
            assert max_total_tokens is not None, "max_total_tokens required for CUDA graph mode"
            assert max_num_pages is not None, "max_num_pages required for CUDA graph mode"
            d = self.device
            self._qo_indptr_buf = torch.zeros(batch_size + 1, dtype=torch.int32, device=d)
            self._paged_kv_indptr_buf = torch.zeros(batch_size + 1, dtype=torch.int32, device=d)
            self._paged_kv_indices_buf = torch.zeros(max_num_pages, dtype=torch.int32, device=d)
            self._paged_kv_last_page_len_buf = torch.ones(batch_size, dtype=torch.int32, device=d)
            self.token_to_page = torch.zeros(max_total_tokens, dtype=torch.long, device=d)
            self.token_to_cache = torch.zeros(max_total_tokens, dtype=torch.long, device=d)
        else:
            self.token_to_page = None
            self.token_to_cache = None
        self._total_tokens = 0

    def plan(
        self,
        qo_indptr: torch.Tensor,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        causal: bool = True,
        dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        """Token->page map and work partition on the GPU (``flashinfer_utils.py:162-256``).

        ``_total_tokens`` is read from ``qo_indptr[-1]``: free for CPU inputs,
        one device sync for device inputs (as the reference, ``:215``).
        """
        srcs = [qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len]
        on_cpu = all(t.device.type == "cpu" for t in srcs)
        total_tokens = int(qo_indptr[-1]) if on_cpu else int(qo_indptr[-1].item())
        self._plan(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, total_tokens, causal, dtype)

    def plan_device(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor, paged_kv_indices: torch.Tensor,
                    paged_kv_last_page_len: torch.Tensor, total_tokens: int, causal: bool = True,
                    dtype: torch.dtype = torch.bfloat16) -> None:
        """:meth:`plan` for device index tensors whose token count the caller knows (no sync)."""
        self._plan(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, total_tokens, causal, dtype)

    def _plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, total_tokens, causal,
              dtype) -> None:
        n_req = qo_indptr.shape[0] - 1
        if paged_kv_indptr.shape[0] != n_req + 1 or paged_kv_last_page_len.shape[0] != n_req:
            raise ValueError("index tensors disagree on the number of requests")
        dev = self.device
        self.dtype = dtype
        self.causal = bool(causal)
        srcs = [qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len]
        on_cpu = all(t.device.type == "cpu" for t in srcs)
        self._total_tokens = total_tokens
        if self.use_cuda_graph:
            if n_req != self.batch_size:  # captured launches bake the batch in
                raise ValueError(f"CUDA-graph mode plans a fixed batch of {self.batch_size}, got {n_req}")
            if total_tokens > self.max_total_tokens:
                raise ValueError(f"{total_tokens} tokens > max_total_tokens {self.max_total_tokens}")
            if paged_kv_indices.shape[0] > self._paged_kv_indices_buf.shape[0]:
                raise ValueError("paged_kv_indices exceeds max_num_pages")
            dests = [self._qo_indptr_buf, self._paged_kv_indptr_buf, self._paged_kv_indices_buf,
                     self._paged_kv_last_page_len_buf]
        else:
            dests = [None] * 4
        if on_cpu:
            qo, indptr, indices, last = self._staging.upload([t.to(torch.int32) for t in srcs], dev, dests)
        else:
            qo, indptr, indices, last = [_as_device_int(t, torch.int32, dev) for t in srcs]
            if self.use_cuda_graph:
                for d, s in zip(dests, (qo, indptr, indices, last)):
                    if d.data_ptr() != s.data_ptr():
                        d[: s.shape[0]].copy_(s)
                qo, indptr, indices, last = dests
        if not self.use_cuda_graph:
            self._qo_indptr_buf = qo
            self.token_to_page = torch.empty(total_tokens, dtype=torch.long, device=dev)
            self.token_to_cache = torch.empty(total_tokens, dtype=torch.long, device=dev)
        batch = n_req
        max_tokens = self.max_total_tokens if self.use_cuda_graph else total_tokens
        ws_bytes = self._workspace.numel() * self._workspace.element_size()
        _lib.check(
            _lib.lib().mi_prefill_plan(
                qo.data_ptr(), indptr.data_ptr(), indices.data_ptr(), last.data_ptr(), n_req, max_tokens,
                self.page_size, self.num_qo_heads, self.num_kv_heads, self.head_dim,
                self.token_to_page.data_ptr(), self.token_to_cache.data_ptr(), self.token_to_page.shape[0],
                self._workspace.data_ptr(), ws_bytes, _lib.stream_ptr(dev),
            ),
            "mi_prefill_plan",
        )
        self._qo, self._indptr, self._indices, self._last = qo, indptr, indices, last
        self._n_req = n_req
        self._plan_batch = batch
        self._plan_max_tokens = max_tokens
        # Which of run()'s two launches has work: known on the host for CPU
        # inputs outside graph mode; otherwise (a captured graph serves any
        # later mix, device inputs are not read back) both are launched, and
        # a launch without work exits at once.
        if on_cpu and not self.use_cuda_graph:
            # a request of at most `short` (token, q-head) rows goes to the split-KV
            # decode kernel (mi_prefill_short), a longer one to the MFMA tiles
            short = _lib.lib().mi_prefill_short_rows(n_req, self.num_qo_heads, self.num_kv_heads, self.head_dim)
            rows = torch.diff(qo_indptr.to(torch.int64)) * (self.num_qo_heads // self.num_kv_heads)
            self._run_short = bool(((rows > 0) & (rows <= short)).any())
            self._run_tiles = bool((rows > short).any())
        else:
            self._run_short = self._run_tiles = True

    def run(self, q: torch.Tensor, kv_cache_layer: torch.Tensor, k_scale: torch.Tensor | None = None,
            v_scale: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Ragged paged attention (``flashinfer_utils.py:258-269``): q ``[tokens, Hq, D]`` -> o."""
        if self.dtype is None:
            raise RuntimeError("plan() must be called before run()")
        if q.dtype != self.dtype:
            q = q.to(self.dtype)
        if q.dim() != 3 or q.shape[1] != self.num_qo_heads or q.shape[2] != self.head_dim:
            raise ValueError(f"q shape {tuple(q.shape)} does not match the wrapper")
        if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
            q = q.contiguous()
        desc = _lib.paged_kv_desc(kv_cache_layer, k_scale, v_scale)
        if desc.num_kv_heads != self.num_kv_heads or desc.head_dim != self.head_dim or desc.page_size != self.page_size:
            raise ValueError("kv_cache_layer geometry does not match the wrapper")
        if out is None:
            out = torch.empty(q.shape[0], self.num_qo_heads, self.head_dim, dtype=q.dtype, device=q.device)
        qs = _q_strides(q, "q")
        os_ = _q_strides(out, "out")
        ws_bytes = self._workspace.numel() * self._workspace.element_size()
        args = [q.data_ptr(), _lib.TORCH_TO_MI[q.dtype], qs[0], qs[1], desc, self._qo.data_ptr(),
                self._indptr.data_ptr(), self._indices.data_ptr(), self._last.data_ptr(), self._plan_batch,
                self._plan_max_tokens, self.num_qo_heads, 1 if self.causal else 0, 1.0 / math.sqrt(self.head_dim),
                self._workspace.data_ptr(), ws_bytes, out.data_ptr(), os_[0], os_[1], None]
        # The MFMA tiles (long-query requests) and the split-KV decode of the
        # short-query requests write disjoint rows: run the HBM-bound decode
        # on a side stream so it overlaps the compute-bound tiles.
        main = torch.cuda.current_stream(q.device)
        if self._run_tiles and self._run_short:
            side = self._side
            side.wait_stream(main)
            args[-1] = main.cuda_stream
            _lib.check(_lib.lib().mi_prefill_tiles(*args), "mi_prefill_tiles")
            args[-1] = side.cuda_stream
            _lib.check(_lib.lib().mi_prefill_short(*args), "mi_prefill_short")
            main.wait_stream(side)
        elif self._run_tiles or self._run_short:
            args[-1] = main.cuda_stream
            fn = "mi_prefill_tiles" if self._run_tiles else "mi_prefill_short"
            _lib.check(getattr(_lib.lib(), fn)(*args), fn)
        return out

    def set_kv_cache(self, kv_cache_layer: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
        """Scatter the planned tokens' K/V into their pages (``flashinfer_utils.py:271-288``)."""
        _append(kv_cache_layer, k, v, *self._append_target(), k_scale, v_scale)

    def _append_target(self):
        """(page ids, slot ids pointer, index stride, tokens, device token count) of this step's append."""
        n_dev = self._qo.data_ptr() + 4 * self._n_req  # qo_indptr[n_req]: real count on the device
        return self.token_to_page, self.token_to_cache.data_ptr(), 1, self._total_tokens, n_dev


# Reference names (mstar/utils/flashinfer_utils.py) for drop-in use.
FlashInferPrefillWrapper = PagedPrefillWrapper
FlashInferDecodeWrapper = PagedDecodeWrapper
