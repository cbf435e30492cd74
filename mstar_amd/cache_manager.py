"""BatchedCacheManager with GPU batch packing.

Keeps the methods M*'s model code calls on ``mstar.engine.cache_manager.
BatchedCacheManager`` (``cache_manager.py:56-881``): ``plan_attention``,
``run_attention``, ``plan_rope``, ``apply_rope``, ``plan_attention_batched_cfg``,
``plan_rope_batched_cfg``, ``snapshot_all``, ``set_layer_idx``, ``set_active_label(s)``,
``get_qo_indptr_buf``, ``advance_seq_len(s)``, ``set_custom_pos_advance``,
``flush_to_store``, plus the pre-planned-label fast path used by the CUDA-graph
runner (``_pre_planned_labels``, ``cache_manager.py:202-217``).  One method has
no reference counterpart: ``apply_rope_and_run_attention`` fuses the RoPE of
``apply_rope`` with the K/V append of ``run_attention`` into one kernel.

What changes is how a step is packed (``_plan_attention_impl``,
``cache_manager.py:229-424``).  The reference walks every request in Python,
re-flattens every page list into CPU tensors and lets the wrapper copy them to
the device.  Here the host only allocates pages (same FIFO allocator, same
batch order, same ``AllocationFailedError``), sends the pages allocated since
the last step to the device block table, and one GPU kernel (``mi_pack``)
builds ``qo_indptr``, ``kv_indptr``, ``kv_indices``, ``last_page_len`` and the
decode write locations.  The wrapper's ``plan()`` then builds its split-KV or
prefill partition on the GPU from those device tensors.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .kv_store import KVCacheConfig, KVRequestState, PagedAllocationManager, _host_step
from .paged_attention import PagedDecodeWrapper, PagedPrefillWrapper
from .rope import apply_llama31_rope_pos_ids_inplace, apply_rope_pos_ids_inplace, rope_positions
from .trace import trace_range

_LLAMA31_KEYS = ("low_freq_factor", "high_freq_factor", "old_context_len")


@contextlib.contextmanager
def _unsynced_on_error(states: list[KVRequestState]):
    """If planning fails between the allocation and the queued pack launch,
    the states' new pages may be marked as on the device without having
    reached the block table: mark them unsynced so the next step resends
    their whole page lists."""
    try:
        yield
    except BaseException:
        for st in states:
            st.pages_changed()
        raise


@dataclass
class _PlanState:
    """Per-label plan state (``cache_manager.py:9-37``)."""

    wrapper: PagedPrefillWrapper | PagedDecodeWrapper | None = None
    pos_ids: torch.Tensor | None = None
    seq_lens: list[int] | None = None
    write_store: bool = True
    custom_pos_advance: list[int] | None = None


class WorkspaceBufferManager:
    """One workspace buffer per label (``cache_manager.py:40-53``)."""

    def __init__(self, size: int, device):
        self.size = size
        self.device = device
        self.buffers: dict[str, torch.Tensor] = {}

    def get(self, label: str = "main") -> torch.Tensor:
        if label not in self.buffers:
            self.buffers[label] = torch.empty(self.size, dtype=torch.uint8, device=self.device)
        return self.buffers[label]


def _step_tensors(b: int, total_pages: int, decode: bool, device):
    """Fresh device outputs of one pack (qo_indptr, kv_indptr, kv_indices,
    last_page_len and, for decode steps, the int64 write locations), carved
    from one allocation at 256-byte aligned offsets."""
    al = lambda x: (x + 63) // 64 * 64  # int32 elements per 256 bytes
    n_loc = al(4 * b) if decode else 0
    o_qo = n_loc
    o_ip = o_qo + al(b + 1)
    o_last = o_ip + al(b + 1)
    o_idx = o_last + al(b)
    buf = torch.empty(o_idx + max(total_pages, 1), dtype=torch.int32, device=device)
    loc = buf[: 4 * b].view(torch.int64).view(b, 2) if decode else None
    return (buf[o_qo:o_qo + b + 1], buf[o_ip:o_ip + b + 1], buf[o_idx:o_idx + max(total_pages, 1)],
            buf[o_last:o_last + b], loc)


class BatchedCacheManager:
    """Batched paged attention for the requests of one step (``cache_manager.py:56``)."""

    def __init__(
        self,
        request_ids: list[str],
        active_labels_per_request: dict[str, str],
        kv_cache: torch.Tensor,
        alloc_manager: PagedAllocationManager,
        buffer_manager: WorkspaceBufferManager,
        kv_cache_config: KVCacheConfig,
        device,
        cuda_graph_plan_states: dict[str, _PlanState] | None = None,
        auto_write_store: bool = False,
        enable_nvtx: bool = False,
        kv_scales: torch.Tensor | None = None,
    ):
        """``kv_scales`` (extension): fp32 ``[num_layers, 2, num_kv_heads]`` per-head
        dequantisation scales of an fp8-e4m3 ``kv_cache``."""
        self.request_ids = request_ids
        self.active_labels = active_labels_per_request
        self.kv_cache = kv_cache
        self.alloc_manager = alloc_manager
        self.buffer_manager = buffer_manager
        self.kv_cache_config = kv_cache_config
        self.device = torch.device(device)
        self.layer_idx = 0
        self.enable_nvtx = enable_nvtx
        self.auto_write_store = auto_write_store
        self.kv_scales = kv_scales
        self._cuda_graph_mode = cuda_graph_plan_states is not None
        self._plan_states: dict[str, _PlanState] = cuda_graph_plan_states if cuda_graph_plan_states is not None else {}
        self._pre_planned_labels: set[str] = set()
        self._plan_done_event = None
        # step metadata uploads: the device's shared pinned staging pair (managers
        # are short-lived, one per batch in the reference engine)
        self._pack = _lib.uploader(self.device)
        self._states_cache: dict = {}
        if alloc_manager.block_table is None:
            raise ValueError("the allocation manager needs a device (block table) for GPU packing")

    # ------------------------------------------------------------ labels
    def _get_state(self, request_id: str, label: str | None = None) -> KVRequestState:
        label = label or self.active_labels.get(request_id, "main")
        return self.alloc_manager.get_state(request_id, label)

    def set_active_labels(self, labels: dict[str, str]) -> None:
        self.active_labels = labels

    def set_active_label(self, label: str) -> None:
        self.active_labels = {rid: label for rid in self.request_ids}

    def set_layer_idx(self, layer_idx: int) -> None:
        self.layer_idx = layer_idx

    def get_qo_indptr_buf(self, label: str = "main") -> torch.Tensor | None:
        ps = self._plan_states.get(label)
        if ps is None or ps.wrapper is None:
            return None
        return getattr(ps.wrapper, "_qo_indptr_buf", None)

    def _single_active_label(self) -> str:
        labels = list(self.active_labels.values())
        assert len(set(labels)) == 1, f"All active labels must be the same, got {labels}"
        return labels[0]

    # ------------------------------------------------------------ planning
    def plan_attention(self, seq_lens: list[int] | None = None, dtype: torch.dtype | None = None,
                       is_causal: bool = True, write_store: bool = True, label: str | None = None) -> None:
        """Allocate pages, pack the step on the GPU and plan the wrapper (``cache_manager.py:167-227``)."""
        nv = self.enable_nvtx
        with trace_range(nv, "cache.plan_attention"):
            effective = label if label is not None else self._single_active_label()
            if effective in self._pre_planned_labels:
                with trace_range(nv, "cache.plan_attention.skipped_pre_planned"):
                    self._pre_planned_labels.discard(effective)
                    ps = self._plan_states.get(effective)
                    if ps is not None:
                        ps.seq_lens = seq_lens
                        ps.write_store = write_store
                return
            self._plan_attention_impl(seq_lens, dtype, is_causal, write_store, effective)

    def _alloc_entries(self, entries: list[tuple[str, str]], seq_lens, states=None,
                       generation: int | None = None) -> np.ndarray:
        """FIFO allocation in batch order (``cache_manager.py:278-285``) and the pack
        kernel's input: per entry ``[slot | seq_len | new_len | num_pages | pages
        already on the device]``, followed by the pages not yet on the device.

        Raises AllocationFailedError before any kernel is launched."""
        n = len(entries)
        if len(seq_lens) != n:
            raise ValueError(f"{len(seq_lens)} seq_lens for {n} requests")
        if states is None:
            generation = self.alloc_manager.state_generation
            states = [self._get_state(rid, label) for rid, label in entries]
        am = self.alloc_manager
        if _host_step is not None and am.block_table is not None:
            return am.alloc_pack_meta(entries, states, seq_lens, generation)
        seq = np.array([st.seq_len for st in states], dtype=np.int64)
        sl = np.asarray(seq_lens, dtype=np.int64).reshape(n)
        self.alloc_manager.alloc_batch(entries, states, seq + sl, generation)
        slots, npg, old, new_pages = self.alloc_manager.block_table.prepare_meta(states)
        meta = np.empty((5, n), dtype=np.int32)
        meta[0] = slots
        meta[1] = seq
        meta[2] = sl
        meta[3] = npg
        meta[4] = old
        return np.concatenate([meta.reshape(-1), new_pages])

    def _label_states(self, label: str) -> tuple[list[tuple[str, str]], list[KVRequestState], int]:
        """Entries ``(rid, label)`` of every request, their state objects and the
        allocation manager's ``state_generation`` they were read at; kept while
        the request list and the allocation manager's states are unchanged."""
        am = self.alloc_manager
        key = tuple(self.request_ids)
        c = self._states_cache.get(label)
        gen = am.state_generation
        if c is not None and c[0] == gen and c[1] == key:
            return c[2], c[3], gen
        entries = [(rid, label) for rid in key]
        states = [am.get_state(rid, label) for rid in key]
        self._states_cache[label] = (gen, key, entries, states)
        return entries, states, gen

    def _launch_pack(self, meta: np.ndarray, qo, kv_indptr, kv_indices, last, loc, plan_wrapper=None,
                     total_pages: int | None = None) -> None:
        """One upload of the step's metadata + new pages, one pack kernel; with
        ``plan_wrapper`` (a decode wrapper, decode step) the same launch also
        writes that wrapper's split-KV plan (``mi_pack_plan``)."""
        b = qo.shape[0] - 1
        if total_pages is None:
            total_pages = int(meta[3 * b:4 * b].sum())
        bt = self.alloc_manager.block_table
        grid = max(1, min(256, (total_pages + 1023) // 1024))  # about one page per thread
        stream = _lib.stream_ptr(self.device)
        w = plan_wrapper
        ws = w._workspace if w is not None else None
        plan_args = (w.num_qo_heads if w is not None else 0, w.num_kv_heads if w is not None else 0,
                     w.head_dim if w is not None else 0, ws.data_ptr() if ws is not None else None,
                     ws.numel() * ws.element_size() if ws is not None else 0)
        loc_ptr = loc.data_ptr() if loc is not None else None
        ps = self.kv_cache_config.page_size
        if meta.size <= _lib.PACK_HOST_META_MAX:
            # a step whose metadata fits the kernel's argument (as given up to
            # PACK_HOST_META values, compact beyond): no copy to the device
            meta = np.ascontiguousarray(meta, dtype=np.int32)
            rc = bt.launch(lambda table: _lib.lib().mi_pack_plan_host(
                meta.ctypes.data, meta.size, b, table, bt.stride, ps, qo.data_ptr(), kv_indptr.data_ptr(),
                kv_indices.data_ptr(), last.data_ptr(), loc_ptr, grid, *plan_args, stream))
            if rc == _lib.MI_OK:
                return
            if rc != _lib.MI_ERR_UNSUPPORTED or meta.size <= _lib.PACK_HOST_META:
                _lib.check(rc, "mi_pack_plan_host")
            # too large for the argument: the metadata goes to the device below
        dmeta = self._pack.upload(meta)
        base = dmeta.data_ptr()

        def pack(table):
            args = [base, base + 4 * b, base + 8 * b, base + 12 * b, b, table, bt.stride, base + 16 * b,
                    base + 20 * b, ps, qo.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(), last.data_ptr(),
                    loc_ptr, grid]
            if w is None:
                _lib.check(_lib.lib().mi_pack(*args, stream), "mi_pack")
            else:
                _lib.check(_lib.lib().mi_pack_plan(*args, *plan_args, stream), "mi_pack_plan")

        bt.launch(pack)

    def _plan_attention_impl(self, seq_lens, dtype, is_causal, write_store, label) -> None:
        assert self.kv_cache is not None
        if dtype is None:
            dtype = torch.bfloat16 if self.kv_cache.dtype == torch.float8_e4m3fn else self.kv_cache.dtype
        cfg = self.kv_cache_config
        ps_ = cfg.page_size
        b = len(self.request_ids)
        nv = self.enable_nvtx
        # host side: FIFO allocation and the block-table delta (the reference builds its page lists here)
        entries, states, gen = self._label_states(label)
        with _unsynced_on_error(states):
            with trace_range(nv, "cache.plan_attention.build_lists"):
                meta = self._alloc_entries(entries, seq_lens, states, gen)
            total_pages = int(meta[3 * b:4 * b].sum())
            new_lens = meta[2 * b:3 * b]
            is_decode = bool((new_lens == 1).all())

            ps = self._plan_states.get(label)
            if ps is not None and ps.wrapper is not None:
                wrapper = ps.wrapper
            else:
                cls = PagedDecodeWrapper if is_decode else PagedPrefillWrapper
                wrapper = cls(
                    workspace_buffer=self.buffer_manager.get(label),
                    num_qo_heads=cfg.num_qo_heads,
                    num_kv_heads=cfg.num_kv_heads,
                    head_dim=cfg.head_dim,
                    page_size=ps_,
                    device=self.device,
                    enable_nvtx=self.enable_nvtx,
                )
                ps = _PlanState(wrapper=wrapper)
                self._plan_states[label] = ps

            # device: one upload of [slot | seq_len | new_len | num_pages], one pack kernel
            graph_static = isinstance(wrapper, PagedDecodeWrapper) and wrapper.use_cuda_graph
            graph_static_pf = isinstance(wrapper, PagedPrefillWrapper) and wrapper.use_cuda_graph
            if graph_static or graph_static_pf:
                qo = wrapper._qo_indptr_buf if graph_static_pf else torch.empty(b + 1, dtype=torch.int32, device=self.device)
                kv_indptr = wrapper._paged_kv_indptr_buf
                kv_indices = wrapper._paged_kv_indices_buf
                last = wrapper._paged_kv_last_page_len_buf
                if total_pages > kv_indices.shape[0]:
                    raise ValueError(f"{total_pages} pages > wrapper max_num_pages {kv_indices.shape[0]}")
                loc = None
                if is_decode:
                    loc = wrapper.kv_cache_locations if graph_static and b == wrapper.batch_size else \
                        torch.empty(b, 2, dtype=torch.long, device=self.device)
            else:
                qo, kv_indptr, kv_indices, last, loc = _step_tensors(b, total_pages, is_decode, self.device)
            fused = isinstance(wrapper, PagedDecodeWrapper) and is_decode and (not graph_static or b == wrapper.batch_size)
            # device side: one upload of the step's metadata and one pack launch (the reference's torch.tensor builds)
            with trace_range(nv, "cache.plan_attention.make_tensors"):
                self._launch_pack(meta, qo, kv_indptr, kv_indices, last, loc, plan_wrapper=wrapper if fused else None,
                                  total_pages=total_pages)
        self._last_pack = (qo, kv_indptr, kv_indices[:total_pages], last, loc)
        with trace_range(nv, "cache.plan_attention.wrapper_plan"):
            if fused:
                wrapper._adopt_plan(kv_indptr, kv_indices[:total_pages], last, loc, dtype)
            elif isinstance(wrapper, PagedDecodeWrapper):
                wrapper.plan(kv_indptr, kv_indices[:total_pages], last, kv_cache_locations=loc, dtype=dtype)
            else:
                wrapper.plan_device(qo, kv_indptr, kv_indices[:total_pages], last,
                                    total_tokens=int(meta[2 * b:3 * b].sum()), causal=is_causal, dtype=dtype)
        ps.seq_lens = list(seq_lens)
        ps.write_store = write_store

    # ------------------------------------------------------------ multi-label (CFG)
    def plan_attention_batched_cfg(self, labels: list[str], seq_lens: list[int], is_causal: bool = False,
                                   write_store: bool = False, dtype=torch.bfloat16,
                                   combined_label: str = "_cfg_batched") -> None:
        """One ragged batch over (label, request) pairs, label-major (``cache_manager.py:522-609``).

        Each (label, request) pair is one entry with its own pages; all
        entries are allocated in that order and packed by one GPU kernel,
        then planned on a fresh prefill wrapper under ``combined_label``.
        """
        assert self.kv_cache is not None
        cfg = self.kv_cache_config
        entries = [(rid, label) for label in labels for rid in self.request_ids]
        sls = [int(seq_lens[i]) for _ in labels for i in range(len(self.request_ids))]
        generation = self.alloc_manager.state_generation
        states = [self._get_state(rid, label) for rid, label in entries]
        with _unsynced_on_error(states):
            meta = self._alloc_entries(entries, sls, states, generation)
            n = len(entries)
            total_pages = int(meta[3 * n:4 * n].sum())
            qo = torch.empty(n + 1, dtype=torch.int32, device=self.device)
            kv_indptr = torch.empty(n + 1, dtype=torch.int32, device=self.device)
            kv_indices = torch.empty(max(total_pages, 1), dtype=torch.int32, device=self.device)
            last = torch.empty(n, dtype=torch.int32, device=self.device)
            self._launch_pack(meta, qo, kv_indptr, kv_indices, last, None)
        self._last_pack = (qo, kv_indptr, kv_indices[:total_pages], last, None)
        wrapper = PagedPrefillWrapper(
            workspace_buffer=self.buffer_manager.get(combined_label),
            num_qo_heads=cfg.num_qo_heads,
            num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim,
            page_size=cfg.page_size,
            device=self.device,
            enable_nvtx=self.enable_nvtx,
        )
        wrapper.plan_device(qo, kv_indptr, kv_indices[:total_pages], last, total_tokens=sum(sls),
                            causal=is_causal, dtype=dtype)
        self._plan_states[combined_label] = _PlanState(wrapper=wrapper, seq_lens=sls, write_store=write_store)

    def plan_rope_batched_cfg(self, labels: list[str], seq_lens: list[int],
                              per_label_pos_ids: dict[str, list[torch.Tensor]] | None = None,
                              combined_label: str = "_cfg_batched") -> None:
        """Position ids of the batched-CFG entries, label-major (``cache_manager.py:611-650``).

        A label with explicit position tensors takes their concatenation; the
        others count from each request's ``position_id_start`` for that label
        (expanded on the GPU).  A label given an empty list counts too.
        """
        b = len(self.request_ids)
        parts = []
        for label in labels:
            given = per_label_pos_ids.get(label) if per_label_pos_ids else None
            if given:
                parts.append(torch.cat([t.to(device=self.device, dtype=torch.long) for t in given]))
                continue
            meta = np.empty(2 * b + 1, dtype=np.int32)
            meta[0] = 0
            meta[1:b + 1] = np.cumsum(seq_lens, dtype=np.int64)
            meta[b + 1:] = [self._get_state(rid, label).position_id_start for rid in self.request_ids]
            n = int(meta[b]) if b else 0
            out = torch.empty(n, dtype=torch.long, device=self.device)
            if n:
                dev = self._pack.upload(meta)
                rope_positions(dev[: b + 1], dev[b + 1:], out, n)
            parts.append(out)
        self._plan_states[combined_label].pos_ids = parts[0] if len(parts) == 1 else torch.cat(parts)

    def snapshot_all(self, from_label: str, to_label: str, realloc: bool = False, write_store: bool = True) -> None:
        """Copy every request's KV history from one label to another (``cache_manager.py:840-870``).

        Same page bookkeeping as the reference (the destination keeps its
        first ``seq_len // page_size`` pages, grows to the source length,
        takes its seq_len and position start); the page copies of all
        requests and layers go to the GPU as one ``mi_copy_pages`` launch.
        """
        assert self.kv_cache is not None
        ps_ = self.kv_cache_config.page_size
        src, dst = [], []
        for rid in self.request_ids:
            from_state = self._get_state(rid, from_label)
            if realloc:
                self.alloc_manager.reset_label(rid, to_label)
            to_state = self._get_state(rid, to_label)
            start = to_state.seq_len // ps_
            self.alloc_manager.alloc(rid, to_label, seq_len=from_state.seq_len)
            to_state.seq_len = from_state.seq_len
            to_state.position_id_start = from_state.position_id_start
            a, b = from_state.page_indices[start:], to_state.page_indices[start:]
            if len(a) != len(b):
                raise ValueError(f"{rid}: {len(a)} source pages vs {len(b)} destination pages from page {start}")
            src.extend(a)
            dst.extend(b)
            if write_store:
                self.alloc_manager.flush_to_store(rid, label=to_label)
        if src:
            kv = self.kv_cache
            page = kv[0, 0]
            if not page.is_contiguous():
                raise ValueError("snapshot_all needs each page of the KV pool to be contiguous")
            esz = kv.element_size()
            n = len(src)
            dev = self._pack.upload(np.asarray(src + dst, dtype=np.int32))
            _lib.check(
                _lib.lib().mi_copy_pages(
                    kv.data_ptr(), kv.stride(0) * esz, kv.shape[0], kv.stride(1) * esz, page.numel() * esz,
                    kv.shape[1], dev.data_ptr(), dev.data_ptr() + 4 * n, n, _lib.stream_ptr(self.device),
                ),
                "mi_copy_pages",
            )

    # ------------------------------------------------------------ running
    def _layer_scales(self, layer_idx: int):
        if self.kv_scales is None:
            return None, None
        return self.kv_scales[layer_idx, 0], self.kv_scales[layer_idx, 1]

    def run_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      layer_idx: int | None = None) -> torch.Tensor:
        """Append this step's K/V, then attend (``cache_manager.py:653-701``)."""
        if layer_idx is None:
            layer_idx = self.layer_idx
        orig_dtype = q.dtype
        label = self._single_active_label()
        ps = self._plan_states[label]
        assert self.kv_cache is not None and ps.wrapper is not None
        layer = self.kv_cache[layer_idx]
        ks, vs = self._layer_scales(layer_idx)
        ps.wrapper.set_kv_cache(layer, k, v, ks, vs)
        if self.auto_write_store and ps.write_store:
            for rid in self.request_ids:
                self.alloc_manager.flush_to_store(rid, label=label, layers=layer_idx)
        return ps.wrapper.run(q, layer, ks, vs).to(orig_dtype)

    # ------------------------------------------------------------ rope
    def plan_rope(self, seq_lens: list[int], pos_ids: torch.Tensor | None = None, label: str | None = None) -> None:
        """Position ids for ``apply_rope`` (``cache_manager.py:426-520``).

        Without ``pos_ids``, request r contributes ``position_id_start[r] ..
        + seq_lens[r] - 1``; the list is expanded on the GPU from one small
        upload (cumulative lengths + starts) instead of a Python list of every
        token.  In CUDA-graph mode an existing ``pos_ids`` buffer is rewritten
        in place so captured launches keep their address.
        """
        nv = self.enable_nvtx
        with trace_range(nv, "cache.plan_rope"):
            eff = label if label is not None else self._single_active_label()
            ps = self._plan_states.get(eff)
            if ps is None:
                ps = self._plan_states[eff] = _PlanState()
            if pos_ids is not None:
                with trace_range(nv, "cache.plan_rope.copy_pos_ids"):
                    src = pos_ids.to(device=self.device, dtype=torch.long)
                    if self._cuda_graph_mode and ps.pos_ids is not None:
                        ps.pos_ids[: src.shape[0]].copy_(src, non_blocking=True)
                    else:
                        ps.pos_ids = src
                return
            b = len(self.request_ids)
            if len(seq_lens) != b:
                raise ValueError(f"{len(seq_lens)} seq_lens for {b} requests")
            with trace_range(nv, "cache.plan_rope.build_pos_ids"):
                meta = np.empty(2 * b + 1, dtype=np.int32)
                meta[0] = 0
                meta[1:b + 1] = np.cumsum(seq_lens, dtype=np.int64)
                meta[b + 1:] = [self._get_state(rid, eff).position_id_start for rid in self.request_ids]
            n = int(meta[b]) if b else 0
            if self._cuda_graph_mode and ps.pos_ids is not None:
                if ps.pos_ids.shape[0] < n:
                    raise ValueError(f"{n} positions do not fit the static pos_ids buffer ({ps.pos_ids.shape[0]})")
                out = ps.pos_ids
            else:
                out = torch.empty(n, dtype=torch.long, device=self.device)
            if n:
                # the positions are expanded on the device from one small upload
                with trace_range(nv, "cache.plan_rope.copy_pos_ids"):
                    dev = self._pack.upload(meta)
                    rope_positions(dev[: b + 1], dev[b + 1:], out, n)
            ps.pos_ids = out

    def apply_rope(self, q: torch.Tensor, k: torch.Tensor, rotary_dim: int | None = None, interleave: bool = False,
                   rope_scale: float = 1, rope_theta: float = 10000.0, rope_dtype=None, **kwargs):
        """RoPE at the active label's planned positions (``cache_manager.py:702-760``).

        Same dtype handling as the reference: ``rope_dtype`` if given, else the
        autocast dtype, else fp32 inputs run in bf16; q and k are rotated in
        place in that dtype and returned in the caller's dtype.  Llama-3.1
        smoothing applies when any of ``low_freq_factor``,
        ``high_freq_factor``, ``old_context_len`` is passed (not None).
        """
        label = self._single_active_label()
        ps = self._plan_states[label]
        assert ps.pos_ids is not None, "plan_rope() must run before apply_rope()"
        orig_dtype = q.dtype
        if rope_dtype is not None:
            q, k = q.to(rope_dtype), k.to(rope_dtype)
        elif torch.is_autocast_enabled("cuda"):
            dt = torch.get_autocast_dtype("cuda")
            q, k = q.to(dt), k.to(dt)
        elif q.dtype == torch.float32:
            q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
        llama31 = {key: v for key, v in kwargs.items() if key in _LLAMA31_KEYS and v is not None}
        if llama31:
            apply_llama31_rope_pos_ids_inplace(q, k, ps.pos_ids, rotary_dim=rotary_dim, interleave=interleave,
                                               rope_scale=rope_scale, rope_theta=rope_theta, **llama31)
        else:
            apply_rope_pos_ids_inplace(q, k, ps.pos_ids, rotary_dim=rotary_dim, interleave=interleave,
                                       rope_scale=rope_scale, rope_theta=rope_theta)
        return q.to(orig_dtype), k.to(orig_dtype)

    def apply_rope_and_run_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                     rotary_dim: int | None = None, interleave: bool = False, rope_scale: float = 1,
                                     rope_theta: float = 10000.0, rope_dtype=None, layer_idx: int | None = None,
                                     keep_k: bool = True, **kwargs) -> torch.Tensor:
        """``apply_rope(q, k, ...)`` then ``run_attention(q, k, v)`` with the rotation and the append fused.

        One ``mi_rope_append`` launch rotates q (and k, unless ``keep_k`` is
        False) and writes the rotated k and v to the layer's pages; the cache
        and the attention output are bit-identical to the two-call sequence.
        Dtype handling and Llama-3.1 keywords are those of ``apply_rope``; v
        is converted to the rope dtype with q and k.
        """
        if layer_idx is None:
            layer_idx = self.layer_idx
        label = self._single_active_label()
        ps = self._plan_states[label]
        assert ps.pos_ids is not None, "plan_rope() must run before apply_rope_and_run_attention()"
        assert self.kv_cache is not None and ps.wrapper is not None
        orig_dtype = q.dtype
        dt = rope_dtype
        if dt is None and torch.is_autocast_enabled("cuda"):
            dt = torch.get_autocast_dtype("cuda")
        if dt is None and q.dtype == torch.float32:
            dt = torch.bfloat16
        if dt is not None:
            q, k, v = q.to(dt), k.to(dt), v.to(dt)
        elif v.dtype != k.dtype:
            v = v.to(k.dtype)
        llama31 = {key: val for key, val in kwargs.items() if key in _LLAMA31_KEYS and val is not None}
        if llama31:  # apply_llama31_rope_pos_ids_inplace defaults for the factors not given
            llama31 = {"low_freq_factor": 1.0, "high_freq_factor": 4.0, "old_context_len": 8192, **llama31}
        layer = self.kv_cache[layer_idx]
        ks, vs = self._layer_scales(layer_idx)
        ps.wrapper.rope_set_kv_cache(layer, q, k, v, ps.pos_ids, rotary_dim=rotary_dim, interleave=interleave,
                                     rope_scale=rope_scale, rope_theta=rope_theta, k_scale=ks, v_scale=vs,
                                     keep_k=keep_k, llama31=llama31 or None)
        if self.auto_write_store and ps.write_store:
            for rid in self.request_ids:
                self.alloc_manager.flush_to_store(rid, label=label, layers=layer_idx)
        return ps.wrapper.run(q, layer, ks, vs).to(orig_dtype)

    # ------------------------------------------------------------ advance
    def advance_seq_len(self, n: int | None = None, pos_id_n: int | None = None) -> None:
        if n is None:
            return self.advance_seq_lens(pos_id_n)
        for rid in self.request_ids:
            st = self._get_state(rid)
            st.seq_len += n
            st.position_id_start += pos_id_n if pos_id_n is not None else n

    def set_custom_pos_advance(self, pos_advance: list[int] | None, label: str | None = None) -> None:
        if label is None:
            labels = list(self.active_labels.values())
            if not labels:
                return
            assert len(set(labels)) == 1, f"All active labels must be the same to omit ``label``, got {labels}"
            label = labels[0]
        ps = self._plan_states.get(label)
        if ps is not None:
            ps.custom_pos_advance = list(pos_advance) if pos_advance is not None else None

    def advance_seq_lens(self, pos_id_ns: list[int] | int | None = None) -> None:
        """``seq_len += seq_lens[i]`` per request (``cache_manager.py:811-838``)."""
        labels = set(self.active_labels[rid] for rid in self.request_ids)
        if len(labels) == 1 and pos_id_ns is None:  # one label, default advance: one pass over the states
            label = labels.pop()
            ps = self._plan_states[label]
            _, states, _ = self._label_states(label)
            if _host_step is not None:
                _host_step.advance(states, ps.seq_lens, ps.custom_pos_advance)
            else:
                adv = ps.custom_pos_advance if ps.custom_pos_advance is not None else ps.seq_lens
                for st, n, a in zip(states, ps.seq_lens, adv):
                    st.seq_len += n
                    st.position_id_start += a
            for ps in self._plan_states.values():
                ps.custom_pos_advance = None
            return
        for i, rid in enumerate(self.request_ids):
            ps = self._plan_states[self.active_labels[rid]]
            n = ps.seq_lens[i]
            st = self._get_state(rid)
            st.seq_len += n
            if pos_id_ns is None:
                st.position_id_start += ps.custom_pos_advance[i] if ps.custom_pos_advance is not None else n
            elif isinstance(pos_id_ns, int):
                st.position_id_start += pos_id_ns
            else:
                st.position_id_start += pos_id_ns[i]
        for ps in self._plan_states.values():
            ps.custom_pos_advance = None

    def flush_to_store(self) -> None:
        for rid in self.request_ids:
            for label in self.alloc_manager.request_states[rid]:
                ps = self._plan_states.get(label)
                if ps is None or not ps.write_store:
                    continue
                self.alloc_manager.flush_to_store(rid, label)
