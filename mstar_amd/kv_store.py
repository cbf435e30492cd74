"""Host page allocator, per-request KV state and the device block table.

Host side mirrors M*'s ``mstar/engine/kv_store.py``:

* :class:`PageAllocator` — FIFO free list (``kv_store.py:25-67``): pages start
  in order ``0..N-1``, allocation pops from the head, ``free`` appends to the
  tail.  Page ids therefore depend on batch order exactly as in the reference.
* :class:`KVCacheConfig`, :class:`KVRequestState`, :class:`AllocationFailedError`
  (``kv_store.py:70-154``).
* :class:`PagedAllocationManager` — the subset of ``kv_store.py:394-614`` that
  the attention path uses (``alloc``, ``get_state``, ``add_request``,
  ``remove_request``, ``reset_label``).  Remote transfer engines, CPU offload
  and the distributed store are outside this library.

Device side (new): :class:`DeviceBlockTable` keeps a copy of every request's
page list in HBM (``int32 [slots, max_pages_per_seq]``).  Only pages allocated
since the previous step are sent (one small host->device copy plus one
scatter kernel), so the GPU packing kernel (``mi_pack``) can flatten the batch
without the reference's per-step re-flattening of every page list on the host
(``cache_manager.py:288``).
"""

from __future__ import annotations

import collections
import threading
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib


class PageAllocator:
    """Thread-safe FIFO page allocator (``kv_store.py:25-67``)."""

    def __init__(self, max_num_pages: int):
        self.max_num_pages = max_num_pages
        self.free_pages: collections.deque[int] = collections.deque(range(max_num_pages))
        self._lock = threading.Lock()

    def allocate(self, n: int) -> list[int]:
        with self._lock:
            if len(self.free_pages) < n:
                raise RuntimeError(
                    f"Not enough free pages: requested {n}, available {len(self.free_pages)}"
                )
            return [self.free_pages.popleft() for _ in range(n)]

    def try_allocate(self, n: int) -> list[int] | None:
        """Like :meth:`allocate` but returns None instead of raising."""
        with self._lock:
            if len(self.free_pages) < n:
                return None
            return [self.free_pages.popleft() for _ in range(n)]

    def free(self, pages: list[int]) -> None:
        with self._lock:
            self.free_pages.extend(pages)

    @property
    def num_free(self) -> int:
        return len(self.free_pages)


@dataclass
class KVCacheConfig:
    """KV cache geometry (``kv_store.py:70-101``)."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    max_seq_len: int
    max_num_pages: int = 2048
    page_size: int = 128
    num_qo_heads: int | None = None
    cpu_offload_pages: int = 0
    nodes: list[str] | None = None

    def __post_init__(self):
        if self.num_qo_heads is None:
            self.num_qo_heads = self.num_kv_heads
        self._sharded = False
        self.original_num_kv_heads = self.num_kv_heads
        self.original_num_qo_heads = self.num_qo_heads

    def shard(self, tp_size: int):
        """Head sharding for tensor parallelism (``kv_store.py:95-101``)."""
        if tp_size >= self.original_num_kv_heads:
            self.num_kv_heads = 1
        else:
            if self.original_num_kv_heads % tp_size:
                raise ValueError(f"{self.original_num_kv_heads} kv heads do not split over {tp_size}")
            self.num_kv_heads = self.original_num_kv_heads // tp_size
        if self.original_num_qo_heads % tp_size:
            raise ValueError(f"{self.original_num_qo_heads} q heads do not split over {tp_size}")
        self.num_qo_heads = self.original_num_qo_heads // tp_size
        self._sharded = True


@dataclass
class KVRequestState:
    """Per-request, per-label KV state (``kv_store.py:111-127``).

    ``slot`` is this state's row in the :class:`DeviceBlockTable` (-1: none yet).
    """

    page_indices: list[int] = field(default_factory=list)
    seq_len: int = 0
    position_id_start: int = 0
    read_in_progress: bool = False
    is_paused: bool = False
    slot: int = -1
    _dev_list: object = field(default=None, repr=False, compare=False)
    _dev_len: int = field(default=0, repr=False, compare=False)


class AllocationFailedError(RuntimeError):
    """Page pool too small for a request (``kv_store.py:133-154``)."""

    def __init__(self, pages_short: int, request_id: str, label: str, message: str | None = None):
        super().__init__(
            message
            or f"Page allocation failed: {pages_short} page(s) short for request {request_id!r} label {label!r}"
        )
        self.pages_short = pages_short
        self.request_id = request_id
        self.label = label


class DeviceBlockTable:
    """HBM copy of the page lists of live request states.

    ``table[slot, p]`` is page ``p`` of the state that owns ``slot``.  States
    get a slot the first time they are synced; :meth:`release` returns it.
    :meth:`sync` sends only what changed since the previous sync: appended
    pages, or the whole list if the state's list object was replaced or
    shortened.
    """

    def __init__(self, max_pages_per_seq: int, device: torch.device, max_slots: int = 256):
        self.device = torch.device(device)
        self.stride = int(max_pages_per_seq)
        self.table = torch.zeros(max_slots, self.stride, dtype=torch.int32, device=self.device)
        self._free_slots = list(range(max_slots - 1, -1, -1))
        self._lock = threading.Lock()
        self._staging: torch.Tensor | None = None
        self._staging_event: torch.cuda.Event | None = None

    @property
    def max_slots(self) -> int:
        return self.table.shape[0]

    def _grow(self) -> None:
        old = self.table
        new_slots = old.shape[0] * 2
        self.table = torch.zeros(new_slots, self.stride, dtype=torch.int32, device=self.device)
        self.table[: old.shape[0]].copy_(old)
        self._free_slots = list(range(new_slots - 1, old.shape[0] - 1, -1)) + self._free_slots

    def acquire(self, state: KVRequestState) -> int:
        with self._lock:
            if state.slot < 0:
                if not self._free_slots:
                    self._grow()
                state.slot = self._free_slots.pop()
                state._dev_list = None
                state._dev_len = 0
            return state.slot

    def release(self, state: KVRequestState) -> None:
        with self._lock:
            if state.slot >= 0:
                self._free_slots.append(state.slot)
                state.slot = -1
                state._dev_list = None
                state._dev_len = 0

    def prepare(self, states: list[KVRequestState]) -> tuple[np.ndarray, np.ndarray]:
        """What ``mi_pack`` must add to the table for ``states``: per state the
        number of leading pages already on the device, and all the other pages
        concatenated in order.  The caller hands both to the pack kernel, which
        writes them into the table; the states are marked as synced."""
        old = np.empty(len(states), dtype=np.int32)
        parts = []
        for i, st in enumerate(states):
            self.acquire(st)
            pl = st.page_indices
            n = len(pl)
            if n > self.stride:
                raise ValueError(f"request holds {n} pages, block table rows hold {self.stride}")
            start = st._dev_len if (st._dev_list is pl and n >= st._dev_len) else 0
            old[i] = start
            if n > start:
                parts.append(pl[start:])
            st._dev_list = pl
            st._dev_len = n
        new = np.fromiter((p for part in parts for p in part), dtype=np.int32) if parts else np.zeros(0, np.int32)
        return old, new

    def sync(self, states: list[KVRequestState], stream: torch.cuda.Stream | None = None) -> None:
        """Bring the device rows of ``states`` up to date (async on ``stream``)."""
        slots, poss, pages = [], [], []
        for st in states:
            slot = self.acquire(st)
            pl = st.page_indices
            n = len(pl)
            if n > self.stride:
                raise ValueError(f"request holds {n} pages, block table rows hold {self.stride}")
            start = st._dev_len if (st._dev_list is pl and n >= st._dev_len) else 0
            if n > start:
                slots.append(np.full(n - start, slot, dtype=np.int32))
                poss.append(np.arange(start, n, dtype=np.int32))
                pages.append(np.asarray(pl[start:], dtype=np.int32))
            st._dev_list = pl
            st._dev_len = n
        if not slots:
            return
        upd = np.concatenate([np.concatenate(slots), np.concatenate(poss), np.concatenate(pages)])
        m = upd.size // 3
        dev = self._upload(upd, stream)
        st_ptr = (stream or torch.cuda.current_stream(self.device)).cuda_stream
        base = dev.data_ptr()
        _lib.check(
            _lib.lib().mi_block_table_update(
                self.table.data_ptr(), self.stride, base, base + 4 * m, base + 8 * m, m, st_ptr
            ),
            "mi_block_table_update",
        )

    def _upload(self, arr: np.ndarray, stream) -> torch.Tensor:
        """Async H2D of a small int32 array through a reused pinned buffer."""
        n = arr.size
        if self._staging is None or self._staging.numel() < n:
            self._staging = torch.empty(max(n, 4096), dtype=torch.int32, pin_memory=True)
            self._staging_event = None
        if self._staging_event is not None:
            self._staging_event.synchronize()  # previous copy out of the staging buffer is done
        self._staging[:n].numpy()[:] = arr
        s = stream or torch.cuda.current_stream(self.device)
        with torch.cuda.stream(s):
            dev = torch.empty(n, dtype=torch.int32, device=self.device)
            dev.copy_(self._staging[:n], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(s)
        self._staging_event = ev
        return dev


class PagedAllocationManager:
    """Page allocation and per-request state (``kv_store.py:394-614``, attention subset).

    ``device`` enables the :class:`DeviceBlockTable` used by the GPU packer.
    """

    def __init__(self, config: KVCacheConfig, kv_cache: torch.Tensor | None = None,
                 device: torch.device | str | None = None):
        self.config = config
        self.page_allocator = PageAllocator(config.max_num_pages)
        self.request_states: dict[str, dict[str, KVRequestState]] = {}
        self.kv_cache = kv_cache
        self.pending_reads: dict[str, dict[str, list]] = {}
        self._lock = threading.RLock()
        if device is None and kv_cache is not None and kv_cache.is_cuda:
            device = kv_cache.device
        self.block_table: DeviceBlockTable | None = None
        if device is not None:
            max_pages_per_seq = (config.max_seq_len + config.page_size - 1) // config.page_size
            self.block_table = DeviceBlockTable(max_pages_per_seq, torch.device(device))

    @property
    def num_free_pages(self) -> int:
        return self.page_allocator.num_free

    @property
    def total_pages(self) -> int:
        return self.config.max_num_pages

    def flush_to_store(self, request_id: str, label: str, layers=None):
        """No-op, as in the reference (``kv_store.py:445-451``)."""
        return

    def _new_state(self) -> KVRequestState:
        return KVRequestState()

    def get_state(self, request_id: str, label: str) -> KVRequestState:
        if label not in self.request_states[request_id]:
            self.request_states[request_id][label] = self._new_state()
        return self.request_states[request_id][label]

    def alloc(self, request_id: str, label: str, seq_len: int) -> None:
        """Grow the state's page list to ``ceil(seq_len / page_size)`` pages (``kv_store.py:463-482``)."""
        with self._lock:
            state = self.request_states[request_id][label]
            ps = self.config.page_size
            num_new = (seq_len + ps - 1) // ps - len(state.page_indices)
            if num_new > 0:
                new_pages = self.page_allocator.try_allocate(num_new)
                if new_pages is None:
                    raise AllocationFailedError(
                        pages_short=num_new - self.page_allocator.num_free,
                        request_id=request_id,
                        label=label,
                        message=(
                            f"Not enough free pages: requested {num_new}, "
                            f"available {self.page_allocator.num_free}"
                        ),
                    )
                state.page_indices.extend(new_pages)

    def get_labels(self, request_id: str) -> list[str]:
        return list(self.request_states[request_id].keys())

    def reset_label(self, request_id: str, label: str, free: bool = True) -> None:
        with self._lock:
            old = self.request_states[request_id].get(label)
            if old is not None:
                if free:
                    self.page_allocator.free(old.page_indices)
                if self.block_table is not None:
                    self.block_table.release(old)
            self.request_states[request_id][label] = self._new_state()

    def add_request(self, request_id: str, labels: list[str] | None = None) -> None:
        labels = labels or []
        with self._lock:
            self.request_states[request_id] = {label: self._new_state() for label in labels}
            self.pending_reads[request_id] = {label: [] for label in labels}

    def remove_request(self, request_id: str) -> None:
        with self._lock:
            for state in self.request_states[request_id].values():
                self.page_allocator.free(state.page_indices)
                if self.block_table is not None:
                    self.block_table.release(state)
            del self.request_states[request_id]
            del self.pending_reads[request_id]
