"""Host page allocator, per-request KV state and the device block table.

Host side mirrors M*'s ``mstar/engine/kv_store.py``:

* :class:`PageAllocator` — FIFO free list (``kv_store.py:25-67``): pages start
  in order ``0..N-1``, allocation pops from the head, ``free`` appends to the
  tail.  Page ids therefore depend on batch order exactly as in the reference.
* :class:`KVCacheConfig`, :class:`PositionInfo`, :class:`KVRequestState`,
  :class:`AllocationFailedError`, :class:`TransferEngineInfo`,
  :class:`StoreWritePolicy` (``kv_store.py:70-175``).
* :class:`PagedAllocationManager` — ``kv_store.py:394-660``: allocation and
  request state (``alloc``, ``get_state``, ``add_request``, ``remove_request``,
  ``reset_label``), remote reads (``start_async_retrieve``, ``sync_retrieve``,
  ``check_retrieve_ready``, ``get_per_label_seq_info``, through
  :class:`mstar_amd.kv_transfer.DeviceKVTransferEngine`) and CPU offload
  (``offload_request`` / ``reload_request`` with
  :class:`mstar_amd.kv_transfer.CPUPagePool`).  The Mooncake/RDMA transport
  and the distributed store are outside this library; a transport moves
  the buffers of :func:`mstar_amd.kv_transfer.pack_wire`.

Device side (new): :class:`DeviceBlockTable` keeps a copy of every request's
page list in HBM (``int32 [slots, max_pages_per_seq]``).  Only pages allocated
since the previous step are sent (one small host->device copy plus one
scatter kernel), so the GPU packing kernel (``mi_pack``) can flatten the batch
without the reference's per-step re-flattening of every page list on the host
(``cache_manager.py:288``).
"""

from __future__ import annotations

import collections
import enum
import threading
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from . import _lib

try:  # the planning step's per-request loops in C (csrc/host_step.c); the Python loops below specify them
    from . import _host_step
except ImportError:  # not built yet
    _host_step = None


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

    def get_node_str(self) -> str:
        """Key of this cache among an engine's caches (``kv_store.py:90-93``):
        the node names joined by ``///``, or ``ALL_NODES`` when the config
        lists none."""
        if self.nodes is None:
            return "ALL_NODES"
        return "///".join(self.nodes)

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
class PositionInfo:
    """What a model's ``prepare_inputs`` reads of one label (``kv_store.py:105-108``)."""

    full_seq_len: int = 0
    position_id_start: int = 0


@dataclass
class KVRequestState:
    """Per-request, per-label KV state (``kv_store.py:111-127``).

    ``slot`` is this state's row in the :class:`DeviceBlockTable` (-1: none yet).

    Page-list contract (what the reference's code paths do): ``page_indices``
    only grows by ``append``/``extend``, or is replaced by a new list object.
    The block table sends a grown list's new tail and a replaced list whole;
    it also resends the whole list when the first page or the page last synced
    no longer sits where it was, which catches edits in place of those entries
    (``page_indices[:] = ...``).  Other in-place edits must be followed by
    :meth:`pages_changed`.
    """

    page_indices: list[int] = field(default_factory=list)
    seq_len: int = 0
    position_id_start: int = 0
    read_in_progress: bool = False
    is_paused: bool = False
    slot: int = -1
    _dev_list: object = field(default=None, repr=False, compare=False)
    _dev_len: int = field(default=0, repr=False, compare=False)
    _dev_ends: tuple = field(default=(-1, -1), repr=False, compare=False)

    def get_pos_info(self) -> PositionInfo:
        """Sequence length and first position id (``kv_store.py:123-127``)."""
        return PositionInfo(full_seq_len=self.seq_len, position_id_start=self.position_id_start)

    def pages_changed(self) -> None:
        """Mark ``page_indices`` as edited in place: the next sync resends all of it."""
        self._dev_list = None
        self._dev_len = 0


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


@dataclass
class TransferEngineInfo:
    """The worker's tensor transport, as the engine hands it to the
    allocation manager (``kv_store.py:164-168``)."""

    my_entity_id: str
    my_session_id: str
    transfer_engine: Any


class StoreWritePolicy(enum.Enum):
    """Whether a worker's KV may be read elsewhere (``kv_store.py:171-174``)."""

    ALWAYS = "always"
    NEVER = "never"


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
        self._retired: list[torch.Tensor] = []
        self._lock = threading.Lock()
        self._staging: torch.Tensor | None = None
        self._staging_event: torch.cuda.Event | None = None

    @property
    def max_slots(self) -> int:
        return self.table.shape[0]

    def _grow(self) -> None:
        """Double the table (called with ``_lock`` held).  Every launch that
        reads or writes the table takes ``_lock`` from reading
        ``table.data_ptr()`` until the launch is queued (:meth:`launch`), so
        no launch can pick up the old table after this swap; launches queued
        before it are drained by the device synchronisation before the copy,
        and the copy itself by the one after it.  The old tensor is kept
        (``_retired``) until the table is dropped, so even a launch made
        outside that protocol cannot write into memory handed out again.
        Growth only happens when more states are live than the table has
        rows (it starts at ``max_slots``), never under graph capture
        (planning is not captured)."""
        old = self.table
        on_gpu = self.device.type == "cuda"
        if on_gpu:
            torch.cuda.synchronize(self.device)
        new_slots = old.shape[0] * 2
        table = torch.zeros(new_slots, self.stride, dtype=torch.int32, device=self.device)
        table[: old.shape[0]].copy_(old)
        if on_gpu:
            torch.cuda.synchronize(self.device)
        self._retired.append(old)
        self.table = table
        self._free_slots = list(range(new_slots - 1, old.shape[0] - 1, -1)) + self._free_slots

    def launch(self, fn):
        """``fn(table_ptr)`` with the table lock held: for the kernels that
        read or write the table, so the pointer they get stays the live table
        until they are queued (see :meth:`_grow`)."""
        with self._lock:
            return fn(self.table.data_ptr())

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

    @staticmethod
    def _synced_prefix(st: KVRequestState, pl: list, n: int) -> int:
        """Leading pages of ``pl`` that the device row already holds: the
        synced length when ``pl`` is the synced list object, at least as long
        as then, with its first page and its last synced page unchanged;
        otherwise 0 (the whole list is sent)."""
        m = st._dev_len
        if st._dev_list is not pl or n < m:
            return 0
        if m and (pl[0], pl[m - 1]) != st._dev_ends:
            return 0
        return m

    @staticmethod
    def _mark_synced(st: KVRequestState, pl: list, n: int) -> None:
        st._dev_list = pl
        st._dev_len = n
        st._dev_ends = (pl[0], pl[n - 1]) if n else (-1, -1)

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
            start = self._synced_prefix(st, pl, n)
            old[i] = start
            if n > start:
                parts.append(pl[start:])
            self._mark_synced(st, pl, n)
        new = np.fromiter((p for part in parts for p in part), dtype=np.int32) if parts else np.zeros(0, np.int32)
        return old, new

    def prepare_meta(self, states: list[KVRequestState]):
        """:meth:`prepare` plus each state's slot and page count:
        ``(slots, num_pages, old, new)``, int32 arrays."""
        slots, npg, old, parts = [], [], [], []
        stride = self.stride
        for st in states:
            if st.slot < 0:
                self.acquire(st)
            pl = st.page_indices
            n = len(pl)
            if st._dev_list is pl and n == st._dev_len and (not n or (pl[0], pl[n - 1]) == st._dev_ends):
                start = n  # nothing new (most requests of a decode step)
            else:
                if n > stride:
                    raise ValueError(f"request holds {n} pages, block table rows hold {stride}")
                start = self._synced_prefix(st, pl, n)
                if n > start:
                    parts.append(pl[start:])
                self._mark_synced(st, pl, n)
            slots.append(st.slot)
            npg.append(n)
            old.append(start)
        new = np.fromiter((p for part in parts for p in part), dtype=np.int32) if parts else np.zeros(0, np.int32)
        return (np.array(slots, dtype=np.int32), np.array(npg, dtype=np.int32), np.array(old, dtype=np.int32),
                new)

    def sync(self, states: list[KVRequestState], stream: torch.cuda.Stream | None = None) -> None:
        """Bring the device rows of ``states`` up to date (async on ``stream``).
        If the update cannot be queued, the states are marked unsynced again."""
        slots, poss, pages = [], [], []
        try:
            for st in states:
                slot = self.acquire(st)
                pl = st.page_indices
                n = len(pl)
                if n > self.stride:
                    raise ValueError(f"request holds {n} pages, block table rows hold {self.stride}")
                start = self._synced_prefix(st, pl, n)
                if n > start:
                    slots.append(np.full(n - start, slot, dtype=np.int32))
                    poss.append(np.arange(start, n, dtype=np.int32))
                    pages.append(np.asarray(pl[start:], dtype=np.int32))
                self._mark_synced(st, pl, n)
            if not slots:
                return
            upd = np.concatenate([np.concatenate(slots), np.concatenate(poss), np.concatenate(pages)])
            m = upd.size // 3
            dev = self._upload(upd, stream)
            st_ptr = (stream or torch.cuda.current_stream(self.device)).cuda_stream
            base = dev.data_ptr()
            self.launch(lambda table: _lib.check(
                _lib.lib().mi_block_table_update(table, self.stride, base, base + 4 * m, base + 8 * m, m, st_ptr),
                "mi_block_table_update"))
        except BaseException:
            for st in states:
                st.pages_changed()
            raise

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
    """Page allocation and per-request state (``kv_store.py:394-660``).

    Constructed as the reference engine constructs it
    (``kv_cache_engine.py:150-157``: ``config``, ``kv_cache``,
    ``transfer_engine_info``).  The transport in ``transfer_engine_info``
    selects the KV reader the way ``kv_store.py:413-426`` does:

    * ``None``, the reference's ``LocalTransferEngine``, or any transport
      whose ``get_async_reader(device)`` returns None (single node: the
      producer's pool is device-addressable) -> a
      :class:`mstar_amd.kv_transfer.DeviceKVTransferEngine` over ``kv_cache``,
      built on first use;
    * an object that already is a KV reader (has ``read_pages_async``) ->
      used as it is;
    * anything else, e.g. the Mooncake RDMA transport, -> ``ValueError``, as
      the reference raises for a transport it does not support: cross-node
      RDMA page reads are outside this library (a transport can move the
      buffers of :func:`mstar_amd.kv_transfer.pack_wire` instead).

    Keyword extensions: ``device`` places the :class:`DeviceBlockTable` the
    GPU packer reads (default: ``kv_cache``'s device when it is a GPU
    tensor); ``transfer_engine`` passes a KV reader directly.
    """

    def __init__(self, config: KVCacheConfig, kv_cache: torch.Tensor | None = None,
                 transfer_engine_info: TransferEngineInfo | None = None, *,
                 device: torch.device | str | None = None, transfer_engine=None):
        self.config = config
        if transfer_engine is None and transfer_engine_info is not None:
            transfer_engine = self._reader_for(transfer_engine_info, kv_cache)
        self._kv_transfer_engine = transfer_engine
        self.page_allocator = PageAllocator(config.max_num_pages)
        self.request_states: dict[str, dict[str, KVRequestState]] = {}
        self.kv_cache = kv_cache
        self.write_policy = StoreWritePolicy.ALWAYS
        self.pending_reads: dict[str, dict[str, list]] = {}
        self._lock = threading.RLock()
        # Bumped whenever a state object is created or a request removed, so
        # callers can keep lists of state objects between steps.
        self.state_generation = 0
        if device is None and kv_cache is not None and kv_cache.is_cuda:
            device = kv_cache.device
        self.block_table: DeviceBlockTable | None = None
        if device is not None:
            max_pages_per_seq = (config.max_seq_len + config.page_size - 1) // config.page_size
            self.block_table = DeviceBlockTable(max_pages_per_seq, torch.device(device))

    @staticmethod
    def _reader_for(info: TransferEngineInfo, kv_cache: torch.Tensor | None):
        """The KV reader for ``info.transfer_engine`` (None: build the device
        reader on first use); see the class docstring."""
        te = info.transfer_engine
        if te is None:
            return None
        if hasattr(te, "read_pages_async"):
            return te
        if type(te).__name__ == "LocalTransferEngine":
            return None
        reader = getattr(te, "get_async_reader", None)
        if reader is not None and reader(kv_cache.device if kv_cache is not None else None) is None:
            return None
        raise ValueError(
            f"Unsupported transfer engine type: {type(te)} (remote page reads over RDMA are outside this "
            "library; single-node transports and device-addressable pools are supported)")

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
        self.state_generation += 1
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

    def alloc_pack_meta(self, entries: list[tuple[str, str]], states: list[KVRequestState], seq_lens,
                        generation: int | None = None) -> np.ndarray:
        """:meth:`alloc_batch` to ``seq_len + seq_lens[i]`` followed by the block
        table's :meth:`DeviceBlockTable.prepare_meta`, in the host_step extension:
        the pack kernel's int32 input ``[slot | seq_len | new_len | num_pages |
        pages on the device]`` (one entry per state each) followed by the pages
        not yet on the device.  Same allocation order, errors and state
        updates as the two Python methods."""
        hs = _host_step
        bt = self.block_table
        sl = list(seq_lens)
        with self._lock:
            if generation is None or generation != self.state_generation:
                for i, (rid, label) in enumerate(entries):
                    live = self.get_state(rid, label)
                    if live is not states[i]:
                        states[i] = live
            total, need = hs.needs(states, sl, self.config.page_size)
            pages = None
            if total:
                pages = self.page_allocator.try_allocate(total)
                if pages is None:  # entry by entry: the first that does not fit raises, earlier ones keep theirs
                    for i in np.flatnonzero(np.frombuffer(need, dtype=np.int32) > 0).tolist():
                        self.alloc(entries[i][0], entries[i][1], states[i].seq_len + int(sl[i]))
            meta = hs.extend_meta(states, sl, need, pages, bt.stride, bt.acquire)
        return np.frombuffer(meta, dtype=np.int32)

    def alloc_batch(self, entries: list[tuple[str, str]], states: list[KVRequestState],
                    seq_lens_after: np.ndarray, generation: int | None = None) -> None:
        """``alloc(rid, label, seq_lens_after[i])`` for every entry, in order.

        ``states[i]`` is the caller's state object for ``entries[i]``, looked
        up when ``state_generation`` read ``generation``.  If a state was
        replaced or removed since (another thread's ``reset_label`` or
        ``remove_request``), the live state is looked up under the lock, as
        ``alloc`` does, and written back into ``states``, so pages never go to
        a state that is no longer the request's.  When the free list holds
        every page the batch needs, the pages are taken in one pass and handed
        out in entry order, which is what the sequential calls would give;
        otherwise the entries are allocated one by one, so the first one that
        does not fit raises ``AllocationFailedError`` with the earlier ones
        holding their pages, as in the reference.
        """
        ps = self.config.page_size
        with self._lock:
            if generation is None or generation != self.state_generation:
                for i, (rid, label) in enumerate(entries):
                    live = self.get_state(rid, label)
                    if live is not states[i]:
                        states[i] = live
            npg = np.array([len(st.page_indices) for st in states], dtype=np.int64)
            need = (np.asarray(seq_lens_after, dtype=np.int64) + ps - 1) // ps - npg
            idx = np.flatnonzero(need > 0).tolist()
            if not idx:
                return
            pages = self.page_allocator.try_allocate(int(need[idx].sum()))
            if pages is None:
                for i in idx:
                    self.alloc(entries[i][0], entries[i][1], int(seq_lens_after[i]))
                return
            off = 0
            for i in idx:
                k = int(need[i])
                states[i].page_indices.extend(pages[off:off + k])
                off += k

    def get_labels(self, request_id: str) -> list[str]:
        return list(self.request_states[request_id].keys())

    def reset_label(self, request_id: str, label: str, free: bool = True) -> None:
        self.wait_for_retrieves(request_id, label)
        with self._lock:
            old = self.request_states[request_id].get(label)
            if old is not None:
                if free:
                    self.page_allocator.free(old.page_indices)
                if self.block_table is not None:
                    self.block_table.release(old)
            self.request_states[request_id][label] = self._new_state()

    def cleanup(self) -> None:
        """Shut the KV reader down at engine shutdown (``kv_store.py:592-593``):
        reads still in flight land first."""
        if self._kv_transfer_engine is not None:
            self._kv_transfer_engine.shutdown()

    def add_request(self, request_id: str, labels: list[str] | None = None) -> None:
        labels = labels or []
        with self._lock:
            self.request_states[request_id] = {label: self._new_state() for label in labels}
            self.pending_reads[request_id] = {label: [] for label in labels}

    def remove_request(self, request_id: str) -> None:
        for label in self.request_states[request_id]:
            self.wait_for_retrieves(request_id, label)
        with self._lock:
            for state in self.request_states[request_id].values():
                self.page_allocator.free(state.page_indices)
                if self.block_table is not None:
                    self.block_table.release(state)
            del self.request_states[request_id]
            del self.pending_reads[request_id]
            self.state_generation += 1

    # ----- remote reads (kv_store.py:484-581) -----

    @property
    def kv_transfer_engine(self):
        """The engine remote reads go through; built over ``kv_cache`` on first use."""
        if self._kv_transfer_engine is None:
            from .kv_transfer import DeviceKVTransferEngine

            if self.kv_cache is None:
                raise RuntimeError("remote KV reads need the manager's kv_cache")
            self._kv_transfer_engine = DeviceKVTransferEngine(self.kv_cache)
        return self._kv_transfer_engine

    def _settle_reads(self, request_id: str, label: str, block: bool) -> bool:
        """Forget the finished reads of (request, label); with ``block``, wait
        for all of them first.  Keeps the state's ``read_in_progress`` equal to
        "a read is still outstanding" and returns True when none is."""
        per_label = self.pending_reads.get(request_id)
        futures = per_label.get(label, []) if per_label is not None else []
        if block:
            for f in futures:
                f.result()
            left = []
        else:
            left = [f for f in futures if not f.done()]
        if per_label is not None:
            per_label[label] = left
        state = self.request_states.get(request_id, {}).get(label)
        if state is not None:
            state.read_in_progress = bool(left)
        return not left

    def wait_for_retrieves(self, request_id: str, label: str) -> None:
        """Block until every read into (request, label) has landed (``kv_store.py:484-491``)."""
        self._settle_reads(request_id, label, block=True)

    def check_retrieve_ready(self, request_id: str, label: str) -> bool:
        """True once every read of (request, label) has finished (``kv_store.py:493-509``)."""
        if not self.get_state(request_id, label).read_in_progress:
            return True
        return self._settle_reads(request_id, label, block=False)

    def sync_retrieve(self, request_id: str, label: str, seq_info) -> None:
        self.start_async_retrieve(request_id, label, seq_info)
        self.wait_for_retrieves(request_id, label)

    def start_async_retrieve(self, request_id: str, label: str, seq_info) -> None:
        """Read the producer's tokens [local seq_len, seq_info.seq_len) (``kv_store.py:515-566``).

        Same page and token ranges as the reference; all layers of all pages
        go out as one launch on the engine's transfer stream.  The producer
        must have finished writing those pages (the reference's contract,
        ``kv_store.py:548-554``).
        """
        seq_len = seq_info.seq_len
        state = self.get_state(request_id, label)
        if state.seq_len >= seq_len:
            return
        ps = self.config.page_size
        first = state.seq_len // ps
        last = (seq_len - 1) // ps
        self.alloc(request_id, label, seq_len)
        n = last - first + 1
        ts = np.zeros(n, np.int64)
        ts[0] = state.seq_len % ps
        te = np.full(n, ps, np.int64)
        te[-1] = seq_len % ps or ps
        local = np.asarray(state.page_indices[first:last + 1], dtype=np.int64)
        remote = np.asarray(seq_info.page_indices[first:last + 1], dtype=np.int64)
        if remote.size != n:
            raise ValueError(f"producer lists {len(seq_info.page_indices)} pages for {seq_len} tokens")
        future = self.kv_transfer_engine.read_pages_async(seq_info.latest_kv_transfer_info, local, remote, ts, te)
        if future is not None:
            self.pending_reads[request_id].setdefault(label, []).append(future)
        state.seq_len = seq_len
        state.position_id_start = seq_info.pos_id
        state.read_in_progress = future is not None

    def get_per_label_seq_info(self, request_id: str) -> dict:
        """What a consumer needs to read every label of a request (``kv_store.py:568-581``)."""
        from .kv_transfer import SequenceInfo

        info = self.kv_transfer_engine.get_kv_transfer_info()
        out = {}
        for label in list(self.request_states.get(request_id, {})):
            self.wait_for_retrieves(request_id, label)
            st = self.get_state(request_id, label)
            out[label] = SequenceInfo(seq_len=st.seq_len, pos_id=st.position_id_start,
                                      latest_kv_transfer_info=info, page_indices=st.page_indices)
        return out

    # ----- CPU offloading (kv_store.py:617-660) -----

    def offload_request(self, request_id: str, cpu_pool) -> int:
        """Move every label of a request that holds pages to ``cpu_pool`` and
        give its GPU pages back (``kv_store.py:617-644``); returns the number
        of GPU pages freed.

        Per label: reads into it land first, its copy is queued (the pool makes
        the caller's stream wait for the copy, so the freed pages cannot be
        overwritten before they are read), then its pages return to the FIFO
        tail in list order and the state empties.  A label the CPU pool has no
        room for is not recorded there, and its GPU pages are freed anyway, as
        in the reference.  The manager lock is held only for the bookkeeping,
        never while waiting on reads or queueing copies, so a plan thread can
        keep allocating meanwhile.
        """
        with self._lock:
            holding = [(label, st) for label, st in self.request_states[request_id].items() if st.page_indices]
        freed = 0
        for label, st in holding:
            self.wait_for_retrieves(request_id, label)
            cpu_pool.offload_pages(request_id, label, self.kv_cache, st.page_indices, st.seq_len,
                                   st.position_id_start)
            with self._lock:
                pages, st.page_indices, st.seq_len = st.page_indices, [], 0
                self.page_allocator.free(pages)
            freed += len(pages)
        return freed

    def reload_request(self, request_id: str, cpu_pool) -> None:
        """Bring every offloaded label of a request back into fresh GPU pages
        (``kv_store.py:646-660``).

        The pages of all labels are taken from the free list in one call and
        dealt out in label order, which gives each label the page ids the
        reference's label-by-label allocation gives.  A pool too small for the
        whole request raises ``RuntimeError`` before any label changes (the
        reference raises at the first label that does not fit, after
        reloading the ones before it).  One copy per label goes to the pool's
        stream; the caller's stream waits for all of them at the end.
        """
        with self._lock:
            held = cpu_pool.offloaded.get(request_id, {})
            labels = list(held)
            counts = [len(held[label].cpu_page_indices) for label in labels]
            pages = self.page_allocator.allocate(sum(counts))
            start = 0
            for label, n in zip(labels, counts):
                mine = pages[start:start + n]
                start += n
                st = self.get_state(request_id, label)
                seq_len, pos = cpu_pool.reload_pages(request_id, label, self.kv_cache, mine)
                st.page_indices, st.seq_len, st.position_id_start = mine, seq_len, pos
        cpu_pool.sync()
