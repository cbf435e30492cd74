"""KV page transfer on the GPU: remote reads, CPU offload/reload, wire format.

Mirrors the transfer side of M*'s KV store:

* :class:`KVReadInfo`, :class:`SequenceInfo` (``mstar/engine/kv_store.py:177-183``,
  ``mstar/conductor/request_info.py:23-29``);
* :class:`DeviceKVTransferEngine` — the ``KVTransferEngine`` interface
  (``kv_store.py:186-200``: ``read_batched_async``, ``get_kv_transfer_info``,
  ``shutdown``) for a producer pool the device can address directly (another
  pool on this GPU, or a peer GPU's pool opened through an IPC handle).  The
  reference's ``CudaIpcKVTransferEngine._do_read`` (``kv_store.py:330-380``)
  runs one torch copy per ``KVReadInfo`` on a host thread; here the whole list
  is one ``mi_kv_copy_tokens`` launch on a transfer stream, and the returned
  future is an event;
* :class:`CPUPagePool` (``mstar/engine/cpu_page_pool.py:25-150``) — same
  API; offload and reload are one launch each that reads or writes the pinned
  host pool directly, instead of one copy per page;
* :func:`pack_wire` / :func:`unpack_wire` — a contiguous, layer-major wire
  buffer of the same records, for transports that move one buffer (the
  reference's Mooncake path issues one transfer per (layer, page, K|V)
  segment, ``kv_store.py:261-285``).

Semantics of a read follow ``MooncakeKVTransferEngine._get_ptr_nbytes``
(``kv_store.py:233-259``): tokens ``[token_start, token_end)`` of both the K
and the V half of (layer, page).  (``CudaIpcKVTransferEngine._do_read`` slices
``tensor[layer, page, token_start:token_end]``, which indexes the K/V axis of
the ``[L, P, 2, ps, H, D]`` pool rather than the token axis; that is not
reproduced.)
"""

from __future__ import annotations

import ctypes
import logging
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from . import _lib
from .kv_store import KVCacheConfig, PageAllocator

logger = logging.getLogger(__name__)


@dataclass
class KVReadInfo:
    """One (layer, page) read (``kv_store.py:177-183``)."""

    layer_idx: int
    local_page_idx: int
    remote_page_idx: int
    token_start: int
    token_end: int


@dataclass
class DeviceKVTransferInfo:
    """What a consumer needs to address a producer's pool (plain values, picklable)."""

    data_ptr: int
    size: tuple
    stride: tuple
    dtype: str
    device: int


@dataclass
class SequenceInfo:
    """A producer's state of one (request, label) (``request_info.py:23-29``)."""

    seq_len: int
    pos_id: int
    latest_kv_transfer_info: Any
    page_indices: list[int] = field(default_factory=list)


def _check_pool(kv: torch.Tensor, name: str) -> None:
    if kv.dim() != 6 or kv.shape[2] != 2:
        raise ValueError(f"{name} must be [layers, pages, 2, page_size, num_kv_heads, head_dim], got {tuple(kv.shape)}")
    if kv.stride(5) != 1 or kv.stride(4) != kv.shape[5] or kv.stride(3) != kv.shape[4] * kv.shape[5]:
        raise ValueError(f"{name}: the token rows (num_kv_heads * head_dim) must be contiguous")
    if not (kv.is_cuda or kv.is_pinned()):
        raise ValueError(f"{name} must be a device tensor or pinned host memory")


def transfer_info(kv: torch.Tensor) -> DeviceKVTransferInfo:
    _check_pool(kv, "kv_cache")
    dev = kv.device.index if kv.is_cuda else -1
    return DeviceKVTransferInfo(kv.data_ptr(), tuple(kv.shape), tuple(kv.stride()), str(kv.dtype), dev)


def pool_desc(info: DeviceKVTransferInfo | torch.Tensor) -> _lib.MiKvPool:
    """``mi_kv_pool`` of a whole pool ``[layers, pages, 2, ps, H, D]``."""
    if isinstance(info, torch.Tensor):
        info = transfer_info(info)
    es = torch.empty(0, dtype=getattr(torch, info.dtype.split(".")[-1])).element_size()
    d = _lib.MiKvPool()
    d.data = info.data_ptr
    d.layer_stride = info.stride[0] * es
    d.page_stride = info.stride[1] * es
    d.kv_stride = info.stride[2] * es
    d.token_stride = info.stride[3] * es
    d.num_pages = info.size[1]
    d.num_layers = info.size[0]
    d.page_size = info.size[3]
    return d


class _Records:
    """Page-level records uploaded as one int32 array (+ int64 row offsets)."""

    def __init__(self, device, dst_pages, src_pages, token_start, token_end, page_size: int, stream,
                 num_pages: tuple[int, int], want_offsets: bool = False):
        dst = np.asarray(dst_pages, dtype=np.int64).reshape(-1)
        src = np.asarray(src_pages, dtype=np.int64).reshape(-1) if src_pages is not None else dst
        self.n = dst.size
        if src.size != self.n:
            raise ValueError("page lists differ in length")
        full = token_start is None
        if full != (token_end is None):
            raise ValueError("give both token_start and token_end, or neither")
        ts = np.zeros(self.n, np.int64) if full else np.asarray(token_start, dtype=np.int64).reshape(-1)
        te = np.full(self.n, page_size, np.int64) if full else np.asarray(token_end, dtype=np.int64).reshape(-1)
        if ts.size != self.n or te.size != self.n:
            raise ValueError("token ranges must have one entry per record")
        if self.n and ((ts < 0).any() or (te > page_size).any() or (te <= ts).any()):
            raise ValueError(f"token ranges must satisfy 0 <= token_start < token_end <= {page_size}")
        for arr, lim, what in ((dst, num_pages[0], "destination"), (src, num_pages[1], "source")):
            if self.n and (arr.min() < 0 or arr.max() >= lim):
                raise IndexError(f"{what} page id out of range [0, {lim})")
        self.rows = int((te - ts).sum())
        parts = [dst, src] + ([] if full else [ts, te])
        host = torch.from_numpy(np.concatenate(parts).astype(np.int32)).pin_memory()
        with torch.cuda.stream(stream):
            self.dev = host.to(device, non_blocking=True)
            self.off = None
            if want_offsets and not full:
                off = np.concatenate([[0], np.cumsum(te - ts)]).astype(np.int64)
                self.off = torch.from_numpy(off).pin_memory().to(device, non_blocking=True)
        self._host = host  # keep the pinned source alive until the copy has run
        self.full = full

    def ptr(self, k: int):
        """Device address of part ``k`` (0 dst, 1 src, 2 ts, 3 te)."""
        if k >= 2 and self.full:
            return None
        return self.dev.data_ptr() + 4 * k * self.n

    @property
    def off_ptr(self):
        return None if self.off is None else self.off.data_ptr()


def _stream_of(device: torch.device, stream: torch.cuda.Stream | None) -> torch.cuda.Stream:
    return stream if stream is not None else torch.cuda.current_stream(device)


def copy_tokens(src: DeviceKVTransferInfo | torch.Tensor, dst: torch.Tensor, dst_pages, src_pages,
                token_start=None, token_end=None, layer_begin: int = 0, layer_end: int | None = None,
                stream: torch.cuda.Stream | None = None, device: torch.device | None = None) -> None:
    """One launch: for every record and layer, dst rows [ts, te) := src rows (K and V)."""
    sinfo = src if isinstance(src, DeviceKVTransferInfo) else transfer_info(src)
    dinfo = transfer_info(dst)
    if sinfo.dtype != dinfo.dtype or tuple(sinfo.size[2:]) != tuple(dinfo.size[2:]):
        raise ValueError("source and destination pools differ in dtype or page shape")
    layer_end = dinfo.size[0] if layer_end is None else layer_end
    if not (0 <= layer_begin <= layer_end <= min(dinfo.size[0], sinfo.size[0])):
        raise ValueError("layer range outside the pools")
    if device is None:
        device = dst.device if dst.is_cuda else torch.device("cuda", sinfo.device)
    s = _stream_of(device, stream)
    rec = _Records(device, dst_pages, src_pages, token_start, token_end, dinfo.size[3], s,
                   (dinfo.size[1], sinfo.size[1]))
    if rec.n == 0 or layer_end == layer_begin:
        return
    sd, dd = pool_desc(sinfo), pool_desc(dinfo)
    _lib.check(
        _lib.lib().mi_kv_copy_tokens(ctypes.byref(sd), ctypes.byref(dd), rec.ptr(1), rec.ptr(0), rec.ptr(2),
                                     rec.ptr(3), rec.n, layer_begin, layer_end, s.cuda_stream),
        "mi_kv_copy_tokens",
    )
    rec.dev.record_stream(s)


def wire_nbytes(kv: torch.Tensor, num_rows: int, layer_begin: int = 0, layer_end: int | None = None) -> int:
    """Bytes of a wire buffer holding ``num_rows`` token rows per layer (K and V each)."""
    layer_end = kv.shape[0] if layer_end is None else layer_end
    return 2 * num_rows * (layer_end - layer_begin) * kv.stride(3) * kv.element_size()


def pack_wire(kv: torch.Tensor, pages, token_start=None, token_end=None, layer_begin: int = 0,
              layer_end: int | None = None, out: torch.Tensor | None = None,
              stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Gather records of ``kv`` into a contiguous uint8 wire buffer (layer-major)."""
    info = transfer_info(kv)
    layer_end = info.size[0] if layer_end is None else layer_end
    if not (0 <= layer_begin <= layer_end <= info.size[0]):
        raise ValueError("layer range outside the pool")
    device = kv.device if kv.is_cuda else torch.device("cuda")
    s = _stream_of(device, stream)
    rec = _Records(device, pages, None, token_start, token_end, info.size[3], s, (info.size[1], info.size[1]),
                   want_offsets=True)
    nbytes = wire_nbytes(kv, rec.rows, layer_begin, layer_end)
    if out is None:
        with torch.cuda.stream(s):
            out = torch.empty(nbytes, dtype=torch.uint8, device=device)
    elif out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < nbytes:
        raise ValueError(f"out must be a contiguous uint8 buffer of at least {nbytes} bytes")
    if rec.n and layer_end > layer_begin:
        d = pool_desc(info)
        _lib.check(
            _lib.lib().mi_kv_wire_pack(ctypes.byref(d), rec.ptr(0), rec.ptr(2), rec.ptr(3), rec.off_ptr, rec.n,
                                       layer_begin, layer_end, out.data_ptr(), out.numel(), s.cuda_stream),
            "mi_kv_wire_pack",
        )
        rec.dev.record_stream(s)
        if rec.off is not None:
            rec.off.record_stream(s)
    return out[:nbytes]


def unpack_wire(wire: torch.Tensor, kv: torch.Tensor, pages, token_start=None, token_end=None,
                layer_begin: int = 0, layer_end: int | None = None,
                stream: torch.cuda.Stream | None = None) -> None:
    """Scatter a wire buffer written by :func:`pack_wire` into ``kv``'s pages."""
    info = transfer_info(kv)
    layer_end = info.size[0] if layer_end is None else layer_end
    if not (0 <= layer_begin <= layer_end <= info.size[0]):
        raise ValueError("layer range outside the pool")
    if wire.dtype != torch.uint8 or not wire.is_contiguous() or not (wire.is_cuda or wire.is_pinned()):
        raise ValueError("wire must be a contiguous uint8 device (or pinned host) buffer")
    device = kv.device if kv.is_cuda else wire.device
    s = _stream_of(device, stream)
    rec = _Records(device, pages, None, token_start, token_end, info.size[3], s, (info.size[1], info.size[1]),
                   want_offsets=True)
    need = wire_nbytes(kv, rec.rows, layer_begin, layer_end)
    if wire.numel() < need:
        raise ValueError(f"wire holds {wire.numel()} bytes, the records need {need}")
    if rec.n and layer_end > layer_begin:
        d = pool_desc(info)
        _lib.check(
            _lib.lib().mi_kv_wire_unpack(wire.data_ptr(), wire.numel(), ctypes.byref(d), rec.ptr(0), rec.ptr(2),
                                         rec.ptr(3), rec.off_ptr, rec.n, layer_begin, layer_end, s.cuda_stream),
            "mi_kv_wire_unpack",
        )
        rec.dev.record_stream(s)
        if rec.off is not None:
            rec.off.record_stream(s)


class TransferFuture:
    """Completion of an asynchronous transfer: an event on the transfer stream."""

    def __init__(self, event: torch.cuda.Event):
        self._event = event

    def done(self) -> bool:
        return self._event.query()

    def result(self, timeout=None):
        self._event.synchronize()
        return None


class DeviceKVTransferEngine:
    """``KVTransferEngine`` over device-addressable pools (``kv_store.py:186-200``).

    ``read_batched_async`` orders the read after the work already queued on
    the caller's current stream (as the reference's read waits on an event
    recorded there, ``kv_store.py:335-345``) and runs it on the engine's own
    transfer stream.
    """

    def __init__(self, kv_cache: torch.Tensor, stream: torch.cuda.Stream | None = None):
        _check_pool(kv_cache, "kv_cache")
        if not kv_cache.is_cuda:
            raise ValueError("kv_cache must be a device tensor")
        self._kv_cache = kv_cache
        self._device = kv_cache.device
        self._stream = stream or torch.cuda.Stream(device=self._device)
        self._transfer_info = transfer_info(kv_cache)

    def get_kv_transfer_info(self) -> DeviceKVTransferInfo:
        return self._transfer_info

    def read_pages_async(self, remote_kv_info: DeviceKVTransferInfo, local_pages, remote_pages, token_start=None,
                         token_end=None, layer_begin: int = 0, layer_end: int | None = None) -> TransferFuture | None:
        """Page-level records for a layer range: one launch."""
        if len(local_pages) == 0:
            return None
        self._stream.wait_stream(torch.cuda.current_stream(self._device))
        copy_tokens(remote_kv_info, self._kv_cache, local_pages, remote_pages, token_start, token_end,
                    layer_begin, layer_end, stream=self._stream, device=self._device)
        ev = torch.cuda.Event()
        ev.record(self._stream)
        return TransferFuture(ev)

    def read_batched_async(self, remote_kv_info: DeviceKVTransferInfo,
                           read_info: list[KVReadInfo]) -> TransferFuture | None:
        """The reference's per-(layer, page) list (``kv_store.py:330-345``).

        Records that cover every layer of the pool (what ``start_async_retrieve``
        produces) go out in one launch; other records in one launch per layer.
        """
        if not read_info:
            return None
        num_layers = self._kv_cache.shape[0]
        by_rec: dict[tuple, set] = {}
        for r in read_info:
            by_rec.setdefault((r.local_page_idx, r.remote_page_idx, r.token_start, r.token_end), set()).add(r.layer_idx)
        groups: dict[tuple, list] = {}
        for key, layers in by_rec.items():
            if len(layers) == num_layers and min(layers) == 0 and max(layers) == num_layers - 1:
                groups.setdefault((0, num_layers), []).append(key)
            else:
                for layer in sorted(layers):
                    groups.setdefault((layer, layer + 1), []).append(key)
        self._stream.wait_stream(torch.cuda.current_stream(self._device))
        for (lb, le), keys in groups.items():
            arr = np.asarray(keys, dtype=np.int64)
            copy_tokens(remote_kv_info, self._kv_cache, arr[:, 0], arr[:, 1], arr[:, 2], arr[:, 3], lb, le,
                        stream=self._stream, device=self._device)
        ev = torch.cuda.Event()
        ev.record(self._stream)
        return TransferFuture(ev)

    def shutdown(self) -> None:
        self._stream.synchronize()


@dataclass
class OffloadedState:
    """A (request, label) held in the CPU pool (``cpu_page_pool.py:17-22``)."""

    cpu_page_indices: list[int]
    seq_len: int
    position_id_start: int


class CPUPagePool:
    """Pinned host mirror of the paged KV pool (``cpu_page_pool.py:25-150``).

    Offload and reload are single launches that read the device pool and
    write the pinned host pool (or the reverse) directly over the bus.  The
    launch runs on the pool's own stream after the work queued on the
    caller's stream; after an offload the caller's stream also waits for it,
    so pages the caller frees and reuses are not overwritten before they
    have been read.
    """

    def __init__(self, kv_cache_config: KVCacheConfig, max_cpu_pages: int,
                 kv_cache_dtype: torch.dtype = torch.bfloat16):
        self.config = kv_cache_config
        self.page_allocator = PageAllocator(max_cpu_pages)
        self.cpu_kv_cache = torch.zeros(
            kv_cache_config.num_layers, max_cpu_pages, 2, kv_cache_config.page_size,
            kv_cache_config.num_kv_heads, kv_cache_config.head_dim, dtype=kv_cache_dtype, pin_memory=True,
        )
        self.offloaded: dict[str, dict[str, OffloadedState]] = {}
        self._stream: torch.cuda.Stream | None = None

    def _get_stream(self, device) -> torch.cuda.Stream:
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=device)
        return self._stream

    def is_offloaded(self, request_id: str) -> bool:
        return request_id in self.offloaded and len(self.offloaded[request_id]) > 0

    def offload_pages(self, request_id: str, label: str, gpu_kv_cache: torch.Tensor, gpu_page_indices: list[int],
                      seq_len: int, position_id_start: int) -> None:
        """GPU pages -> CPU pages, all layers, one launch (``cpu_page_pool.py:63-98``)."""
        n = len(gpu_page_indices)
        if n == 0:
            return
        cpu_pages = self.page_allocator.try_allocate(n)
        if cpu_pages is None:
            logger.warning("CPU page pool exhausted: cannot offload %d pages for %s/%s", n, request_id, label)
            return
        dev = gpu_kv_cache.device
        cur = torch.cuda.current_stream(dev)
        s = self._get_stream(dev)
        s.wait_stream(cur)
        copy_tokens(gpu_kv_cache, self.cpu_kv_cache, cpu_pages, gpu_page_indices, stream=s, device=dev)
        cur.wait_stream(s)
        self.offloaded.setdefault(request_id, {})[label] = OffloadedState(cpu_pages, seq_len, position_id_start)

    def reload_pages(self, request_id: str, label: str, gpu_kv_cache: torch.Tensor,
                     gpu_page_indices: list[int]) -> tuple[int, int]:
        """CPU pages -> GPU pages, one launch, then free the CPU pages (``cpu_page_pool.py:100-124``)."""
        state = self.offloaded[request_id][label]
        if len(state.cpu_page_indices) != len(gpu_page_indices):
            raise ValueError("reload needs one GPU page per offloaded page")
        dev = gpu_kv_cache.device
        s = self._get_stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        copy_tokens(self.cpu_kv_cache, gpu_kv_cache, gpu_page_indices, state.cpu_page_indices, stream=s, device=dev)
        self.page_allocator.free(state.cpu_page_indices)
        del self.offloaded[request_id][label]
        if not self.offloaded[request_id]:
            del self.offloaded[request_id]
        return state.seq_len, state.position_id_start

    def sync(self) -> None:
        """The caller's stream waits for every queued copy (``cpu_page_pool.py:126-129``)."""
        if self._stream is not None:
            torch.cuda.current_stream(self._stream.device).wait_stream(self._stream)

    def remove_request(self, request_id: str) -> None:
        if request_id not in self.offloaded:
            return
        for state in self.offloaded[request_id].values():
            self.page_allocator.free(state.cpu_page_indices)
        del self.offloaded[request_id]

    @property
    def num_free_pages(self) -> int:
        return self.page_allocator.num_free
