"""CPU restatement of KV page transfer: remote reads, offload/reload, wire format.

Test infrastructure only (see ``oracle/__init__.py``).

A pool here is a numpy array ``[layers, pages, 2, page_size, row]`` of any
dtype (``row`` = num_kv_heads * head_dim elements), the layout of
``mstar/engine/kv_cache_engine.py:132-136`` with the head and dim axes
flattened.  A record is ``(dst_page, src_page, token_start, token_end)``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .packing import FifoPages


@dataclass(frozen=True)
class ReadInfo:
    """``KVReadInfo`` (``mstar/engine/kv_store.py:177-183``)."""

    layer_idx: int
    local_page_idx: int
    remote_page_idx: int
    token_start: int
    token_end: int


def read_records(have: int, want: int, page_size: int, local_pages, remote_pages) -> list[tuple]:
    """Page-level records of ``start_async_retrieve`` (``kv_store.py:516-552``).

    The local state holds ``have`` tokens, the remote one ``want``; pages
    ``have // ps .. (want - 1) // ps`` are read, the first from token
    ``have % ps``, the last up to ``want % ps or ps``.  ``local_pages`` is
    the local page list after it has been grown to ``want`` tokens.
    """
    if have >= want:
        return []
    first = have // page_size
    last = (want - 1) // page_size
    out = []
    for pos in range(first, last + 1):
        ts = 0 if pos > first else have % page_size
        te = page_size if pos != last else (want % page_size or page_size)
        out.append((int(local_pages[pos]), int(remote_pages[pos]), ts, te))
    return out


def per_layer(records, num_layers: int) -> list[ReadInfo]:
    """The reference's ``KVReadInfo`` list: page-major, then layer (``kv_store.py:540-547``)."""
    return [ReadInfo(layer, lp, rp, ts, te) for (lp, rp, ts, te) in records for layer in range(num_layers)]


def ptr_nbytes(base: int, strides, element_size: int, layer: int, page: int, token_start: int,
               token_end: int) -> tuple[list[int], int]:
    """``MooncakeKVTransferEngine._get_ptr_nbytes`` (``kv_store.py:233-259``).

    ``strides`` are the element strides of the 6-d pool ``[L, P, 2, ps, H, D]``;
    returns the byte addresses of the K and V segments and their common size.
    """
    layer_stride, page_stride, kv_stride, token_stride = strides[:4]
    nbytes = (token_end - token_start) * token_stride * element_size
    ptrs = [base + (layer * layer_stride + page * page_stride + kv * kv_stride + token_start * token_stride)
            * element_size for kv in (0, 1)]
    return ptrs, nbytes


def copy_tokens(src: np.ndarray, dst: np.ndarray, records, layer_begin: int = 0, layer_end: int | None = None):
    """Apply records to ``dst`` in place, through flat byte addressing.

    Each (layer, K|V) segment is located with :func:`ptr_nbytes` on the
    pools' own byte buffers, as a remote-read transport would address it.
    Records with out-of-range pages or empty/out-of-page ranges are skipped.
    """
    layers, pages, two, ps, row = src.shape
    assert two == 2 and dst.shape[2:] == src.shape[2:] and src.dtype == dst.dtype
    assert src.flags.c_contiguous and dst.flags.c_contiguous
    layer_end = layers if layer_end is None else layer_end
    es = src.itemsize
    s_flat = src.reshape(-1).view(np.uint8)
    d_flat = dst.reshape(-1).view(np.uint8)
    s_str = [x // es for x in src.strides]
    d_str = [x // es for x in dst.strides]
    for dp, sp, ts, te in records:
        if not (0 <= sp < pages and 0 <= dp < dst.shape[1] and 0 <= ts < te <= ps):
            continue
        for layer in range(layer_begin, layer_end):
            sptr, n = ptr_nbytes(0, s_str, es, layer, sp, ts, te)
            dptr, _ = ptr_nbytes(0, d_str, es, layer, dp, ts, te)
            for a, b in zip(sptr, dptr):
                d_flat[b:b + n] = s_flat[a:a + n]
    return dst


def wire_offsets(records) -> np.ndarray:
    """Exclusive prefix sum of record row counts (``len + 1`` entries)."""
    rows = [te - ts for (_, _, ts, te) in records]
    return np.concatenate([[0], np.cumsum(rows, dtype=np.int64)]).astype(np.int64)


def wire_pack(pool: np.ndarray, pages, token_start, token_end, layer_begin: int = 0,
              layer_end: int | None = None) -> np.ndarray:
    """The wire buffer of ``mi_kv_wire_pack``: layer-major blocks, each the
    records in order, each record its K rows then its V rows."""
    layer_end = pool.shape[0] if layer_end is None else layer_end
    parts = []
    for layer in range(layer_begin, layer_end):
        for p, ts, te in zip(pages, token_start, token_end):
            parts.append(pool[layer, p, 0, ts:te].reshape(-1))
            parts.append(pool[layer, p, 1, ts:te].reshape(-1))
    if not parts:
        return np.zeros(0, np.uint8)
    return np.concatenate(parts).view(np.uint8)


def wire_unpack(wire: np.ndarray, pool: np.ndarray, pages, token_start, token_end, layer_begin: int = 0,
                layer_end: int | None = None) -> np.ndarray:
    """Inverse of :func:`wire_pack` into ``pool`` (in place)."""
    layer_end = pool.shape[0] if layer_end is None else layer_end
    row = pool.shape[-1]
    flat = wire.view(pool.dtype)
    at = 0
    for layer in range(layer_begin, layer_end):
        for p, ts, te in zip(pages, token_start, token_end):
            for kv in (0, 1):
                n = (te - ts) * row
                pool[layer, p, kv, ts:te] = flat[at:at + n].reshape(te - ts, row)
                at += n
    return pool


class CpuPool:
    """``CPUPagePool`` bookkeeping (``mstar/engine/cpu_page_pool.py:25-150``).

    ``offload`` takes CPU pages from a FIFO list and copies GPU pages there
    (all layers); when the list is short it records nothing (the reference
    logs a warning and returns, ``:77-83``).  ``reload`` copies back into the
    given GPU pages and frees the CPU pages.
    """

    def __init__(self, num_pages: int, shape_tail, dtype):
        self.free = FifoPages(num_pages)
        self.data = np.zeros((shape_tail[0], num_pages) + tuple(shape_tail[1:]), dtype=dtype)
        self.offloaded: dict[str, dict[str, tuple]] = {}

    def offload(self, rid: str, label: str, gpu: np.ndarray, gpu_pages, seq_len: int, pos: int) -> None:
        if not gpu_pages:
            return
        cpu_pages = self.free.take(len(gpu_pages))
        if cpu_pages is None:
            return
        for g, c in zip(gpu_pages, cpu_pages):
            self.data[:, c] = gpu[:, g]
        self.offloaded.setdefault(rid, {})[label] = (cpu_pages, seq_len, pos)

    def reload(self, rid: str, label: str, gpu: np.ndarray, gpu_pages) -> tuple[int, int]:
        cpu_pages, seq_len, pos = self.offloaded[rid][label]
        for c, g in zip(cpu_pages, gpu_pages, strict=True):
            gpu[:, g] = self.data[:, c]
        self.free.give(cpu_pages)
        del self.offloaded[rid][label]
        if not self.offloaded[rid]:
            del self.offloaded[rid]
        return seq_len, pos
