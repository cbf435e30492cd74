"""CPU restatement of allocation, batch packing and the per-token page map.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import collections
from dataclasses import dataclass, field

import numpy as np


class FifoPages:
    """FIFO free-page list (``mstar/engine/kv_store.py:37-63``).

    Pages start in order ``0..N-1``; ``take`` pops from the head; ``give``
    appends to the tail.
    """

    def __init__(self, num_pages: int):
        self.free = collections.deque(range(num_pages))

    def take(self, n: int) -> list[int] | None:
        if len(self.free) < n:
            return None
        return [self.free.popleft() for _ in range(n)]

    def give(self, pages: list[int]) -> None:
        self.free.extend(pages)


@dataclass
class ReqState:
    """Per-request KV state (``kv_store.py:111-118``)."""

    pages: list[int] = field(default_factory=list)
    seq_len: int = 0


class OutOfPages(Exception):
    def __init__(self, index: int, short: int):
        super().__init__(f"request {index}: {short} page(s) short")
        self.index = index
        self.short = short


def alloc(state: ReqState, pool: FifoPages, seq_len: int, page_size: int) -> None:
    """Grow ``state.pages`` to ceil(seq_len/page_size) pages (``kv_store.py:463-482``)."""
    need = (seq_len + page_size - 1) // page_size - len(state.pages)
    if need > 0:
        got = pool.take(need)
        if got is None:
            raise OutOfPages(-1, need - len(pool.free))
        state.pages.extend(got)


@dataclass
class Packed:
    qo_indptr: np.ndarray      # int32 [B+1]
    kv_indptr: np.ndarray      # int32 [B+1]
    kv_indices: np.ndarray     # int32 [sum pages]
    last_page_len: np.ndarray  # int32 [B]
    kv_locations: np.ndarray | None  # int64 [B, 2] when every new_len == 1


def pack(states: list[ReqState], new_lens: list[int], pool: FifoPages, page_size: int) -> Packed:
    """Allocate and pack one step, in batch order (``cache_manager.py:272-322``).

    Raises :class:`OutOfPages` at the first request the pool cannot serve;
    earlier requests keep their new pages, as in the reference.
    """
    qo = [0]
    kv = [0]
    indices: list[int] = []
    last: list[int] = []
    locs: list[list[int]] = []
    for i, (st, sl) in enumerate(zip(states, new_lens)):
        total = st.seq_len + sl
        try:
            alloc(st, pool, total, page_size)
        except OutOfPages as e:
            raise OutOfPages(i, e.short) from None
        qo.append(qo[-1] + sl)
        indices.extend(st.pages)
        kv.append(kv[-1] + len(st.pages))
        lpl = total % page_size or page_size
        last.append(lpl)
        if sl == 1:
            locs.append([st.pages[-1], lpl - 1])
    return Packed(
        qo_indptr=np.asarray(qo, dtype=np.int32),
        kv_indptr=np.asarray(kv, dtype=np.int32),
        kv_indices=np.asarray(indices, dtype=np.int32),
        last_page_len=np.asarray(last, dtype=np.int32),
        kv_locations=np.asarray(locs, dtype=np.int64).reshape(-1, 2) if len(locs) == len(states) else None,
    )


def token_map(qo_indptr, kv_indptr, kv_indices, last_page_len, page_size: int,
              tail_len: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Per-new-token (page, slot) (``flashinfer_utils.py:211-256``).

    kv_len_after = (pages-1)*page_size + last_page_len; token j of request r
    lands at absolute position kv_len_after - qo_len + j.  With ``tail_len``
    the result is padded with zeros to that length (graph-mode tail,
    ``:251-253``).
    """
    qo_indptr = np.asarray(qo_indptr, dtype=np.int64)
    kv_indptr = np.asarray(kv_indptr, dtype=np.int64)
    kv_indices = np.asarray(kv_indices, dtype=np.int64)
    last_page_len = np.asarray(last_page_len, dtype=np.int64)
    lens = np.diff(qo_indptr)
    starts = qo_indptr[:-1]
    total = int(lens.sum())
    npages = np.diff(kv_indptr)
    kv_len_after = (npages - 1) * page_size + last_page_len
    seg = np.repeat(np.arange(len(lens)), lens)
    intra = np.arange(total) - np.repeat(starts, lens)
    g = kv_len_after[seg] - lens[seg] + intra
    page_off = np.floor_divide(g, page_size)
    t2p = kv_indices[kv_indptr[:-1][seg] + page_off]
    t2c = g - page_off * page_size
    if tail_len is not None and tail_len > total:
        t2p = np.concatenate([t2p, np.zeros(tail_len - total, dtype=np.int64)])
        t2c = np.concatenate([t2c, np.zeros(tail_len - total, dtype=np.int64)])
    return t2p.astype(np.int64), t2c.astype(np.int64)


def decode_locations(kv_indptr, kv_indices, last_page_len) -> np.ndarray:
    """Decode write locations (``flashinfer_utils.py:433-436``): (last page, last_page_len-1)."""
    kv_indptr = np.asarray(kv_indptr, dtype=np.int64)
    kv_indices = np.asarray(kv_indices, dtype=np.int64)
    page = kv_indices[kv_indptr[1:] - 1]
    pos = np.asarray(last_page_len, dtype=np.int64) - 1
    return np.stack([page, pos], axis=1)


def split_chunks(kv_indptr, page_size: int, target_units: int, num_kv_heads: int,
                 min_chunk_tokens: int = 1024, slots: int | None = None, small_chunk_tokens: int = 256,
                 max_small_items: int = 16) -> tuple[int, np.ndarray]:
    """Split-KV partition rule of the GPU plan: (item_pages, items per request).

    target = max(16, target_units // (4 * num_kv_heads)) (4 wavefronts per
    item) and item_pages = max(ceil(min_chunk_tokens/page_size),
    ceil(total_pages/target)), except for a small job (ceil(total_pages/target)
    below the minimum chunk) when ``slots`` is given: then item_pages is the
    smallest value in [lo, ceil(min_chunk_tokens/page_size)] whose item count
    is at most ``slots``, with lo = max(ceil(small_chunk_tokens/page_size),
    ceil(total_pages/target), ceil(longest request's pages/max_small_items)).
    Each request's page list is cut into ceil(pages/item_pages) consecutive
    items.  This is the build's own schedule (FlashInfer's is not reproduced);
    the attention result must not depend on it beyond rounding.
    """
    kv_indptr = np.asarray(kv_indptr, dtype=np.int64)
    npages = np.diff(kv_indptr)
    target = max(16, target_units // (4 * num_kv_heads))
    total = int(kv_indptr[-1] - kv_indptr[0])
    cmin = -(-min_chunk_tokens // page_size)
    cp = -(-total // target)
    count = lambda c: int(np.where(npages > 0, -(-npages // c), 0).sum())
    if cp >= cmin or slots is None:
        cp = max(cp, cmin)
    else:
        longest = int(npages.max(initial=0))
        lo = max(-(-small_chunk_tokens // page_size), cp, -(-longest // max_small_items), 1)
        lo = min(lo, cmin)
        hi = cmin
        while lo < hi:
            mid = (lo + hi) // 2
            if count(mid) <= slots:
                hi = mid
            else:
                lo = mid + 1
        cp = lo
    return cp, np.where(npages > 0, -(-npages // cp), 0)


def snapshot(from_state: ReqState, to_state: ReqState, pool: FifoPages, page_size: int,
             cache=None, realloc: bool = False) -> tuple[ReqState, list[tuple[int, int]]]:
    """``snapshot_all`` for one request (``mstar/engine/cache_manager.py:840-870``).

    With ``realloc`` the destination's pages go back to the pool and it starts
    empty.  The destination keeps its first ``seq_len // page_size`` pages,
    grows to the source's length, takes its seq_len, and pages from there on
    are copied source -> destination (all layers of ``cache [L, pages, ...]``
    when given).  Returns the destination state and the (src, dst) pairs.
    """
    if realloc:
        pool.give(to_state.pages)
        to_state = ReqState()
    start = to_state.seq_len // page_size
    alloc(to_state, pool, from_state.seq_len, page_size)
    to_state.seq_len = from_state.seq_len
    pairs = list(zip(from_state.pages[start:], to_state.pages[start:], strict=True))
    if cache is not None:
        for s, d in pairs:
            cache[:, d] = cache[:, s]
    return to_state, pairs
