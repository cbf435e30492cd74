"""Host allocation paths of the manager against the oracle's FIFO restatement (CPU).

``PagedAllocationManager.alloc_batch`` takes the pages of a whole step in one
pass over the free list; it must hand out exactly the pages the oracle's
request-by-request ``alloc`` (kv_store.py:463-482) gives, in batch order, and
on a pool that runs out it must raise at the same request with the same
shortfall while the earlier requests keep their pages.
"""

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from mstar_amd.kv_store import AllocationFailedError, KVCacheConfig, PagedAllocationManager
from oracle import packing as P


def _manager(pages, ps):
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=1, head_dim=64, max_seq_len=1 << 20, max_num_pages=pages,
                        page_size=ps)
    return PagedAllocationManager(cfg)


@settings(max_examples=60, deadline=None)
@given(steps=st.lists(st.lists(st.integers(0, 70), min_size=1, max_size=12), min_size=1, max_size=6),
       ps=st.sampled_from([1, 4, 16]), pool_pages=st.integers(1, 120))
def test_alloc_batch_matches_sequential_fifo(steps, ps, pool_pages):
    width = max(len(s) for s in steps)
    mgr = _manager(pool_pages, ps)
    pool = P.FifoPages(pool_pages)
    rids = [f"r{i}" for i in range(width)]
    for r in rids:
        mgr.add_request(r, ["main"])
    ostates = [P.ReqState() for _ in rids]
    for step in steps:
        step = (step + [0] * width)[:width]
        entries = [(r, "main") for r in rids]
        states = [mgr.get_state(r, "main") for r in rids]
        after = np.array([st_.seq_len + n for st_, n in zip(states, step)])
        exp_err = None
        for i, (o, n) in enumerate(zip(ostates, step)):
            try:
                P.alloc(o, pool, o.seq_len + n, ps)
            except P.OutOfPages as e:
                exp_err = (i, e.short)
                break
        if exp_err is None:
            mgr.alloc_batch(entries, states, after)
        else:
            with pytest.raises(AllocationFailedError) as e:
                mgr.alloc_batch(entries, states, after)
            assert (e.value.request_id, e.value.pages_short) == (rids[exp_err[0]], exp_err[1])
        assert [s.page_indices for s in states] == [o.pages for o in ostates]
        assert list(mgr.page_allocator.free_pages) == list(pool.free)
        if exp_err is not None:
            return
        for s, o, n in zip(states, ostates, step):
            s.seq_len += n
            o.seq_len += n


def test_state_generation_tracks_new_and_removed_states():
    mgr = _manager(16, 4)
    g0 = mgr.state_generation
    mgr.add_request("a", ["main"])
    g1 = mgr.state_generation
    assert g1 > g0
    mgr.get_state("a", "main")          # existing: unchanged
    assert mgr.state_generation == g1
    mgr.get_state("a", "cfg")           # new label: a new state object
    g2 = mgr.state_generation
    assert g2 > g1
    mgr.reset_label("a", "main")
    g3 = mgr.state_generation
    assert g3 > g2
    mgr.remove_request("a")
    assert mgr.state_generation > g3
