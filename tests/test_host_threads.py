"""Allocator and manager under thread contention (CPU).

M*'s engine runs ``plan()`` of the next step on a plan thread while the GPU
thread resets labels and removes finished requests
(``mstar/engine/cuda_graph_runner.py:1031-1078``, ``worker.py:2031-2036``).
These tests port the invariants of the reference's
``test/modular/test_page_allocator_thread_safety.py:67-120`` (page
conservation, no page handed out twice, ``try_allocate`` against concurrent
``free``, ``alloc`` racing ``reset_label``, request add/alloc/remove cycles)
and extend them to this build's batched paths: ``alloc_batch`` and the
device block table's slot bookkeeping.
"""

import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from mstar_amd.kv_store import (AllocationFailedError, DeviceBlockTable, KVCacheConfig, KVRequestState,
                                PageAllocator, PagedAllocationManager)


def _manager(pages: int, ps: int = 8) -> PagedAllocationManager:
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=1, head_dim=64, max_seq_len=pages * ps, max_num_pages=pages,
                        page_size=ps)
    return PagedAllocationManager(cfg)


def _run(workers):
    with ThreadPoolExecutor(max_workers=len(workers)) as ex:
        for f in [ex.submit(w) for w in workers]:
            f.result()


def test_alloc_free_cycles_conserve_pages():
    alloc = PageAllocator(64)

    def worker():
        for _ in range(200):
            got = alloc.try_allocate(2)
            if got is not None:
                assert len(set(got)) == 2
                alloc.free(got)

    _run([worker] * 16)
    assert alloc.num_free == 64
    assert sorted(alloc.free_pages) == list(range(64))


def test_racing_allocations_never_share_a_page():
    for _ in range(20):
        alloc = PageAllocator(8)
        gate = threading.Barrier(4)
        got, lock = [], threading.Lock()

        def worker():
            gate.wait()
            pages = alloc.try_allocate(2)
            if pages is not None:
                with lock:
                    got.extend(pages)

        _run([worker] * 4)
        assert len(got) == len(set(got)) == 8
        assert alloc.num_free == 0


def test_try_allocate_against_concurrent_free():
    alloc = PageAllocator(32)
    held = alloc.allocate(32)
    held_lock = threading.Lock()
    stop = threading.Event()
    out = [0]
    out_lock = threading.Lock()

    def consumer():
        while not stop.is_set():
            pages = alloc.try_allocate(1)
            if pages is None:
                continue
            with out_lock:
                out[0] += 1
                assert out[0] + alloc.num_free <= 32 + len(held)
                out[0] -= 1
            alloc.free(pages)

    def producer():
        for _ in range(500):
            with held_lock:
                if not held:
                    continue
                p = held.pop()
            alloc.free([p])
            back = alloc.try_allocate(1)
            if back is not None:
                with held_lock:
                    held.extend(back)

    with ThreadPoolExecutor(max_workers=8) as ex:
        cons = [ex.submit(consumer) for _ in range(4)]
        prods = [ex.submit(producer) for _ in range(4)]
        for f in prods:
            f.result()
        stop.set()
        for f in cons:
            f.result()
    alloc.free(held)
    assert sorted(alloc.free_pages) == list(range(32))


def test_alloc_racing_reset_label_conserves_pages():
    mgr = _manager(64)
    mgr.add_request("r", ["main"])
    lens = [8, 16, 24, 16, 8]

    def allocer():
        for i in range(300):
            try:
                mgr.alloc("r", "main", lens[i % len(lens)])
            except (KeyError, RuntimeError):
                pass

    def resetter():
        for _ in range(300):
            mgr.reset_label("r", "main")

    _run([allocer, allocer, resetter, resetter])
    mgr.reset_label("r", "main")
    assert mgr.page_allocator.num_free == 64
    assert mgr.request_states["r"]["main"].page_indices == []


def test_add_alloc_remove_cycles_conserve_pages():
    mgr = _manager(128)

    def worker(t):
        for i in range(50):
            rid = f"r{t}_{i}"
            mgr.add_request(rid, ["main"])
            try:
                mgr.alloc(rid, "main", 16)
            except RuntimeError:
                pass
            mgr.remove_request(rid)

    _run([lambda t=t: worker(t) for t in range(8)])
    assert mgr.page_allocator.num_free == 128
    assert mgr.request_states == {} and mgr.pending_reads == {}


def test_alloc_batch_against_resets_and_removals():
    """Plan threads allocate whole steps (``alloc_batch``) while another thread
    resets labels and removes requests: afterwards every live page list is
    disjoint from the others and from the free list, and together they hold
    every page exactly once."""
    pages = 512
    mgr = _manager(pages, ps=4)
    groups = [[f"g{t}_{i}" for i in range(6)] for t in range(3)]
    for g in groups:
        for rid in g:
            mgr.add_request(rid, ["main"])
    stop = threading.Event()

    def planner(g):
        rng = np.random.default_rng(len(g[0]))
        for _ in range(150):
            entries = [(rid, "main") for rid in g]
            try:
                with mgr._lock:  # the states of one step, read together
                    gen = mgr.state_generation
                    states = [mgr.get_state(rid, "main") for rid in g]
                after = np.array([st.seq_len + int(rng.integers(0, 9)) for st in states])
                mgr.alloc_batch(entries, states, after, gen)
                for st, n in zip(states, after):
                    st.seq_len = int(n)
            except AllocationFailedError:
                for rid in g:
                    mgr.reset_label(rid, "main")

    def janitor():
        i = 0
        while not stop.is_set():
            g = groups[i % len(groups)]
            mgr.reset_label(g[i % len(g)], "main")
            i += 1

    with ThreadPoolExecutor(max_workers=4) as ex:
        j = ex.submit(janitor)
        ps = [ex.submit(planner, g) for g in groups]
        for f in ps:
            f.result()
        stop.set()
        j.result()
    held = [p for g in groups for rid in g for p in mgr.get_state(rid, "main").page_indices]
    assert len(held) == len(set(held))
    assert sorted(held + list(mgr.page_allocator.free_pages)) == list(range(pages))


def test_block_table_slots_under_contention():
    """Threads preparing disjoint request sets on one block table (with growth)
    never share a slot, and release returns every slot."""
    bt = DeviceBlockTable(32, torch.device("cpu"), max_slots=2)
    sets = [[KVRequestState(page_indices=[t * 100 + i]) for i in range(16)] for t in range(6)]

    def worker(states):
        for _ in range(40):
            bt.prepare_meta(states)
            for st in states[::3]:
                bt.release(st)

    _run([lambda s=s: worker(s) for s in sets])
    live = [st.slot for s in sets for st in s if st.slot >= 0]
    assert len(live) == len(set(live))
    for s in sets:
        for st in s:
            bt.release(st)
    assert sorted(bt._free_slots) == list(range(bt.max_slots))
