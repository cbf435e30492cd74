"""The host_step extension (csrc/host_step.c) against the Python loops it
replaces: PagedAllocationManager.alloc_batch + DeviceBlockTable.prepare_meta
(the pack kernel's metadata) and advance_seq_lens, on identical managers driven
through the same random step sequences (decode steps, prefill chunks, lists
replaced or edited in place, new and removed requests, a pool that runs dry).

Every test runs on both builds of the extension: the default one (on this
CPython 3.10 it reads instance dicts directly) and ``_host_step_generic``,
compiled with ``MI_DIRECT_DICT=0``: the generic attribute protocol that
CPython 3.11 and later compile (the reference targets 3.12)."""
import importlib
import random

import numpy as np
import pytest

from mstar_amd import kv_store
from mstar_amd.kv_store import AllocationFailedError, KVCacheConfig, PagedAllocationManager


def _load(name):
    try:
        return importlib.import_module(f"mstar_amd.{name}")
    except ImportError:
        return None


BUILDS = {name: _load(name) for name in ("_host_step", "_host_step_generic")}


@pytest.fixture(params=list(BUILDS))
def hs(request, monkeypatch):
    mod = BUILDS[request.param]
    if mod is None:
        pytest.skip(f"{request.param} not built (mstar_amd.build.build_host)")
    monkeypatch.setattr(kv_store, "_host_step", mod)
    return mod


def _mgr(pages: int) -> PagedAllocationManager:
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=2, head_dim=64, max_seq_len=4096, max_num_pages=pages,
                        page_size=16, num_qo_heads=4)
    return PagedAllocationManager(cfg, None, device="cpu")


def _py_meta(am, entries, states, seq_lens, gen):
    """The Python path of BatchedCacheManager._alloc_entries."""
    seq = np.array([st.seq_len for st in states], dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int64)
    am.alloc_batch(entries, states, seq + sl, gen)
    slots, npg, old, new = am.block_table.prepare_meta(states)
    head = np.stack([slots, seq.astype(np.int32), sl.astype(np.int32), npg, old]).astype(np.int32)
    return np.concatenate([head.reshape(-1), new])


def _snapshot(am):
    out = {}
    for rid, labels in am.request_states.items():
        for label, st in labels.items():
            out[(rid, label)] = (list(st.page_indices), st.seq_len, st.position_id_start, st.slot, st._dev_len,
                                 st._dev_ends)
    return out, list(am.page_allocator.free_pages), list(am.block_table._free_slots)


def _advance_py(states, seq_lens, adv):
    adv = seq_lens if adv is None else adv
    for st, n, a in zip(states, seq_lens, adv):
        st.seq_len += n
        st.position_id_start += a


@pytest.mark.parametrize("seed", range(6))
def test_host_step_matches_python_loops(seed, hs):
    rng = random.Random(seed)
    a, b = _mgr(600), _mgr(600)
    rids = []
    nxt = 0
    for step in range(60):
        # membership changes, mirrored on both managers
        if rng.random() < 0.3 or not rids:
            rid = f"r{nxt}"
            nxt += 1
            for m in (a, b):
                m.add_request(rid, ["main"])
            rids.append(rid)
        if rng.random() < 0.1 and len(rids) > 1:
            rid = rids.pop(rng.randrange(len(rids)))
            for m in (a, b):
                m.remove_request(rid)
        entries = [(r, "main") for r in rids]
        sa = [a.get_state(r, "main") for r in rids]
        sb = [b.get_state(r, "main") for r in rids]
        # occasional list replacement / in-place edit (with and without the marker)
        if rng.random() < 0.2:
            i = rng.randrange(len(rids))
            kind = rng.randrange(3)
            for st in (sa[i], sb[i]):
                if kind == 0 and st.page_indices:
                    st.page_indices = list(st.page_indices)  # same pages, new list object
                elif kind == 1 and len(st.page_indices) > 1:
                    st.page_indices[0], st.page_indices[-1] = st.page_indices[-1], st.page_indices[0]
                elif kind == 2 and st.page_indices:
                    st.page_indices[len(st.page_indices) // 2] = st.page_indices[len(st.page_indices) // 2]
                    st.pages_changed()
        seq_lens = [rng.choice([1, 1, 1, 7, 40, 200]) for _ in rids]
        gen_a = a.state_generation - (1 if rng.random() < 0.2 else 0)  # sometimes a stale generation
        gen_b = gen_a - a.state_generation + b.state_generation
        ea = eb = None
        try:
            ma = _py_meta(a, entries, sa, seq_lens, gen_a)
        except AllocationFailedError as e:
            ea = e
        try:
            mb = b.alloc_pack_meta(entries, sb, seq_lens, gen_b)
        except AllocationFailedError as e:
            eb = e
        assert (ea is None) == (eb is None), (step, ea, eb)
        if ea is not None:
            assert (ea.request_id, ea.pages_short) == (eb.request_id, eb.pages_short)
            # the pool ran dry: free everything and start over on both
            for m in (a, b):
                for r in list(m.request_states):
                    m.remove_request(r)
            rids.clear()
            assert _snapshot(a) == _snapshot(b)
            continue
        assert ma.dtype == mb.dtype == np.int32
        assert np.array_equal(ma, mb), step
        assert _snapshot(a) == _snapshot(b), step
        # advance, default and custom position advances
        adv = None if rng.random() < 0.7 else [rng.randrange(3) for _ in rids]
        _advance_py(sa, seq_lens, adv)
        hs.advance(sb, seq_lens, adv)
        assert _snapshot(a) == _snapshot(b), step


def test_host_step_matches_python_loops_at_large_batch(hs):
    a, b = _mgr(40000), _mgr(40000)
    rng = random.Random(9)
    rids = [f"r{i}" for i in range(1100)]
    for m in (a, b):
        for r in rids:
            m.add_request(r, ["main"])
    entries = [(r, "main") for r in rids]
    for step in range(3):
        sl = [rng.randint(1, 40) if step == 0 else 1 for _ in rids]
        sa = [a.get_state(r, "main") for r in rids]
        sb = [b.get_state(r, "main") for r in rids]
        ma = _py_meta(a, entries, sa, sl, a.state_generation)
        mb = b.alloc_pack_meta(entries, sb, sl, b.state_generation)
        assert np.array_equal(ma, mb)
        _advance_py(sa, sl, None)
        hs.advance(sb, sl, None)
        assert _snapshot(a) == _snapshot(b)


def test_host_step_accepts_numpy_lengths(hs):
    a, b = _mgr(64), _mgr(64)
    for m in (a, b):
        for r in ("x", "y"):
            m.add_request(r, ["main"])
    entries = [("x", "main"), ("y", "main")]
    sl = np.array([17, 3], dtype=np.int64)
    ma = _py_meta(a, entries, [a.get_state(r, l) for r, l in entries], sl, a.state_generation)
    mb = b.alloc_pack_meta(entries, [b.get_state(r, l) for r, l in entries], sl, b.state_generation)
    assert np.array_equal(ma, mb)
    hs.advance([b.get_state(r, l) for r, l in entries], sl, None)
    assert [b.get_state(r, "main").seq_len for r in ("x", "y")] == [17, 3]


def test_host_step_rejects_rows_longer_than_the_table(hs):
    m = _mgr(600)
    m.add_request("x", ["main"])
    st = m.get_state("x", "main")
    st.page_indices = list(range(300))  # 300 pages > 4096 / 16 = 256 per row
    with pytest.raises(ValueError, match="block table rows hold 256"):
        m.alloc_pack_meta([("x", "main")], [st], [0], m.state_generation)


def test_generic_build_uses_attribute_protocol():
    """The generic build reads and writes state attributes through
    getattr/setattr, so it also works on objects without an instance dict."""
    gen = BUILDS["_host_step_generic"]
    if gen is None:
        pytest.skip("_host_step_generic not built")

    class Slotted:
        __slots__ = ("seq_len", "position_id_start", "page_indices")

    st = Slotted()
    st.seq_len, st.position_id_start, st.page_indices = 5, 2, [1]
    gen.advance([st], [3], None)
    assert (st.seq_len, st.position_id_start) == (8, 5)


def test_host_step_needs_counts_pages(hs):
    m = _mgr(64)
    m.add_request("x", ["main"])
    st = m.get_state("x", "main")
    st.seq_len = 15
    st.page_indices = [5]
    total, need = hs.needs([st], [1], 16)
    assert total == 0 and np.frombuffer(need, np.int32).tolist() == [0]
    total, need = hs.needs([st], [2], 16)
    assert total == 1 and np.frombuffer(need, np.int32).tolist() == [1]
    with pytest.raises(ValueError):
        hs.needs([st], [1, 1], 16)
