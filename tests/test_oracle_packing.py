"""Pin the packing oracle (oracle/packing.py) against independent derivations.

* hand-computed known answers (including the T=0 quirk, cache_manager.py:291);
* a token-by-token brute-force simulation of allocation (one token at a time,
  a new page whenever the current one is full) — a different algorithm that
  must produce the same FIFO page ids, lengths and write slots;
* invariants over random ragged batches (hypothesis);
* page conservation, as test_page_allocator_thread_safety.py:67-93 asserts.
"""

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import packing as P


def test_known_answer_two_steps():
    pool = P.FifoPages(8)
    s = [P.ReqState(), P.ReqState()]
    out = P.pack(s, [17, 16], pool, 16)
    assert out.qo_indptr.tolist() == [0, 17, 33]
    assert out.kv_indptr.tolist() == [0, 2, 3]
    assert out.kv_indices.tolist() == [0, 1, 2]
    assert out.last_page_len.tolist() == [1, 16]
    assert out.kv_locations is None  # not a decode batch
    s[0].seq_len, s[1].seq_len = 17, 16
    out = P.pack(s, [1, 1], pool, 16)
    assert out.kv_indptr.tolist() == [0, 2, 4]
    assert out.kv_indices.tolist() == [0, 1, 2, 3]  # r1 crossed a page boundary: page 3
    assert out.last_page_len.tolist() == [2, 1]
    assert out.kv_locations.tolist() == [[1, 1], [3, 0]]


def test_zero_length_request_quirk():
    # T = 0 gives last_page_len = page_size with zero pages (cache_manager.py:291)
    pool = P.FifoPages(4)
    out = P.pack([P.ReqState(), P.ReqState()], [0, 3], pool, 16)
    assert out.kv_indptr.tolist() == [0, 0, 1]
    assert out.last_page_len.tolist() == [16, 3]
    assert out.kv_indices.tolist() == [0]


def test_fifo_reuse_order():
    pool = P.FifoPages(4)
    a = pool.take(3)
    assert a == [0, 1, 2]
    pool.give([1, 0])
    assert pool.take(3) == [3, 1, 0]  # free list is FIFO: 3 was free first, then 1, 0
    assert pool.take(1) is None


def test_out_of_pages_keeps_earlier_allocations():
    pool = P.FifoPages(3)
    s = [P.ReqState(), P.ReqState(), P.ReqState()]
    with pytest.raises(P.OutOfPages) as e:
        P.pack(s, [32, 32, 1], pool, 16)
    assert e.value.index == 1 and e.value.short == 1
    assert s[0].pages == [0, 1] and s[1].pages == [] and len(pool.free) == 1


def _simulate(seq_before, new_lens, page_size, pool_size, perm=None):
    """Token-by-token allocation: pages appear when a token starts a new page."""
    free = list(range(pool_size))
    pages = []
    tok_pos = []  # per request: list of (page, slot) of its new tokens
    for r, (s0, sl) in enumerate(zip(seq_before, new_lens)):
        pl = []
        for t in range(s0 + sl):
            if t % page_size == 0:
                pl.append(free.pop(0))
        pages.append(pl)
        tok_pos.append([(pl[t // page_size], t % page_size) for t in range(s0, s0 + sl)])
    return pages, tok_pos


@settings(max_examples=60, deadline=None)
@given(
    lens=st.lists(st.tuples(st.integers(0, 70), st.integers(0, 40)), min_size=1, max_size=12),
    page_size=st.sampled_from([1, 4, 16, 32]),
)
def test_pack_matches_token_by_token_simulation(lens, page_size):
    seq_before = [a for a, _ in lens]
    new = [b for _, b in lens]
    pool_size = sum(-(-(a + b) // page_size) for a, b in lens) + 3
    sim_pages, sim_tok = _simulate(seq_before, new, page_size, pool_size)
    # oracle: a first step allocates the prefix, a second the new tokens
    pool = P.FifoPages(pool_size)
    states = [P.ReqState() for _ in lens]
    for st_, a in zip(states, seq_before):
        P.alloc(st_, pool, a, page_size)
        st_.seq_len = a
    # allocation of the prefix happens request by request, so replay the
    # simulation in the same two-phase order
    pool2 = list(range(pool_size))
    two_phase = []
    for a in seq_before:
        two_phase.append([pool2.pop(0) for _ in range(-(-a // page_size))])
    for pl, a, b in zip(two_phase, seq_before, new):
        need = -(-(a + b) // page_size) - len(pl)
        pl.extend(pool2.pop(0) for _ in range(max(need, 0)))
    out = P.pack(states, new, pool, page_size)
    assert [s.pages for s in states] == two_phase
    # lengths and layout
    T = np.array(seq_before) + np.array(new)
    npages = np.diff(out.kv_indptr)
    assert out.kv_indptr[-1] == len(out.kv_indices)
    assert np.all((T == 0) | ((npages - 1) * page_size + out.last_page_len == T))
    assert np.all((out.last_page_len >= 1) & (out.last_page_len <= page_size))
    assert out.qo_indptr.tolist() == [0] + np.cumsum(new).tolist()
    # per-token map against direct positions (seq_len_before + j)
    t2p, t2c = P.token_map(out.qo_indptr, out.kv_indptr, out.kv_indices, out.last_page_len, page_size)
    expect = []
    for pl, a, b in zip(two_phase, seq_before, new):
        expect += [(pl[t // page_size], t % page_size) for t in range(a, a + b)]
    assert list(zip(t2p.tolist(), t2c.tolist())) == expect
    # single-phase allocation equals the token-by-token simulation
    pool3 = P.FifoPages(pool_size)
    st3 = [P.ReqState() for _ in lens]
    P.pack(st3, list(T), pool3, page_size)
    assert [s.pages for s in st3] == sim_pages


def test_decode_locations_match_last_token():
    pool = P.FifoPages(64)
    rng = np.random.default_rng(0)
    seq = rng.integers(0, 90, size=10).tolist()
    states = [P.ReqState() for _ in seq]
    for s, a in zip(states, seq):
        P.alloc(s, pool, a, 16)
        s.seq_len = a
    out = P.pack(states, [1] * 10, pool, 16)
    for r, s in enumerate(states):
        t = s.seq_len  # the new token's absolute position
        assert out.kv_locations[r].tolist() == [s.pages[t // 16], t % 16]
    loc = P.decode_locations(out.kv_indptr, out.kv_indices, out.last_page_len)
    assert (loc == out.kv_locations).all()


def test_token_map_graph_tail_is_zero():
    t2p, t2c = P.token_map([0, 3], [0, 1], [5], [3], 16, tail_len=6)
    assert t2p.tolist() == [5, 5, 5, 0, 0, 0] and t2c.tolist() == [0, 1, 2, 0, 0, 0]


def test_pages_are_conserved_through_alloc_and_free():
    pool = P.FifoPages(64)
    rng = np.random.default_rng(1)
    live = []
    for _ in range(200):
        if live and rng.random() < 0.4:
            pool.give(live.pop(int(rng.integers(len(live)))).pages)
            continue
        s = P.ReqState()
        try:
            P.alloc(s, pool, int(rng.integers(1, 60)), 8)
            live.append(s)
        except P.OutOfPages:
            pass
    held = [p for s in live for p in s.pages]
    assert len(held) == len(set(held))
    assert sorted(held + list(pool.free)) == list(range(64))


def test_split_chunks_cover_every_page_once():
    kv_indptr = np.array([0, 0, 3, 40, 41, 300])
    cp, n = P.split_chunks(kv_indptr, 16, 64, 4, min_chunk_tokens=256)
    assert cp == max(16, -(-300 // 16))
    pages = np.diff(kv_indptr)
    for npg, k in zip(pages, n):
        assert (k == 0) == (npg == 0)
        if npg:
            assert (k - 1) * cp < npg <= k * cp


def test_split_chunks_small_job_rule_against_brute_force():
    # a small job: the smallest item size in [lo, min chunk] whose item count fits the slots
    rng = np.random.default_rng(5)
    for trial in range(200):
        n = int(rng.integers(1, 12))
        pages = rng.integers(0, 300, n)
        kv_indptr = np.concatenate([[0], np.cumsum(pages)])
        slots = int(rng.integers(1, 200))
        cp, k = P.split_chunks(kv_indptr, 16, 4096, 4, slots=slots)
        total, cmin = int(pages.sum()), 64
        cnt = lambda c: sum(-(-int(x) // c) for x in pages)
        ctarget = -(-total // 256)
        if ctarget >= cmin:
            assert cp == ctarget
            continue
        lo = min(max(16, ctarget, -(-int(pages.max()) // 16), 1), cmin)
        fits = [c for c in range(lo, cmin + 1) if cnt(c) <= slots]
        assert cp == (fits[0] if fits else cmin), (trial, pages.tolist(), slots, cp)
        assert int(k.sum()) == cnt(cp) and all(-(-int(x) // cp) <= 16 or cp == cmin for x in pages)
    # without slots the rule is the plain minimum chunk
    assert P.split_chunks(np.array([0, 5, 9]), 16, 4096, 4)[0] == 64


def test_snapshot_copies_history_and_keeps_leading_pages():
    import torch

    ps = 4
    pool = P.FifoPages(40)
    cache = torch.arange(40 * 3, dtype=torch.float32).reshape(1, 40, 3)  # one layer, 3 values per page
    src = P.ReqState()
    P.alloc(src, pool, 10, ps)
    src.seq_len = 10
    dst, pairs = P.snapshot(src, P.ReqState(), pool, ps, cache)
    assert dst.seq_len == 10 and len(dst.pages) == 3 and set(dst.pages).isdisjoint(src.pages)
    assert pairs == list(zip(src.pages, dst.pages))
    assert torch.equal(cache[0, dst.pages], cache[0, src.pages])
    # the source grows: only pages from dst.seq_len // ps on are copied again
    P.alloc(src, pool, 19, ps)
    src.seq_len = 19
    cache[0, src.pages[2]] += 100.0  # the partially filled page changed
    before = cache.clone()
    dst, pairs = P.snapshot(src, dst, pool, ps, cache)
    assert [s for s, _ in pairs] == src.pages[2:] and len(dst.pages) == 5
    assert torch.equal(cache[0, dst.pages], cache[0, src.pages])
    assert torch.equal(cache[0, dst.pages[:2]], before[0, dst.pages[:2]])  # leading pages untouched
    # realloc returns the old pages to the pool first (FIFO tail) and copies everything
    n_free = len(pool.free)
    dst2, pairs = P.snapshot(src, dst, pool, ps, cache, realloc=True)
    assert len(pairs) == 5 and len(pool.free) == n_free  # 5 freed, 5 taken
    assert torch.equal(cache[0, dst2.pages], cache[0, src.pages])


def test_snapshot_rejects_mismatched_page_counts():
    pool = P.FifoPages(16)
    src = P.ReqState()
    P.alloc(src, pool, 20, 4)  # 5 pages for 20 tokens, but only 6 tokens counted as cached
    src.seq_len = 6
    with pytest.raises(ValueError):
        P.snapshot(src, P.ReqState(), pool, 4)
