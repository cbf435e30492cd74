"""The transfer oracle (``oracle/transfer.py``) pinned by independent means.

* byte arithmetic of a (layer, page, K|V, token range) segment against the
  addresses torch computes for the same slice of a real 6-d pool;
* page-level read records against a brute-force per-token walk;
* pool-to-pool copies against numpy multi-axis indexing;
* the wire layout against a hand-written known answer, the closed-form
  offsets of the C header, and pack/unpack round trips;
* CPU-pool bookkeeping against the FIFO allocator's order.
"""

import numpy as np
import pytest
import torch

from oracle import transfer as T


def test_ptr_nbytes_matches_torch_slices():
    kv = torch.zeros(3, 5, 2, 4, 2, 8, dtype=torch.bfloat16)
    strides = kv.stride()
    rng = np.random.default_rng(0)
    for _ in range(50):
        layer, page = int(rng.integers(3)), int(rng.integers(5))
        ts = int(rng.integers(4))
        te = int(rng.integers(ts + 1, 5))
        ptrs, n = T.ptr_nbytes(kv.data_ptr(), strides, kv.element_size(), layer, page, ts, te)
        for half in (0, 1):
            sl = kv[layer, page, half, ts:te]
            assert ptrs[half] == sl.data_ptr()
            assert n == sl.numel() * sl.element_size()


def test_reference_ipc_read_slices_the_kv_axis():
    """``tensor[layer, page, ts:te]`` on the 6-d pool indexes K/V, not tokens
    (``kv_store.py:374-380``): a first page read from token 5 selects nothing.
    The wire/copy semantics here follow the byte arithmetic instead."""
    kv = torch.zeros(2, 3, 2, 16, 1, 8)
    assert kv[0, 1, 5:16].shape[0] == 0
    assert kv[0, 1, 0:16].shape == (2, 16, 1, 8)


@pytest.mark.parametrize("ps", [1, 4, 16])
def test_read_records_cover_exactly_the_missing_tokens(ps):
    rng = np.random.default_rng(ps)
    for _ in range(200):
        want = int(rng.integers(0, 9 * ps))
        have = int(rng.integers(0, want + 2))
        n = (want + ps - 1) // ps
        local = rng.permutation(1000)[:n].tolist()
        remote = rng.permutation(1000)[:n].tolist()
        recs = T.read_records(have, want, ps, local, remote)
        if have >= want:
            assert recs == []
            continue
        got = []
        for lp, rp, ts, te in recs:
            assert 0 <= ts < te <= ps
            pos = local.index(lp)
            assert remote[pos] == rp
            got += [pos * ps + t for t in range(ts, te)]
        assert got == list(range(have, want))  # every missing token once, in order
        layers = T.per_layer(recs, 3)
        assert len(layers) == 3 * len(recs)
        assert [r.layer_idx for r in layers[:3]] == [0, 1, 2]
        assert {(r.local_page_idx, r.token_start) for r in layers} == {(lp, ts) for lp, _, ts, _ in recs}


def test_copy_tokens_matches_indexing():
    rng = np.random.default_rng(1)
    L, P, ps, row = 3, 12, 8, 6
    src = rng.integers(0, 1 << 16, size=(L, P, 2, ps, row), dtype=np.uint16)
    dst0 = rng.integers(0, 1 << 16, size=(L, P + 3, 2, ps, row), dtype=np.uint16)
    recs = [(0, 5, 0, 8), (7, 1, 3, 4), (14, 2, 0, 1), (3, 11, 6, 8),
            (2, 40, 0, 8), (4, 3, 5, 5), (5, 3, -1, 2), (6, 3, 0, 9)]  # last four are skipped
    for lb, le in ((0, L), (1, 2)):
        got = T.copy_tokens(src, dst0.copy(), recs, lb, le)
        exp = dst0.copy()
        for dp, sp, ts, te in recs[:4]:
            exp[lb:le, dp, :, ts:te] = src[lb:le, sp, :, ts:te]
        np.testing.assert_array_equal(got, exp)


def test_wire_known_answer():
    # value = 1000*layer + 100*page + 10*kv + token; row of one element
    L, P, ps = 2, 3, 2
    pool = np.zeros((L, P, 2, ps, 1), np.int32)
    for layer in range(L):
        for p in range(P):
            for kv in range(2):
                for t in range(ps):
                    pool[layer, p, kv, t, 0] = 1000 * layer + 100 * p + 10 * kv + t
    wire = T.wire_pack(pool, [2, 0], [1, 0], [2, 2]).view(np.int32)
    assert wire.tolist() == [201, 211, 0, 1, 10, 11, 1201, 1211, 1000, 1001, 1010, 1011]


def test_wire_offsets_round_trip_and_layer_blocks():
    rng = np.random.default_rng(2)
    L, P, ps, row = 4, 20, 16, 8
    pool = rng.integers(0, 1 << 16, size=(L, P, 2, ps, row), dtype=np.uint16)
    pages = rng.permutation(P)[:9].tolist()
    ts = rng.integers(0, ps, size=9)
    te = np.minimum(ps, ts + rng.integers(1, ps + 1, size=9))
    recs = [(p, p, int(a), int(b)) for p, a, b in zip(pages, ts, te)]
    off = T.wire_offsets(recs)
    R = int(off[-1])
    wire = T.wire_pack(pool, pages, ts, te).view(np.uint16).reshape(-1, row)
    assert wire.shape[0] == 2 * R * L
    # closed-form position of every record's K and V rows (the C header's formula)
    for layer in range(L):
        for i, (p, a, b) in enumerate(zip(pages, ts, te)):
            k_at = 2 * R * layer + 2 * int(off[i])
            np.testing.assert_array_equal(wire[k_at:k_at + b - a], pool[layer, p, 0, a:b])
            np.testing.assert_array_equal(wire[k_at + b - a:k_at + 2 * (b - a)], pool[layer, p, 1, a:b])
    # a layer range is one contiguous block of the full wire
    sub = T.wire_pack(pool, pages, ts, te, 1, 3).view(np.uint16).reshape(-1, row)
    np.testing.assert_array_equal(sub, wire[2 * R:6 * R])
    # unpack restores exactly the covered rows
    back = T.wire_unpack(T.wire_pack(pool, pages, ts, te), np.zeros_like(pool), pages, ts, te)
    exp = np.zeros_like(pool)
    for p, a, b in zip(pages, ts, te):
        exp[:, p, :, a:b] = pool[:, p, :, a:b]
    np.testing.assert_array_equal(back, exp)


def test_cpu_pool_bookkeeping():
    rng = np.random.default_rng(3)
    gpu = rng.integers(0, 1 << 16, size=(2, 10, 2, 4, 3), dtype=np.uint16)
    pool = T.CpuPool(6, (2, 2, 4, 3), np.uint16)
    pool.offload("a", "main", gpu, [7, 2, 9], 10, 3)
    pool.offload("b", "main", gpu, [1, 4], 5, 0)
    assert pool.offloaded["a"]["main"][0] == [0, 1, 2] and pool.offloaded["b"]["main"][0] == [3, 4]
    pool.offload("c", "main", gpu, [0, 3], 6, 0)  # only one CPU page left: nothing recorded
    assert "c" not in pool.offloaded and list(pool.free.free) == [5]
    saved = gpu.copy()
    gpu[:] = 0
    assert pool.reload("b", "main", gpu, [8, 6]) == (5, 0)
    assert pool.reload("a", "main", gpu, [0, 1, 3]) == (10, 3)
    for g_new, g_old in zip([8, 6, 0, 1, 3], [1, 4, 7, 2, 9]):
        np.testing.assert_array_equal(gpu[:, g_new], saved[:, g_old])
    assert list(pool.free.free) == [5, 3, 4, 0, 1, 2] and pool.offloaded == {}
