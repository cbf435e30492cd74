"""The device block table under failure and under concurrent planning.

* A plan that fails after its pages were allocated (here: a state whose page
  list outgrows the table rows, raised while the step's metadata is built)
  must not leave the other states marked as synced: the next step's
  ``kv_indices`` must hold every page of every request.
* Two planning threads over one allocation manager, with a table that starts
  at 4 rows and doubles while both plan: each step's packed ``kv_indices`` must
  equal the host page lists (a pack launched into a table being replaced
  would lose rows).
"""

import threading

import numpy as np
import pytest
import torch

from gpu_helpers import log
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import DeviceBlockTable, KVCacheConfig, PagedAllocationManager

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS = 8, 2, 64, 16


def _setup(gpu, max_seq_len, pages, slots=None):
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=HKV, head_dim=D, max_seq_len=max_seq_len, max_num_pages=pages,
                        page_size=PS, num_qo_heads=HQ)
    kv = torch.zeros(1, pages, 2, PS, HKV, D, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    if slots is not None:
        mgr.block_table = DeviceBlockTable(mgr.block_table.stride, gpu, max_slots=slots)
    return cfg, kv, mgr, WorkspaceBufferManager(16 << 20, gpu)


def _packed_pages(cm, states):
    qo, kv_indptr, kv_indices, last, loc = cm._last_pack
    torch.cuda.synchronize()
    got = kv_indices.cpu().numpy()
    want = np.array([p for st in states for p in st.page_indices], dtype=np.int32)
    return got, want


def test_failed_plan_resends_pages(gpu):
    cfg, kv, mgr, bufs = _setup(gpu, max_seq_len=64, pages=64)  # rows hold 4 pages
    rids = ["a", "b", "c"]
    for r in rids:
        mgr.add_request(r, ["main"])
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
    cm.plan_attention([20, 10, 5])
    cm.advance_seq_lens()
    # a grows by a page, b would need 5 pages (> 4 per row): raised after a's new page is handed out
    with pytest.raises(ValueError):
        cm.plan_attention([16, 60, 1])
    st = {r: mgr.get_state(r, "main") for r in rids}
    assert len(st["a"].page_indices) == 3
    mgr.remove_request("b")
    rids2 = ["a", "c"]
    cm2 = BatchedCacheManager(rids2, {r: "main" for r in rids2}, kv, mgr, bufs, cfg, gpu)
    cm2.plan_attention([1, 1])
    got, want = _packed_pages(cm2, [st["a"], st["c"]])
    np.testing.assert_array_equal(got, want)
    log("failed plan: next step packs every page")


def test_two_planning_threads_grow_table(gpu):
    cfg, kv, mgr, bufs = _setup(gpu, max_seq_len=1024, pages=4096, slots=4)
    groups = [[f"t{t}r{i}" for i in range(12)] for t in range(2)]
    for g in groups:
        for r in g:
            mgr.add_request(r, ["main"])
    errors = []
    barrier = threading.Barrier(2)

    def run(t):
        try:
            rids = groups[t]
            rng = np.random.default_rng(t)
            own = WorkspaceBufferManager(16 << 20, gpu)  # each thread plans into its own workspace
            barrier.wait()
            for step in range(8):
                sl = rng.integers(1, 40, len(rids)).tolist() if step % 3 == 0 else [1] * len(rids)
                cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, own, cfg, gpu)
                with torch.cuda.stream(torch.cuda.Stream(gpu)):
                    cm.plan_attention(sl, is_causal=True)
                    got, want = _packed_pages(cm, [mgr.get_state(r, "main") for r in rids])
                if not np.array_equal(got, want):
                    errors.append(f"thread {t} step {step}: packed pages differ from the page lists")
                cm.advance_seq_lens()
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors
    assert mgr.block_table.max_slots >= 24
    log(f"two planning threads: table grew to {mgr.block_table.max_slots} rows")
