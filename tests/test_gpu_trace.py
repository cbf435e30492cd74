"""Tracing ranges (``enable_nvtx``) on the planning path.

With ``enable_nvtx=True`` the manager and the decode wrapper push the
reference's range names (``mstar/engine/cache_manager.py:192-227, 269-325,
397-418, 443-512``; ``mstar/utils/flashinfer_utils.py:387-449``) around the
matching phases, balanced, in order; with ``enable_nvtx=False`` they push
nothing.  The recorder replaces the roctx-backed push/pop of
``mstar_amd.trace``.
"""

import pytest
import torch

from mstar_amd import trace
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from mstar_amd.paged_attention import FlashInferDecodeWrapper

pytestmark = pytest.mark.gpu


@pytest.fixture
def recorder(monkeypatch):
    events = []
    monkeypatch.setattr(trace, "range_push", lambda name: events.append(("push", name)))
    monkeypatch.setattr(trace, "range_pop", lambda: events.append(("pop", None)))
    return events


def _closed(events):
    """The ranges as (depth, name) in push order; asserts every push is popped."""
    depth, out = 0, []
    for kind, name in events:
        if kind == "push":
            out.append((depth, name))
            depth += 1
        else:
            depth -= 1
            assert depth >= 0
    assert depth == 0
    return out


def _manager(gpu, nvtx):
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=2, head_dim=128, max_seq_len=4096, max_num_pages=256,
                        page_size=16, num_qo_heads=8)
    kv = torch.zeros(1, 256, 2, 16, 2, 128, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    rids = ["a", "b"]
    for r in rids:
        mgr.add_request(r, ["main"])
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, WorkspaceBufferManager(16 << 20, gpu), cfg,
                             gpu, enable_nvtx=nvtx)
    return cm


def test_manager_and_wrapper_ranges(gpu, recorder):
    cm = _manager(gpu, True)
    cm.plan_attention([40, 3])  # prefill step
    cm.plan_rope([40, 3])
    cm._pre_planned_labels.add("main")
    cm.plan_attention([1, 1])  # pre-planned: skipped
    torch.cuda.synchronize()
    got = _closed(recorder)
    assert got == [
        (0, "cache.plan_attention"),
        (1, "cache.plan_attention.build_lists"),
        (1, "cache.plan_attention.make_tensors"),
        (1, "cache.plan_attention.wrapper_plan"),
        (0, "cache.plan_rope"),
        (1, "cache.plan_rope.build_pos_ids"),
        (1, "cache.plan_rope.copy_pos_ids"),
        (0, "cache.plan_attention"),
        (1, "cache.plan_attention.skipped_pre_planned"),
    ]
    recorder.clear()
    w = FlashInferDecodeWrapper(torch.empty(16 << 20, dtype=torch.uint8, device=gpu), 8, 2, 128, 16, device=gpu,
                                enable_nvtx=True)
    w.plan(torch.tensor([0, 1, 3], dtype=torch.int32), torch.tensor([5, 6, 7], dtype=torch.int32),
           torch.tensor([3, 16], dtype=torch.int32))
    w.plan(torch.tensor([0, 1, 3], dtype=torch.int32), torch.tensor([5, 6, 7], dtype=torch.int32),
           torch.tensor([3, 16], dtype=torch.int32), kv_cache_locations=torch.tensor([[5, 2], [7, 15]]))
    torch.cuda.synchronize()
    assert _closed(recorder) == [
        (0, "flashinfer.decode.metadata_h2d"), (0, "flashinfer.decode.plan_inner"),
        (0, "flashinfer.decode.metadata_h2d"), (0, "flashinfer.decode.kv_location_h2d"),
        (0, "flashinfer.decode.plan_inner"),
    ]


def test_no_ranges_without_nvtx(gpu, recorder):
    cm = _manager(gpu, False)
    cm.plan_attention([40, 3])
    cm.plan_rope([40, 3])
    torch.cuda.synchronize()
    assert recorder == []
