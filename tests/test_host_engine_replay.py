"""The reference engine's calls on the allocation manager and state types, on the CPU.

``engine_replay.MiniEngine`` makes the calls ``mstar/engine/kv_cache_engine.py``
makes (construction with ``transfer_engine_info``, ``get_node_str`` keys,
``write_policy``, ``get_labels`` + ``get_state().get_pos_info()``, the policy
setter, ``request_states`` reads, ``cleanup``).  The GPU half of the sequence
(``BatchedCacheManager`` built by ``_create_cache_manager``, a planned step, the
producer/consumer read) is in ``test_gpu_engine_replay.py``.
"""

import inspect

import pytest
import torch

from engine_replay import LocalTransferEngine, MiniEngine, MooncakeTransferEngine, StubTransferEngine
from mstar_amd.cache_manager import BatchedCacheManager
from mstar_amd.kv_store import (KVCacheConfig, PagedAllocationManager, PositionInfo, StoreWritePolicy,
                                TransferEngineInfo)


def _cfg(nodes=None, pages=64):
    return KVCacheConfig(num_layers=2, num_kv_heads=2, head_dim=64, max_seq_len=1024, max_num_pages=pages,
                         page_size=16, num_qo_heads=8, nodes=nodes)


def _info(te):
    return TransferEngineInfo(my_entity_id="worker0", my_session_id="session0", transfer_engine=te)


def test_node_str_keys():
    """``kv_store.py:90-93``: joined node names, or ALL_NODES."""
    assert _cfg().get_node_str() == "ALL_NODES"
    assert _cfg(["Thinker"]).get_node_str() == "Thinker"
    assert _cfg(["Thinker", "Talker"]).get_node_str() == "Thinker///Talker"
    eng = MiniEngine([_cfg(["A", "B"]), _cfg()], torch.device("cpu"), _info(StubTransferEngine()))
    assert set(eng.kv_management) == {"A///B", "ALL_NODES"}


def test_reference_constructor_and_policy():
    eng = MiniEngine([_cfg()], torch.device("cpu"), _info(StubTransferEngine()))
    am = eng.kv_management["ALL_NODES"].alloc_manager
    assert am.write_policy is StoreWritePolicy.ALWAYS  # kv_store.py:405
    # _create_cache_manager's read and keyword set (kv_cache_engine.py:192-205) bind to this BatchedCacheManager
    autowrite = am.write_policy == StoreWritePolicy.ALWAYS
    inspect.signature(BatchedCacheManager).bind(
        request_ids=["r"], active_labels_per_request={"r": "main"}, kv_cache=am.kv_cache, alloc_manager=am,
        buffer_manager=None, kv_cache_config=am.config, device=torch.device("cpu"), auto_write_store=autowrite,
        enable_nvtx=False)
    eng.set_alloc_write_policy(StoreWritePolicy.NEVER)
    assert am.write_policy is StoreWritePolicy.NEVER
    assert StoreWritePolicy("always") is StoreWritePolicy.ALWAYS and StoreWritePolicy("never") is StoreWritePolicy.NEVER
    # positional order of the reference (config, kv_cache, transfer_engine_info)
    PagedAllocationManager(_cfg(), None, _info(None))


def test_transport_selection():
    """``kv_store.py:413-426``: single-node transports get the device reader,
    an RDMA transport is refused as unsupported."""
    for te in (None, StubTransferEngine(), LocalTransferEngine()):
        am = PagedAllocationManager(config=_cfg(), kv_cache=None, transfer_engine_info=_info(te))
        assert am._kv_transfer_engine is None  # device reader, built on first use
    with pytest.raises(ValueError, match="Unsupported transfer engine"):
        PagedAllocationManager(config=_cfg(), kv_cache=None, transfer_engine_info=_info(MooncakeTransferEngine()))

    class Reader:  # an object that is already a KV reader is used as it is
        def read_pages_async(self, *a, **k):
            return None

        def shutdown(self):
            self.closed = True

    r = Reader()
    am = PagedAllocationManager(config=_cfg(), kv_cache=None, transfer_engine_info=_info(r))
    assert am.kv_transfer_engine is r
    am.cleanup()
    assert r.closed


def test_batch_pos_info_and_lifecycle():
    """Requests through the engine's per-batch reads: ``get_labels`` +
    ``get_state().get_pos_info()`` (``kv_cache_engine.py:789-796``),
    ``request_states`` (``:1095-1105``), ``page_allocator.num_free`` (``:331``)."""
    eng = MiniEngine([_cfg(pages=40)], torch.device("cpu"), _info(StubTransferEngine()))
    key = "ALL_NODES"
    am = eng.kv_management[key].alloc_manager
    eng.add_request("a")
    eng.add_request("b", ["main", "cfg"])
    assert eng.pos_infos(key, ["a", "b"]) == {
        "a": {"main": PositionInfo(0, 0)},
        "b": {"main": PositionInfo(0, 0), "cfg": PositionInfo(0, 0)},
    }
    am.alloc("a", "main", 40)  # 3 pages
    st = am.get_state("a", "main")
    st.seq_len, st.position_id_start = 40, 7
    am.alloc("b", "cfg", 17)  # 2 pages
    am.get_state("b", "cfg").seq_len = 17
    info = eng.pos_infos(key, ["a", "b"])
    assert info["a"]["main"] == PositionInfo(full_seq_len=40, position_id_start=7)
    assert info["b"]["cfg"].full_seq_len == 17 and info["b"]["main"].full_seq_len == 0
    assert sorted(eng.offload_candidates(key)) == [("a", 3), ("b", 2)]
    assert eng.free_pages(key) == 35
    eng.remove_request("a")
    assert eng.free_pages(key) == 38
    eng.shutdown()  # cleanup() with no reader built is a no-op
    assert eng.kv_management[key].kv_cache is None
