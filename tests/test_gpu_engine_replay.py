"""M*'s KV-cache engine sequence on the GPU, through this package's classes.

Two ``engine_replay.MiniEngine`` instances (a producer and a consumer worker,
each with its own pool on this GPU) are driven as ``KVCacheEngine`` drives its
caches: construction with ``transfer_engine_info`` (``kv_cache_engine.py:150-163``),
``_create_cache_manager`` per batch (``:184-205``), the model's
``plan_attention`` / ``run_attention`` per layer / ``advance_seq_lens``,
``flush_to_store`` (``:444``), ``finalize_batch``'s ``get_per_label_seq_info``
(``:724-737``), the consumer's ``sync_retrieve`` (``:760-768``) and
``get_pos_info`` reads (``:789-796``), the policy setter (``:1091-1093``) and
``shutdown`` (``:1145-1150``).  Attention outputs of both workers are checked
against the fp32 oracle over each request's full K/V history.
"""

import pytest
import torch

from engine_replay import MiniEngine, StubTransferEngine
from gpu_helpers import A, log, max_abs
from mstar_amd.kv_store import KVCacheConfig, PositionInfo, StoreWritePolicy, TransferEngineInfo

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS, LAYERS = 8, 2, 128, 16, 2


def _cfg(node):
    return KVCacheConfig(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, max_seq_len=2048, max_num_pages=256,
                         page_size=PS, num_qo_heads=HQ, nodes=[node])


def _step(eng, key, rids, seq_lens, hist, g, causal=True):
    """One batch as the engine runs it: a fresh BatchedCacheManager, plan, one
    run_attention per layer, advance, flush.  Returns the worst max-abs error
    against the oracle over every layer."""
    cm = eng.create_cache_manager(key, rids)
    cm.plan_attention(seq_lens, is_causal=causal)
    n = sum(seq_lens)
    worst = 0.0
    for layer in range(LAYERS):
        q = torch.randn(n, HQ, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16)
        out = cm.run_attention(q.to(eng.device), k.to(eng.device), v.to(eng.device), layer_idx=layer)
        off = 0
        ref = torch.zeros(n, HQ, D)
        for r, sl in zip(rids, seq_lens):
            hk, hv = hist.setdefault((r, layer), ([], []))
            hk.append(k[off:off + sl])
            hv.append(v[off:off + sl])
            if sl:
                o, _ = A.attend(q[off:off + sl], torch.cat(hk), torch.cat(hv), causal=True, sm_scale=D ** -0.5)
                ref[off:off + sl] = o
            off += sl
        worst = max(worst, max_abs(out, ref))
    cm.advance_seq_lens()
    cm.flush_to_store()
    return worst


def test_engine_sequence_producer_consumer(gpu):
    info = TransferEngineInfo(my_entity_id="w0", my_session_id="s0", transfer_engine=StubTransferEngine())
    prod = MiniEngine([_cfg("Thinker")], gpu, info, workspace_mb=64)
    cons = MiniEngine([_cfg("Thinker")], gpu, info, workspace_mb=64)
    key = "Thinker"
    assert set(prod.kv_management) == {key}
    g = torch.Generator().manual_seed(7)
    hist = {}
    rids = ["a", "b", "c"]
    for r in rids:
        prod.add_request(r)
    # producer: a prefill batch, then two decode batches
    errs = [_step(prod, key, rids, [45, 16, 130], hist, g)]
    errs += [_step(prod, key, rids, [1, 1, 1], hist, g) for _ in range(2)]
    assert prod.pos_infos(key, rids) == {
        "a": {"main": PositionInfo(47, 47)}, "b": {"main": PositionInfo(18, 18)}, "c": {"main": PositionInfo(132, 132)}}
    written = prod.finalize(key, rids)
    # consumer: the engine's retrieve, then a decode batch over the copied history
    for r in rids:
        cons.add_request(r)
        cons.sync_retrieve(key, r, written[r])
    assert cons.pos_infos(key, rids) == prod.pos_infos(key, rids)
    am = cons.kv_management[key].alloc_manager
    for r in rids:
        st = am.get_state(r, "main")
        assert not st.read_in_progress and len(st.page_indices) == -(-st.seq_len // PS)
    errs.append(_step(cons, key, rids, [1, 1, 1], hist, g))
    # policy NEVER: the managers the engine creates no longer auto-write the store
    cons.set_alloc_write_policy(StoreWritePolicy.NEVER)
    assert cons.create_cache_manager(key, rids).auto_write_store is False
    assert prod.create_cache_manager(key, rids).auto_write_store is True
    assert max(errs) < 2e-2, errs
    for r in rids:
        prod.remove_request(r)
        cons.remove_request(r)
    assert prod.free_pages(key) == cons.free_pages(key) == 256
    prod.shutdown()
    cons.shutdown()
    log(f"engine sequence: producer prefill+2 decode, consumer retrieve+decode, max_abs {max(errs):.3e}")
