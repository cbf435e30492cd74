"""Packed prefill under HIP graph capture, the way M*'s piecewise graph runner drives it.

Mirrors ``PiecewiseCudaGraphRunner`` (``mstar/engine/cuda_graph_runner.py``):
a persistent graph-mode prefill wrapper per batch size
(``_build_persistent_wrappers``, ``:2405-2425``: ``batch_size=bs``,
``max_total_tokens=bs * capture_seq_len``, ``use_cuda_graph=True``) under a
static ``BatchedCacheManager``; the capture plans every slot at the full
capture length and records every layer's ``run_attention`` (append + ragged
attention, the decode-kernel part on the wrapper's side stream).  Each replay
re-plans the same manager with the real requests first and zero-length
padding requests after them (``_run_flashinfer_packed``, ``:1431``;
``_zero_padding_input``, ``:1659-1690``), copies the real tokens' q/k/v into
the static inputs and replays.

Per replay and layer: the cache equals the oracle's append of the real tokens
bit for bit (padding tokens write nothing), the output rows of the real
tokens are within max-abs 2e-2 of the oracle's causal fp32 attention, and an
eager ``run`` of the same plan right after the replay gives the replay's
output bit for bit.  Replays alternate with eager work and synchronisation,
and the token counts differ from replay to replay.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import A, P, log, max_abs
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager, _PlanState
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from mstar_amd.paged_attention import FlashInferPrefillWrapper

pytestmark = pytest.mark.gpu

PS, LAYERS, SEQ = 16, 2, 64


def _schedule(bs):
    """(live requests, new tokens each) per replay."""
    if bs == 4:
        # chunks over growing prefixes, short (decode-kernel) queries, zero-length padding after the real requests
        return [
            (["r0", "r1", "r2"], [64, 10, 33]),
            (["r0", "r1", "r2", "r3"], [5, 64, 17, 1]),
            (["r1", "r3"], [2, 40]),
            (["r0", "r2", "r3"], [1, 2, 64]),
            (["r3"], [7]),
        ]
    # >= 128 slots: the short-query half reads kv-head pairs (one-token requests); two- and
    # three-token requests (14-21 rows) and chunks go to the tiles
    rng = np.random.default_rng(bs)
    out = []
    for n_live in (bs, bs - 3, 100, bs):
        new = rng.choice([1, 1, 1, 1, 2, 3, 17, 64], n_live).tolist()
        out.append(([f"r{i}" for i in range(n_live)], new))
    return out


# c4's heads (head_dim 128, the ping-pong tiles) and the Pi0.5 heads (head_dim 256, the role-split tiles)
@pytest.mark.parametrize("BS,HQ,HKV,D", [(4, 28, 4, 128), (130, 28, 4, 128), (4, 8, 1, 256)])
def test_packed_prefill_graph_replays_with_padding(gpu, BS, HQ, HKV, D):
    POOL = 512 if BS == 4 else 4096
    cfg = KVCacheConfig(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, max_seq_len=4096, max_num_pages=POOL,
                        page_size=PS, num_qo_heads=HQ)
    g = torch.Generator().manual_seed(11)
    kv = torch.randn(LAYERS, POOL, 2, PS, HKV, D, generator=g).to(torch.bfloat16).to(gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    w = FlashInferPrefillWrapper(bufs.get(f"main_pcgr_{BS}"), HQ, HKV, D, PS, batch_size=BS,
                                 max_total_tokens=BS * SEQ, max_num_pages=POOL, device=gpu, use_cuda_graph=True)
    dummies = [f"__pcg_{i}__" for i in range(BS)]
    for r in dummies:
        mgr.add_request(r, ["main"])
    cm = BatchedCacheManager(list(dummies), {r: "main" for r in dummies}, kv, mgr, bufs, cfg, gpu,
                             cuda_graph_plan_states={"main": _PlanState(wrapper=w)})
    q = torch.zeros(LAYERS, BS * SEQ, HQ, D, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(LAYERS, BS * SEQ, HKV, D, dtype=torch.bfloat16, device=gpu)
    v = torch.zeros(LAYERS, BS * SEQ, HKV, D, dtype=torch.bfloat16, device=gpu)

    def forward():
        return torch.stack([cm.run_attention(q[l], k[l], v[l], layer_idx=l) for l in range(LAYERS)])

    # capture: every slot planned at the full capture length
    cm.plan_attention([SEQ] * BS, is_causal=True)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        forward()  # warm-up outside capture
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = forward()
    for r in dummies:
        mgr.reset_label(r, "main", free=True)
    torch.cuda.synchronize()
    cache_cpu = kv.cpu()  # the oracle's cache starts from what the warm-up left

    real = [f"r{i}" for i in range(BS)]
    for r in real:
        mgr.add_request(r, ["main"])
    from mstar_amd import _lib

    short = _lib.lib().mi_prefill_short_rows(BS, HQ, HKV, D)
    log(f"BS={BS} heads {HQ}/{HKV} D={D}: short-query threshold {short} rows")
    for step, (live, new) in enumerate(_schedule(BS)):
        ids = live + dummies[len(live):]
        sls = new + [0] * (BS - len(live))
        cm.request_ids = ids
        cm.active_labels = {r: "main" for r in ids}
        ntok = sum(sls)
        qs = torch.randn(LAYERS, ntok, HQ, D, generator=g).to(torch.bfloat16)
        ks = torch.randn(LAYERS, ntok, HKV, D, generator=g).to(torch.bfloat16)
        vs = torch.randn(LAYERS, ntok, HKV, D, generator=g).to(torch.bfloat16)
        for name, x in (("q", qs), ("k", ks), ("v", vs)):
            t = {"q": q, "k": k, "v": v}[name]
            t.zero_()
            t[:, :ntok].copy_(x.to(gpu))
        # oracle: the same states and free list, packed by the reference's loop
        states = [mgr.get_state(r, "main") for r in ids]
        ostates = [P.ReqState(pages=list(st.page_indices), seq_len=st.seq_len) for st in states]
        pool = P.FifoPages(0)
        pool.free.extend(mgr.page_allocator.free_pages)
        want = P.pack(ostates, sls, pool, PS)
        t2p, t2c = P.token_map(want.qo_indptr, want.kv_indptr, want.kv_indices, want.last_page_len, PS)

        cm.plan_attention(sls, is_causal=True)
        graph.replay()
        torch.cuda.synchronize()
        out = static_out.clone()
        eager = torch.stack([w.run(q[l], kv[l]) for l in range(LAYERS)])
        torch.cuda.synchronize()
        worst = 0.0
        for layer in range(LAYERS):
            A.append(cache_cpu[layer], t2p, t2c, ks[layer], vs[layer])
            assert torch.equal(kv[layer].cpu().view(torch.int16), cache_cpu[layer].view(torch.int16)), \
                f"replay {step} layer {layer}: cache differs from the oracle's append"
            ref = A.paged_attention(qs[layer], cache_cpu[layer], want.qo_indptr, want.kv_indptr, want.kv_indices,
                                    want.last_page_len, causal=True)
            worst = max(worst, max_abs(out[layer, :ntok], ref))
        assert torch.equal(out[:, :ntok].view(torch.int16), eager[:, :ntok].view(torch.int16)), \
            f"replay {step}: graph output differs from an eager run of the same plan"
        log(f"replay {step}: real={len(live)} tokens={ntok} max_abs={worst:.3e}")
        assert worst < 2e-2
        cm.advance_seq_lens()
        assert [mgr.get_state(r, "main").seq_len for r in live] == [o.seq_len + n for o, n in zip(ostates, new)]
