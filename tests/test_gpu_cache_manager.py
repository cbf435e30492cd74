"""GPU end-to-end: BatchedCacheManager over several steps vs a list-history oracle.

The oracle keeps each request's K/V as a plain growing list per layer — the
reference's own CPU stand-in for the paged path
(test/modular/vjepa2/test_ac_kv_cache_parity.py:28-99) — and attends with the
fp32 oracle (causal, aligned to the end of the history).  Also checks CUDA-graph
capture/replay of the decode wrapper (static buffers, fixed batch).
"""

import numpy as np
import pytest
import torch

from gpu_helpers import A, custom_batch, log, max_abs, workspace
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from mstar_amd.paged_attention import FlashInferDecodeWrapper

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 2e-5)])
def test_manager_steps_match_list_history(gpu, dtype, tol):
    """bf16 pool, and an fp32 pool as the reference allocates for fp32 models
    (kv_cache_engine.py:104-105): the manager plans in the pool's dtype."""
    hq, hkv, d, ps, layers = 16, 4, 128, 16, 2
    cfg = KVCacheConfig(num_layers=layers, num_kv_heads=hkv, head_dim=d, max_seq_len=4096, max_num_pages=600,
                        page_size=ps, num_qo_heads=hq)
    kv = torch.zeros(layers, 600, 2, ps, hkv, d, dtype=dtype, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    rids = [f"r{i}" for i in range(5)]
    for r in rids:
        mgr.add_request(r, ["main"])
    hist = {(r, l): ([], []) for r in rids for l in range(layers)}
    g = torch.Generator().manual_seed(0)
    schedule = [[37, 1, 200, 16, 90]] + [[1] * 5] * 5 + [[3, 0, 20, 1, 17]] + [[1] * 5] * 2
    for step, seq_lens in enumerate(schedule):
        cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
        cm.plan_attention(seq_lens, is_causal=True)
        n = sum(seq_lens)
        worst = 0.0
        for layer in range(layers):
            q = torch.randn(n, hq, d, generator=g).to(dtype)
            k = torch.randn(n, hkv, d, generator=g).to(dtype)
            v = torch.randn(n, hkv, d, generator=g).to(dtype)
            out = cm.run_attention(q.to(gpu), k.to(gpu), v.to(gpu), layer_idx=layer)
            assert out.dtype == dtype
            off = 0
            ref = torch.zeros(n, hq, d)
            for r, sl in zip(rids, seq_lens):
                hk, hv = hist[(r, layer)]
                hk.append(k[off:off + sl])
                hv.append(v[off:off + sl])
                if sl:
                    o, _ = A.attend(q[off:off + sl], torch.cat(hk), torch.cat(hv), causal=True, sm_scale=d ** -0.5)
                    ref[off:off + sl] = o
                off += sl
            worst = max(worst, max_abs(out, ref))
        cm.advance_seq_lens()
        log(f"step {step}: tokens={n} max_abs={worst:.3e}")
        assert worst < tol
    for r in rids:
        st = mgr.get_state(r, "main")
        assert st.seq_len == sum(s[rids.index(r)] for s in schedule)


def test_decode_wrapper_cuda_graph_replay(gpu):
    hq, hkv, d, ps, b = 32, 4, 128, 16, 6
    pool = 800
    cache = torch.randn(pool, 2, ps, hkv, d, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu)
    w = FlashInferDecodeWrapper(workspace(gpu), hq, hkv, d, ps, batch_size=b, max_num_pages=pool, device=gpu,
                                use_cuda_graph=True)
    q_static = torch.zeros(b, hq, d, dtype=torch.bfloat16, device=gpu)
    kn = torch.zeros(b, hkv, d, dtype=torch.bfloat16, device=gpu)
    lens0 = [100, 5, 2000, 17, 64, 900]
    _, kv_indptr, kv_indices, last = custom_batch(lens0, ps, pool, seed=2)
    w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up outside capture
        w.set_kv_cache(cache, kn, kn)
        w.run(q_static, cache)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.set_kv_cache(cache, kn, kn)
        out_static = w.run(q_static, cache)
    g = torch.Generator().manual_seed(3)
    for rep, lens in enumerate([lens0, [3000, 1, 1, 40, 700, 16], [16, 32, 48, 64, 80, 96]]):
        _, kv_indptr, kv_indices, last = custom_batch(lens, ps, pool, seed=10 + rep)
        w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last))
        q_static.copy_(torch.randn(b, hq, d, generator=g).to(torch.bfloat16))
        kn.copy_(torch.randn(b, hkv, d, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        replay = out_static.clone()
        # eager on the same state (append is idempotent for the same token)
        eager = w.run(q_static, cache)
        torch.cuda.synchronize()
        log(f"graph replay {rep}: max diff vs eager {max_abs(replay, eager):.3e}")
        assert torch.equal(replay, eager)
        ref = A.paged_attention(q_static.cpu(), cache.cpu(), None, kv_indptr, kv_indices, last, causal=False)
        assert max_abs(replay, ref) < 2e-2


def test_per_step_managers_with_gpu_behind_host(gpu):
    """One manager per step (as the reference engine builds them) while the GPU runs
    steps behind the host: every step's metadata upload must reach the GPU intact."""
    hq, hkv, d, ps = 8, 2, 64, 16
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=hkv, head_dim=d, max_seq_len=4096, max_num_pages=400,
                        page_size=ps, num_qo_heads=hq)
    kv = torch.zeros(1, 400, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    rids = [f"r{i}" for i in range(6)]
    for r in rids:
        mgr.add_request(r, ["main"])
    g = torch.Generator().manual_seed(4)
    schedule = [[20, 33, 1, 7, 64, 15]] + [[1] * 6] * 11
    ins, outs = [], []
    for seq_lens in schedule:
        cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
        cm.plan_attention(seq_lens, is_causal=True)
        n = sum(seq_lens)
        q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
        k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        torch.cuda._sleep(1_000_000)  # keep the GPU behind: the host plans ahead
        outs.append(cm.run_attention(q.to(gpu, non_blocking=True), k.to(gpu), v.to(gpu)))
        ins.append((q, k, v))
        cm.advance_seq_lens()
    torch.cuda.synchronize()
    hist = {r: ([], []) for r in rids}
    for (q, k, v), out, seq_lens in zip(ins, outs, schedule):
        off = 0
        ref = torch.zeros(q.shape)
        for r, sl in zip(rids, seq_lens):
            hist[r][0].append(k[off:off + sl])
            hist[r][1].append(v[off:off + sl])
            if sl:
                ref[off:off + sl], _ = A.attend(q[off:off + sl], torch.cat(hist[r][0]), torch.cat(hist[r][1]),
                                                causal=True, sm_scale=d ** -0.5)
            off += sl
        assert max_abs(out, ref) < 2e-2
