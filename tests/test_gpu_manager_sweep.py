"""GPU end-to-end sweep: BatchedCacheManager over randomized multi-step schedules
against a list-history oracle (each request's K/V kept as a growing list per
layer and attended in fp32, causal, aligned to the end of its history).

Requests join and leave between steps (their pages go back to the FIFO list
and are handed out again), steps mix prefill chunks and decode tokens, and
batch sizes reach past 150 requests, so one schedule covers both ways the pack
metadata reaches the GPU (kernel argument and staged copy), the paired-kv-head
decode kernels and the per-head ones, and block-table slot reuse.
"""

import random

import pytest
import torch

from gpu_helpers import A, log, max_abs
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,max_req", [(0, 12), (1, 24), (2, 170), (3, 160)])
def test_manager_random_schedule_matches_list_history(gpu, seed, max_req):
    rng = random.Random(seed)
    hq, hkv, d, ps, layers = 16, 4, 128, 16, 1
    pool_pages = 8000
    cfg = KVCacheConfig(num_layers=layers, num_kv_heads=hkv, head_dim=d, max_seq_len=8192,
                        max_num_pages=pool_pages, page_size=ps, num_qo_heads=hq)
    kv = torch.zeros(layers, pool_pages, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(128 << 20, gpu)
    g = torch.Generator().manual_seed(seed)
    live: list[str] = []
    hist: dict = {}
    nxt = 0
    for step in range(12):
        # every fourth step: arrivals (a prefill chunk each, beside the others'
        # chunks or tokens); the steps between are pure decode steps
        prefill_step = step % 4 == 0
        arrivals = min(max_req - len(live), rng.randint(max(1, max_req // 4), max(1, max_req // 2))) \
            if prefill_step else 0
        for _ in range(arrivals):
            rid = f"r{nxt}"
            nxt += 1
            mgr.add_request(rid, ["main"])
            live.append(rid)
            hist[rid] = ([], [])
        if len(live) > 2 and rng.random() < 0.5:
            for rid in rng.sample(live, rng.randint(1, max(1, len(live) // 8))):
                live.remove(rid)
                mgr.remove_request(rid)
                del hist[rid]
        seq_lens = []
        for rid in live:
            if not hist[rid][0]:
                seq_lens.append(rng.randint(1, 300))  # first chunk of a new request
            elif prefill_step and rng.random() < 0.3:
                seq_lens.append(rng.randint(2, 40))
            else:
                seq_lens.append(1)
        cm = BatchedCacheManager(list(live), {r: "main" for r in live}, kv, mgr, bufs, cfg, gpu)
        cm.plan_attention(seq_lens, is_causal=True)
        n = sum(seq_lens)
        q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
        k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        log(f"manager sweep seed={seed} step={step}: {len(live)} requests, {n} tokens, "
            f"decode={all(x == 1 for x in seq_lens)}")
        out = cm.run_attention(q.to(gpu), k.to(gpu), v.to(gpu), layer_idx=0)
        ref = torch.zeros(n, hq, d)
        off = 0
        for rid, sl in zip(live, seq_lens):
            hk, hv = hist[rid]
            hk.append(k[off:off + sl])
            hv.append(v[off:off + sl])
            o, _ = A.attend(q[off:off + sl], torch.cat(hk), torch.cat(hv), causal=True, sm_scale=d ** -0.5)
            ref[off:off + sl] = o
            off += sl
        cm.advance_seq_lens()
        err = max_abs(out, ref)
        log(f"  max_abs={err:.3e}")
        assert err < 2e-2
    for rid in live:
        assert mgr.get_state(rid, "main").seq_len == sum(x.shape[0] for x in hist[rid][0])
