"""The CUDA-graph decode loop of M*'s graph runner, on the GPU path.

Mirrors ``CudaGraphRunner`` (``mstar/engine/cuda_graph_runner.py:289-362,
967-1084``): two double-buffer slots, each with a persistent decode wrapper
(``use_cuda_graph=True``, fixed batch), a static ``pos_ids`` buffer, static
q/k/v inputs and a static ``BatchedCacheManager`` over ``cuda_graph_plan_states``;
one captured graph per slot runs every layer's ``apply_rope`` +
``run_attention``.  Each step pre-plans the next slot on a separate plan
stream (``plan_attention`` into the slot's wrapper, ``_pre_planned_labels``
+ a plan-done event), pads the real batch with dummy requests, replays, and
checks every real request against a list-history oracle (RoPE'd K/V appended
per step, fp32 attention over the whole history, max-abs <= 2e-2).

With ``plan_thread`` the pre-plan runs as in M*'s worker
(``cuda_graph_runner.py:1031-1078``, ``:1375-1396``): on a plan thread
(one-worker executor) that starts once the replaying step has advanced its
request states, while the engine thread frees the replayed slot's padding
states and checks the outputs; the allocator, the device block table and the
shared pinned uploader are then used from two threads at once.
"""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gpu_helpers import A, log, max_abs
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager, _PlanState
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from mstar_amd.paged_attention import FlashInferDecodeWrapper
from oracle import rope as R

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS, LAYERS, BS, POOL = 16, 4, 128, 16, 2, 8, 1024
THETA = 1e6


def _slot(gpu, bufs, cfg, kv, mgr, dummies, slot):
    w = FlashInferDecodeWrapper(bufs.get(f"main_cugraph_slot{slot}"), HQ, HKV, D, PS, batch_size=BS,
                                max_num_pages=POOL, device=gpu, use_cuda_graph=True)
    states = {"main": _PlanState(wrapper=w, pos_ids=torch.zeros(BS, dtype=torch.long, device=gpu))}
    cm = BatchedCacheManager(list(dummies), {r: "main" for r in dummies}, kv, mgr, bufs, cfg, gpu,
                             cuda_graph_plan_states=states)
    q = torch.zeros(LAYERS, BS, HQ, D, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(LAYERS, BS, HKV, D, dtype=torch.bfloat16, device=gpu)
    v = torch.zeros(LAYERS, BS, HKV, D, dtype=torch.bfloat16, device=gpu)
    return {"cm": cm, "q": q, "k": k, "v": v, "out": None, "graph": None}


def _forward(s):
    outs = []
    for layer in range(LAYERS):
        q, k = s["cm"].apply_rope(s["q"][layer], s["k"][layer], rope_theta=THETA)
        outs.append(s["cm"].run_attention(q, k, s["v"][layer], layer_idx=layer))
    return torch.stack(outs)


@pytest.mark.parametrize("plan_thread", [False, True])
def test_double_buffered_decode_graphs(gpu, plan_thread):
    cfg = KVCacheConfig(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, max_seq_len=4096, max_num_pages=POOL,
                        page_size=PS, num_qo_heads=HQ)
    kv = torch.zeros(LAYERS, POOL, 2, PS, HKV, D, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    g = torch.Generator().manual_seed(0)

    # -- real requests: an eager prefill step (prompt K/V go into the history as rotated)
    real = [f"r{i}" for i in range(BS)]
    for r in real:
        mgr.add_request(r, ["main"])
    prompts = [37, 1, 200, 16, 90, 15, 33, 64]
    hist = {(r, l): ([], []) for r in real for l in range(LAYERS)}
    cm0 = BatchedCacheManager(real, {r: "main" for r in real}, kv, mgr, bufs, cfg, gpu)
    cm0.plan_attention(prompts)
    cm0.plan_rope(prompts)
    pos0 = R.positions(prompts, [0] * BS)
    n0 = sum(prompts)
    for layer in range(LAYERS):
        q = torch.randn(n0, HQ, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n0, HKV, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n0, HKV, D, generator=g).to(torch.bfloat16)
        qr, kr = cm0.apply_rope(q.to(gpu), k.to(gpu), rope_theta=THETA)
        cm0.run_attention(qr, kr, v.to(gpu), layer_idx=layer)
        k_rot = R.rope(k, pos0, rope_theta=THETA)
        off = 0
        for r, sl in zip(real, prompts):
            hist[(r, layer)][0].append(k_rot[off:off + sl])
            hist[(r, layer)][1].append(v[off:off + sl].float())
            off += sl
    cm0.advance_seq_lens()

    # -- two slots, each captured once with its dummy batch planned
    dummies = [[f"__cg_slot{s}_{i}__" for i in range(BS)] for s in range(2)]
    slots = []
    for s in range(2):
        for r in dummies[s]:
            mgr.add_request(r, ["main"])
        sl = _slot(gpu, bufs, cfg, kv, mgr, dummies[s], s)
        sl["cm"].plan_attention([1] * BS)
        sl["cm"].plan_rope([1] * BS)
        side = torch.cuda.Stream(device=gpu)
        side.wait_stream(torch.cuda.current_stream(gpu))
        with torch.cuda.stream(side):
            _forward(sl)  # warm-up outside capture
        torch.cuda.current_stream(gpu).wait_stream(side)
        sl["graph"] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(sl["graph"]):
            sl["out"] = _forward(sl)
        for r in dummies[s]:
            mgr.reset_label(r, "main", free=True)
        slots.append(sl)
    torch.cuda.synchronize()

    plan_stream = torch.cuda.Stream(device=gpu)
    replay_done = [None, None]

    def pre_plan(slot, live):
        """pre_plan_for_batch (cuda_graph_runner.py:967-1056): real rids first, dummies pad.

        Runs on the plan stream while the other slot replays; it only waits
        for this slot's previous replay (whose static buffers it rewrites).
        """
        cm = slots[slot]["cm"]
        cm.request_ids = list(live) + dummies[slot][len(live):]
        cm.active_labels = {r: "main" for r in cm.request_ids}
        if replay_done[slot] is not None:
            plan_stream.wait_event(replay_done[slot])
        with torch.cuda.stream(plan_stream):
            cm.plan_attention([1] * BS, label="main")
            cm.plan_rope([1] * BS, label="main")
        ev = torch.cuda.Event()
        ev.record(plan_stream)
        cm._pre_planned_labels = {"main"}
        cm._plan_done_event = ev
        return ev

    live = list(real)
    schedule = [8, 8, 8, 6, 6, 5, 5, 8]  # real batch per step; finished requests leave, padding fills
    ev = pre_plan(0, live)
    main = torch.cuda.current_stream(gpu)
    executor = ThreadPoolExecutor(max_workers=1) if plan_thread else None
    fut = None
    for step, nreal in enumerate(schedule):
        s = step % 2
        sl = slots[s]
        if fut is not None:
            ev = fut.result()  # this slot's pre-plan, run on the plan thread
            fut = None
        live_now = list(sl["cm"].request_ids[:len(live)])
        starts = [mgr.get_state(r, "main").position_id_start for r in live_now]
        # inputs for this step (real rows; padded rows get zeros)
        qs = torch.randn(LAYERS, len(live_now), HQ, D, generator=g).to(torch.bfloat16)
        ks = torch.randn(LAYERS, len(live_now), HKV, D, generator=g).to(torch.bfloat16)
        vs = torch.randn(LAYERS, len(live_now), HKV, D, generator=g).to(torch.bfloat16)
        for name, x in (("q", qs), ("k", ks), ("v", vs)):
            sl[name].zero_()
            sl[name][:, : len(live_now)].copy_(x.to(gpu))
        main.wait_event(ev)
        sl["cm"].plan_attention([1] * BS)  # consumes the pre-planned label (fast path)
        sl["graph"].replay()
        replay_done[s] = torch.cuda.Event()
        replay_done[s].record(main)
        # host bookkeeping of the step while the replay runs: advance, free padding,
        # batch changes, then pre-plan the other slot on the plan stream
        sl["cm"].advance_seq_lens()
        if not plan_thread:
            for r in dummies[s][len(live_now):]:
                mgr.reset_label(r, "main", free=True)
        if step + 1 < len(schedule):
            nxt = schedule[step + 1]
            while len(live) > nxt:  # a request finishes: its pages go back to the pool
                mgr.remove_request(live.pop())
            while len(live) < nxt:  # a new request joins with an empty history
                r = f"n{step}_{len(live)}"
                mgr.add_request(r, ["main"])
                hist.update({(r, l): ([], []) for l in range(LAYERS)})
                live.append(r)
            if plan_thread:
                fut = executor.submit(pre_plan, (step + 1) % 2, list(live))
            else:
                ev = pre_plan((step + 1) % 2, live)
        if plan_thread:  # engine-thread bookkeeping while the plan thread allocates
            for r in dummies[s][len(live_now):]:
                mgr.reset_label(r, "main", free=True)
        torch.cuda.synchronize()
        out = sl["out"].clone()
        worst = 0.0
        for layer in range(LAYERS):
            q_rot = R.rope(qs[layer], np.array(starts), rope_theta=THETA)
            k_rot = R.rope(ks[layer], np.array(starts), rope_theta=THETA)
            for i, r in enumerate(live_now):
                hk, hv = hist[(r, layer)]
                hk.append(k_rot[i:i + 1])
                hv.append(vs[layer][i:i + 1].float())
                o, _ = A.attend(q_rot[i:i + 1], torch.cat(hk), torch.cat(hv), causal=False, sm_scale=D ** -0.5)
                worst = max(worst, max_abs(out[layer, i:i + 1], o))
        log(f"step {step} slot {s}: real={len(live_now)} max_abs={worst:.3e}")
        assert worst < 2e-2
    if executor is not None:
        executor.shutdown()
