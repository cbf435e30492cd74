"""Multi-label (CFG) planning on the GPU path against the CPU oracle.

* ``snapshot_all``: page bookkeeping equal to the oracle's (same FIFO page
  ids, same copy pairs) and the destination pages bit-identical to the
  source pages in every layer, for a first copy, a later copy of a grown
  history (leading pages kept) and a ``realloc`` copy.
* ``plan_attention_batched_cfg`` + ``plan_rope_batched_cfg``: one ragged batch
  of (label, request) entries, label-major; positions bit-exact; every
  entry's attention within 2e-2 of fp32 attention over that label's
  history plus the step's rotated tokens (non-causal, as BAGEL image
  generation runs it).
"""

import numpy as np
import pytest
import torch

from gpu_helpers import A, P, log, max_abs
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from oracle import rope as R

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS, LAYERS, POOL = 8, 2, 64, 16, 2, 256


def _setup(gpu, rids, labels):
    cfg = KVCacheConfig(num_layers=LAYERS, num_kv_heads=HKV, head_dim=D, max_seq_len=4096, max_num_pages=POOL,
                        page_size=PS, num_qo_heads=HQ)
    kv = torch.zeros(LAYERS, POOL, 2, PS, HKV, D, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    for r in rids:
        mgr.add_request(r, labels)
    return cfg, kv, mgr, WorkspaceBufferManager(32 << 20, gpu)


def _step(cm, seq_lens, label, g, gpu):
    """One eager step for ``label``: plan, random K/V for every layer, advance."""
    cm.set_active_label(label)
    cm.plan_attention(seq_lens, label=label)
    n = sum(seq_lens)
    for layer in range(LAYERS):
        q = torch.randn(n, HQ, D, generator=g).to(torch.bfloat16).to(gpu)
        k = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16).to(gpu)
        v = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16).to(gpu)
        cm.run_attention(q, k, v, layer_idx=layer)
    cm.advance_seq_lens()


def test_snapshot_all_matches_oracle(gpu):
    rids = ["a", "b", "c"]
    cfg, kv, mgr, bufs = _setup(gpu, rids, ["main", "cfg_text"])
    g = torch.Generator().manual_seed(0)
    prompts = [37, 16, 90]
    # oracle bookkeeping in lockstep with the manager's FIFO allocator
    pool = P.FifoPages(POOL)
    main = [P.ReqState() for _ in rids]
    text = [P.ReqState() for _ in rids]
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
    _step(cm, prompts, "main", g, gpu)
    P.pack(main, prompts, pool, PS)
    for st, n in zip(main, prompts):
        st.seq_len += n

    def check(realloc):
        nonlocal text
        cm2 = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
        cm2.snapshot_all("main", "cfg_text", realloc=realloc)
        new_text = []
        for i, r in enumerate(rids):
            t, _ = P.snapshot(main[i], text[i], pool, PS, realloc=realloc)
            new_text.append(t)
            got = mgr.get_state(r, "cfg_text")
            assert got.page_indices == t.pages and got.seq_len == t.seq_len
            assert got.position_id_start == mgr.get_state(r, "main").position_id_start
        text = new_text
        torch.cuda.synchronize()
        for r in rids:
            src = mgr.get_state(r, "main").page_indices
            dst = mgr.get_state(r, "cfg_text").page_indices
            assert torch.equal(kv[:, dst].cpu(), kv[:, src].cpu())

    check(False)
    # main grows by a decode step and a prefill chunk; snapshot again (leading pages kept)
    _step(BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu), [1, 1, 1], "main", g, gpu)
    P.pack(main, [1, 1, 1], pool, PS)
    for st in main:
        st.seq_len += 1
    _step(BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu), [20, 3, 33], "main", g, gpu)
    P.pack(main, [20, 3, 33], pool, PS)
    for st, n in zip(main, [20, 3, 33]):
        st.seq_len += n
    check(False)
    check(True)
    assert list(mgr.page_allocator.free_pages) == list(pool.free)


def test_batched_cfg_plan_and_attention(gpu):
    rids = ["a", "b"]
    labels = ["main", "cfg_text", "cfg_img"]
    cfg, kv, mgr, bufs = _setup(gpu, rids, labels)
    g = torch.Generator().manual_seed(1)
    mk = lambda: BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)  # noqa: E731
    _step(mk(), [40, 23], "main", g, gpu)
    mk().snapshot_all("main", "cfg_text")
    _step(mk(), [5, 9], "main", g, gpu)      # main moves on past the snapshot
    _step(mk(), [17, 64], "cfg_img", g, gpu)  # an unrelated history
    for r, p in zip(rids, (100, 7)):
        mgr.get_state(r, "cfg_img").position_id_start = p
    torch.cuda.synchronize()
    hist = {}
    for label in labels:
        for r in rids:
            st = mgr.get_state(r, label)
            hist[(label, r)] = [A.gather_request_kv(kv[layer].cpu(), np.asarray(st.page_indices), st.seq_len)
                                for layer in range(LAYERS)]
    starts = {(label, r): mgr.get_state(r, label).position_id_start for label in labels for r in rids}

    cm = mk()
    n_img = 12
    seq_lens = [n_img] * len(rids)
    cm.plan_attention_batched_cfg(labels, seq_lens, is_causal=False)
    cm.plan_rope_batched_cfg(labels, seq_lens, per_label_pos_ids={"cfg_text": []})
    entries = [(label, r) for label in labels for r in rids]
    pos = cm._plan_states["_cfg_batched"].pos_ids.cpu().numpy()
    expect = np.concatenate([R.positions([n_img], [starts[e]]) for e in entries])
    assert pos.tolist() == expect.tolist()
    cm.set_active_label("_cfg_batched")
    n = n_img * len(entries)
    worst = 0.0
    for layer in range(LAYERS):
        q = torch.randn(n, HQ, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16)
        qr, kr = cm.apply_rope(q.to(gpu), k.to(gpu), rope_theta=1e4)
        out = cm.run_attention(qr, kr, v.to(gpu), layer_idx=layer).cpu()
        q_rot = R.rope(q, expect, rope_theta=1e4)
        k_rot = R.rope(k, expect, rope_theta=1e4)
        for j, e in enumerate(entries):
            sl = slice(j * n_img, (j + 1) * n_img)
            hk, hv = hist[e][layer]
            o, _ = A.attend(q_rot[sl], torch.cat([hk.float(), k_rot[sl]]), torch.cat([hv.float(), v[sl].float()]),
                            causal=False, sm_scale=D ** -0.5)
            worst = max(worst, max_abs(out[sl], o))
    log(f"batched cfg: entries={len(entries)} max_abs={worst:.3e}")
    assert worst < 2e-2
    # every entry's new tokens went to its own label's pages
    for label in labels:
        for r in rids:
            assert mgr.get_state(r, label).seq_len == hist[(label, r)][0][0].shape[0]  # not advanced
