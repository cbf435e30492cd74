"""Parity at the sizes bench.py times, through bench.py's own step.

c2 (B=64), c3 and c5 (B=256) are set up by ``bench.setup`` (the full KV pool,
random pages, the steady-state FIFO free list) and stepped with
``bench.step_once`` (on the pool layers the bench cycles through): ``BatchedCacheManager.plan_attention([1]*B)`` (host FIFO
allocation, block-table delta, ``mi_pack_plan``), ``set_kv_cache``, ``run``
(decode + merge), ``advance_seq_lens``.  Three steps each; per step:

* the pack outputs (``qo_indptr``, ``kv_indptr``, ``kv_indices``,
  ``last_page_len``, write locations) and the allocator's free list equal the
  oracle's pack (``oracle.packing.pack``, ``cache_manager.py:272-322``) of the
  same request states and free list, bit for bit;
* the appended K/V rows at the write locations equal k and v (bf16) or the
  oracle's e4m3fn codes (fp8), bit for bit;
* the attention output is within max-abs 2e-2 (bf16 KV) / 6e-2 (fp8 KV) of
  fp32 attention computed on the GPU (gathered pages, GQA by
  ``repeat_interleave``) over the same cache after the append.

At B=256 the split-KV items of c3 (a plan over kv-head pairs: a quarter as
many items per head as a per-head plan) and c5 span several hundred pages
(the test logs the count and requires more than 256), so every decode
wavefront walks two or more 64-page windows of page ids.
"""

import math

import numpy as np
import pytest
import torch

import bench
from gpu_helpers import A, P, log

pytestmark = pytest.mark.gpu

TOL = {"bf16": 2e-2, "fp8": 6e-2}


def _ref_decode(q, layer, kv_indptr, kv_indices, last, hq, hkv, k_scale=None, v_scale=None):
    """fp32 decode attention per request on the GPU; fp8 pages dequantised with the per-head scales."""
    ps, d = layer.shape[2], layer.shape[-1]
    ip = kv_indptr.tolist()
    lst = last.tolist()
    idx = torch.as_tensor(kv_indices, device=q.device).long()
    out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    for r in range(len(lst)):
        pages = idx[ip[r]:ip[r + 1]]
        if pages.numel() == 0:
            continue
        kv_len = (pages.numel() - 1) * ps + lst[r]
        k = layer[pages, 0].reshape(-1, hkv, d)[:kv_len].float()
        v = layer[pages, 1].reshape(-1, hkv, d)[:kv_len].float()
        if k_scale is not None:
            k = k * k_scale.view(1, hkv, 1)
            v = v * v_scale.view(1, hkv, 1)
        k = k.repeat_interleave(hq // hkv, 1).permute(1, 2, 0).contiguous()  # [H, D, kv]
        v = v.repeat_interleave(hq // hkv, 1).transpose(0, 1).contiguous()  # [H, kv, D]
        s = torch.matmul(q[r].float().unsqueeze(1), k) / math.sqrt(d)  # [H, 1, kv]
        out[r] = torch.matmul(torch.softmax(s, dim=-1), v).squeeze(1)
    return out


@pytest.mark.parametrize("config", ["c2", "c3", "c5"])
def test_bench_step_parity(gpu, config):
    log(f"full-size {config}: setup")
    bt, cfg, kv, mgr, cm, rids, q, k, v = bench.setup(config, gpu)
    s = bt.spec
    b = len(rids)
    fp8 = s.kv_dtype == "fp8"
    for step in range(3):
        li = step % kv.shape[0]  # the bench cycles the pool's layers when one layer's pages fit the MALL
        layer = kv[li]
        ks, vs = bench._layer_scales(cm, li)
        states = [mgr.get_state(r, "main") for r in rids]
        ostates = [P.ReqState(pages=list(st.page_indices), seq_len=st.seq_len) for st in states]
        pool = P.FifoPages(0)
        pool.free.extend(mgr.page_allocator.free_pages)
        want = P.pack(ostates, [1] * b, pool, s.page_size)
        out = bench.step_once(cm, q, k, v, b, layer=li)
        qo, ip, idx, last, loc = cm._last_pack
        torch.cuda.synchronize()
        got = [t.cpu().numpy() for t in (qo, ip, idx, last, loc)]
        np.testing.assert_array_equal(got[0], want.qo_indptr)
        np.testing.assert_array_equal(got[1], want.kv_indptr)
        np.testing.assert_array_equal(got[2], want.kv_indices)
        np.testing.assert_array_equal(got[3], want.last_page_len)
        np.testing.assert_array_equal(got[4], want.kv_locations)
        assert list(mgr.page_allocator.free_pages) == list(pool.free)
        assert [st.page_indices for st in states] == [o.pages for o in ostates]
        # appended rows
        lp = torch.as_tensor(want.kv_locations[:, 0], device=gpu)
        ls = torch.as_tensor(want.kv_locations[:, 1], device=gpu)
        rows_k, rows_v = layer[lp, 0, ls], layer[lp, 1, ls]
        if fp8:
            ek, ev = A.quantize_e4m3(k.cpu(), ks.cpu()), A.quantize_e4m3(v.cpu(), vs.cpu())
            assert torch.equal(rows_k.cpu().view(torch.uint8), ek.view(torch.uint8))
            assert torch.equal(rows_v.cpu().view(torch.uint8), ev.view(torch.uint8))
        else:
            assert torch.equal(rows_k, k) and torch.equal(rows_v, v)
        ref = _ref_decode(q, layer, want.kv_indptr, want.kv_indices, want.last_page_len, s.num_qo_heads,
                          s.num_kv_heads, ks, vs)
        err = (out.float() - ref).abs().max().item()
        hdr = cm._plan_states["main"].wrapper._workspace[:16].view(torch.int32).cpu().tolist()
        log(f"  step {step}: pages={int(want.kv_indptr[-1])} items={hdr[2]} item_pages={hdr[3]} max_abs={err:.3e}")
        assert math.isfinite(err) and err < TOL[s.kv_dtype]
        if config != "c2":
            assert hdr[3] > 256, "B=256 items should span several 64-page windows per wavefront"
