"""GPU parity: RoPE fused with the paged K/V append (mi_rope_append).

The fused kernel must leave q, k and the whole cache bit-identical to
mi_rope_apply followed by mi_kv_append on the same inputs; both of those are
pinned against the CPU oracle (test_gpu_rope.py within the rotation bound,
test_gpu_append.py bit-exact).  The cache's K rows are also checked against the
oracle's rotation directly, within the same bound as test_gpu_rope.py.
"""

import pytest
import torch

from gpu_helpers import A, log, rope_bound
from mstar_amd import _lib
from mstar_amd import rope as MR
from mstar_amd.paged_attention import _append
from oracle import rope as R

pytestmark = pytest.mark.gpu

L31 = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)

CASES = [
    # dtype, cache dtype, D, rotary_dim, interleave, llama31, keep_k, idx_stride
    (torch.bfloat16, torch.bfloat16, 128, 128, False, None, True, 1),
    (torch.bfloat16, torch.bfloat16, 128, 128, False, None, False, 2),
    (torch.bfloat16, torch.float8_e4m3fn, 128, 128, False, None, True, 1),
    (torch.float16, torch.float16, 64, 64, True, None, True, 1),
    (torch.float16, torch.float8_e4m3fn, 128, 96, False, L31, True, 2),
    (torch.bfloat16, torch.bfloat16, 256, 256, True, None, False, 1),
    (torch.bfloat16, torch.float16, 128, 64, False, L31, True, 1),
    (torch.bfloat16, torch.bfloat16, 64, 32, True, None, True, 1),
    (torch.bfloat16, torch.float32, 128, 128, False, None, True, 1),
    (torch.float16, torch.float32, 256, 128, True, L31, False, 2),
]


def _inputs(seed, t, hq, hkv, d, dtype, pool, ps, idx_stride, gpu):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(t, hq, d, generator=g) * 2).to(dtype)
    k = (torch.randn(t, hkv, d, generator=g) * 2).to(dtype)
    v = (torch.randn(t, hkv, d, generator=g) * 2).to(dtype)
    slots = torch.randperm(pool * ps, generator=g)[:t]
    page, slot = slots // ps, slots % ps
    page[3], slot[5] = -1, ps  # skipped: page -1, slot past the page
    page[7] = pool             # skipped: page past the pool
    pos = torch.cat([torch.arange(6), torch.randint(0, 40000, (t - 6,), generator=g)])
    if idx_stride == 2:  # kv_cache_locations layout: (page, slot) pairs
        loc = torch.stack([page, slot], dim=1).contiguous().to(gpu)
        idx = (loc, loc.data_ptr() + 8)
    else:
        pg, sl = page.to(gpu), slot.to(gpu)
        idx = (pg, sl.data_ptr(), sl)
    return q, k, v, pos, idx


def _cache(pool, ps, hkv, d, dtype, gpu, seed):
    base = torch.randn(pool, 2, ps, hkv, d, generator=torch.Generator().manual_seed(seed))
    return base.to(dtype).to(gpu)


@pytest.mark.parametrize("dtype,cdt,d,rd,interleave,llama31,keep_k,idx_stride", CASES)
def test_rope_append_matches_rope_then_append(gpu, dtype, cdt, d, rd, interleave, llama31, keep_k, idx_stride):
    _check_rope_append(gpu, dtype, cdt, d, rd, interleave, llama31, keep_k, idx_stride, 12, 3)


@pytest.mark.parametrize("cdt", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("hq,hkv", [(6, 3), (5, 1), (1, 2)])
def test_rope_append_partial_q_head_groups(gpu, cdt, hq, hkv):
    """q head counts that leave the last group of four q heads partly empty."""
    _check_rope_append(gpu, torch.bfloat16, cdt, 128, 128, False, None, True, 1, hq, hkv)


def _check_rope_append(gpu, dtype, cdt, d, rd, interleave, llama31, keep_k, idx_stride, hq, hkv):
    t, pool, ps = 203, 64, 16
    n_append, n_dev = 190, 170  # tokens >= 170 are graph padding: rotated, not written
    q, k, v, pos, idx = _inputs(d + rd, t, hq, hkv, d, dtype, pool, ps, idx_stride, gpu)
    page_idx, slot_ptr = idx[0], idx[1]
    scales = (None, None)
    if cdt == torch.float8_e4m3fn:
        scales = (A.head_scales(k.float()).to(gpu), A.head_scales(v.float()).to(gpu))
    count = torch.tensor([n_dev], dtype=torch.int32, device=gpu)
    rope_kw = dict(rotary_dim=rd, interleave=interleave, rope_scale=8.0 if llama31 else 1.0,
                   rope_theta=500000.0 if llama31 else 10000.0)
    pos_g = pos.to(gpu)
    # two calls
    q1, k1, v1 = q.to(gpu), k.to(gpu), v.to(gpu)
    c1 = _cache(pool, ps, hkv, d, cdt, gpu, 3)
    if llama31:
        MR.apply_llama31_rope_pos_ids_inplace(q1, k1, pos_g, **rope_kw, **llama31)
    else:
        MR.apply_rope_pos_ids_inplace(q1, k1, pos_g, **rope_kw)
    _append(c1, k1, v1, page_idx, slot_ptr, idx_stride, n_append, count.data_ptr(), *scales)
    # fused
    q2, k2, v2 = q.to(gpu), k.to(gpu), v.to(gpu)
    c2 = _cache(pool, ps, hkv, d, cdt, gpu, 3)
    log(f"rope_append {dtype}->{cdt} D={d} rd={rd} il={interleave} l31={bool(llama31)} keep_k={keep_k} "
        f"stride={idx_stride}")
    MR.rope_append(q2, k2, v2, c2, pos_g, page_idx, slot_ptr, idx_stride, n_append, count.data_ptr(),
                   k_scale=scales[0], v_scale=scales[1], keep_k=keep_k, llama31=llama31, **rope_kw)
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu().view(torch.int16), q1.cpu().view(torch.int16))
    assert torch.equal(k2.cpu().view(torch.int16), (k1 if keep_k else k.to(gpu)).cpu().view(torch.int16))
    assert torch.equal(v2.cpu(), v)
    got, exp = c2.cpu().view(torch.uint8), c1.cpu().view(torch.uint8)
    log(f"  cache bytes differing: {(got != exp).sum().item()}")
    assert torch.equal(got, exp)
    if cdt == dtype:  # K rows of written tokens against the oracle's rotation
        page, slot = (idx[0][:, 0], idx[0][:, 1]) if idx_stride == 2 else (idx[0], idx[2])
        page, slot = page.cpu(), slot.cpu()
        ok = [i for i in range(n_dev) if 0 <= page[i] < pool and 0 <= slot[i] < ps]
        rows = c2.cpu()[page[ok], 0, slot[ok]]
        ref = R.rope(k[ok], pos[ok].numpy(), rotary_dim=rd, interleave=interleave, llama31=llama31, **{
            kk: vv for kk, vv in rope_kw.items() if kk not in ("rotary_dim", "interleave")})
        bound = rope_bound(k[ok], ref, pos[ok].numpy(), rd, interleave, rope_kw["rope_scale"], rope_kw["rope_theta"],
                           llama31)
        assert ((rows.double() - ref.double()).abs() <= bound).all()
        assert len(ok) == n_dev - 3


def test_rope_append_from_fused_projection_views(gpu):
    """q, k, v as views of one [tokens, (Hq + 2 Hkv) * D] projection output."""
    t, hq, hkv, d, pool, ps = 33, 8, 2, 128, 16, 16
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    pos = torch.arange(50, 50 + t, device=gpu)
    page = torch.arange(t, device=gpu) // ps
    slot = torch.arange(t, device=gpu) % ps

    def views(x):
        return (x[:, : hq * d].view(t, hq, d), x[:, hq * d:(hq + hkv) * d].view(t, hkv, d),
                x[:, (hq + hkv) * d:].view(t, hkv, d))

    a, b = qkv.to(gpu), qkv.to(gpu)
    c1 = torch.zeros(pool, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    c2 = torch.zeros_like(c1)
    q1, k1, v1 = views(a)
    MR.apply_rope_pos_ids_inplace(q1, k1, pos)
    _append(c1, k1, v1, page, slot.data_ptr(), 1, t, None, None, None)
    q2, k2, v2 = views(b)
    MR.rope_append(q2, k2, v2, c2, pos, page, slot.data_ptr(), 1, t, None)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())
    assert torch.equal(c1.cpu(), c2.cpu())


def test_rope_append_rejects_bad_arguments(gpu):
    t, hkv, d = 4, 2, 64
    q = torch.zeros(t, 4, d, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(t, hkv, d, dtype=torch.bfloat16, device=gpu)
    cache = torch.zeros(2, 2, 16, hkv, d, dtype=torch.bfloat16, device=gpu)
    idx = torch.zeros(t, dtype=torch.long, device=gpu)
    pos = torch.arange(t, device=gpu)
    with pytest.raises(ValueError):  # v dtype differs
        MR.rope_append(q, k, k.float(), cache, pos, idx, idx.data_ptr(), 1, t, None)
    with pytest.raises(ValueError):  # k heads do not match the cache
        MR.rope_append(q, q, q, cache, pos, idx, idx.data_ptr(), 1, t, None)
    with pytest.raises(ValueError):  # more append tokens than k holds
        MR.rope_append(q, k, k.clone(), cache, pos, idx, idx.data_ptr(), 1, t + 1, None)
    with pytest.raises(ValueError):  # k rows not 16-byte aligned
        kk = torch.zeros(t * hkv * d + 4, dtype=torch.bfloat16, device=gpu)[4:].view(t, hkv, d)
        MR.rope_append(q, kk, k.clone(), cache, pos, idx, idx.data_ptr(), 1, t, None)


def _manager(gpu, kv_dtype, scales=None):
    from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
    from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager

    hq, hkv, d, ps, pages = 16, 4, 128, 16, 512
    cfg = KVCacheConfig(num_layers=2, num_kv_heads=hkv, head_dim=d, max_seq_len=8192, max_num_pages=pages,
                        page_size=ps, num_qo_heads=hq)
    kv = torch.zeros(2, pages, 2, ps, hkv, d, dtype=kv_dtype, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    rids = [f"r{i}" for i in range(6)]
    for i, r in enumerate(rids):
        mgr.add_request(r, ["main"])
        mgr.get_state(r, "main").position_id_start = 100 * i
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    return BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu, kv_scales=scales), cfg


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float32])
def test_manager_fused_rope_attention_matches_two_calls(gpu, kv_dtype):
    """apply_rope_and_run_attention == apply_rope + run_attention: prefill step then decode steps."""
    scales = None
    if kv_dtype == torch.float8_e4m3fn:
        scales = torch.full((2, 2, 4), 0.05, dtype=torch.float32, device=gpu)
    cm1, cfg = _manager(gpu, kv_dtype, scales)
    cm2, _ = _manager(gpu, kv_dtype, scales)
    g = torch.Generator().manual_seed(11)
    steps = [[37, 120, 5, 64, 1, 300], [1] * 6, [1] * 6, [3, 1, 1, 9, 1, 1]]
    for step, seq_lens in enumerate(steps):
        t = sum(seq_lens)
        q = torch.randn(t, cfg.num_qo_heads, cfg.head_dim, generator=g).to(torch.bfloat16).to(gpu)
        k = torch.randn(t, cfg.num_kv_heads, cfg.head_dim, generator=g).to(torch.bfloat16).to(gpu)
        v = torch.randn(t, cfg.num_kv_heads, cfg.head_dim, generator=g).to(torch.bfloat16).to(gpu)
        outs = []
        for fused, cm in ((False, cm1), (True, cm2)):
            cm.plan_attention(seq_lens)
            cm.plan_rope(seq_lens)
            cm.set_layer_idx(step % 2)
            qq, kk, vv = q.clone(), k.clone(), v.clone()
            if fused:
                outs.append(cm.apply_rope_and_run_attention(qq, kk, vv, rope_theta=500000.0))
            else:
                qr, kr = cm.apply_rope(qq, kk, rope_theta=500000.0)
                outs.append(cm.run_attention(qr, kr, vv))
            cm.advance_seq_lens()
        torch.cuda.synchronize()
        log(f"manager fused step {step}: tokens {t}, kv {kv_dtype}")
        assert torch.equal(outs[0].cpu().view(torch.int16), outs[1].cpu().view(torch.int16))
        assert torch.equal(cm1.kv_cache.cpu().view(torch.uint8), cm2.kv_cache.cpu().view(torch.uint8))
