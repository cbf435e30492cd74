"""GPU parity: packing (mi_pack via BatchedCacheManager) and the decode plan are bit-exact.

Multi-step scenarios drive our host allocator and the oracle's FIFO restatement
side by side (prefill, decode steps, request removal with page reuse), and
compare every packed tensor the GPU produces with the oracle's.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import P, log, workspace
from mstar_amd import _lib
from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import AllocationFailedError, KVCacheConfig, PagedAllocationManager

pytestmark = pytest.mark.gpu


def _setup(gpu, max_pages, ps=16, hq=8, hkv=2, d=128, max_seq_len=8192):
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=hkv, head_dim=d, max_seq_len=max_seq_len,
                        max_num_pages=max_pages, page_size=ps, num_qo_heads=hq)
    kv = torch.zeros(1, max_pages, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    return cfg, kv, mgr


def _check_step(cm, rids, label, seq_lens, ostates, opool, ps):
    cm.plan_attention(seq_lens, label=label)
    ref = P.pack(ostates, seq_lens, opool, ps)
    qo, kv_indptr, kv_indices, last, loc = cm._last_pack
    torch.cuda.synchronize()
    assert qo.cpu().numpy().tolist() == ref.qo_indptr.tolist()
    assert kv_indptr.cpu().numpy().tolist() == ref.kv_indptr.tolist()
    assert kv_indices.cpu().numpy().tolist() == ref.kv_indices.tolist()
    assert last.cpu().numpy().tolist() == ref.last_page_len.tolist()
    if ref.kv_locations is not None:
        assert loc.cpu().numpy().tolist() == ref.kv_locations.tolist()
    for st, sl in zip(ostates, seq_lens):
        st.seq_len += sl


def test_pack_multi_step_with_reuse(gpu):
    ps = 16
    cfg, kv, mgr = _setup(gpu, max_pages=3000, ps=ps)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    opool = P.FifoPages(3000)
    rng = np.random.default_rng(0)
    rids = [f"r{i}" for i in range(40)]
    for r in rids:
        mgr.add_request(r, ["main"])
    ostate = {r: P.ReqState() for r in rids}
    live = list(rids)
    for step in range(12):
        if step == 0:
            seq_lens = rng.integers(1, 900, size=len(live)).tolist()  # prefill
        elif step % 4 == 3:
            seq_lens = rng.integers(0, 40, size=len(live)).tolist()   # ragged chunk, zeros allowed
        else:
            seq_lens = [1] * len(live)                                  # decode
        cm = BatchedCacheManager(live, {r: "main" for r in live}, kv, mgr, bufs, cfg, gpu)
        log(f"pack step {step}: B={len(live)} tokens={sum(seq_lens)}")
        _check_step(cm, live, "main", seq_lens, [ostate[r] for r in live], opool, ps)
        for r, sl in zip(live, seq_lens):
            mgr.get_state(r, "main").seq_len += sl
        if step % 3 == 2:  # finish a few requests, start new ones: pages get reused
            for r in list(live[:5]):
                mgr.remove_request(r)
                opool.give(ostate[r].pages)
                live.remove(r)
            for j in range(5):
                r = f"n{step}_{j}"
                mgr.add_request(r, ["main"])
                ostate[r] = P.ReqState()
                live.append(r)


def test_pack_allocation_failure_is_raised_before_launch(gpu):
    cfg, kv, mgr = _setup(gpu, max_pages=10)
    bufs = WorkspaceBufferManager(16 << 20, gpu)
    for r in ("a", "b"):
        mgr.add_request(r, ["main"])
    cm = BatchedCacheManager(["a", "b"], {"a": "main", "b": "main"}, kv, mgr, bufs, cfg, gpu)
    with pytest.raises(AllocationFailedError) as e:
        cm.plan_attention([100, 100])
    assert e.value.request_id == "b" and e.value.pages_short == 4  # 7 pages asked, 3 left
    assert len(mgr.get_state("a", "main").page_indices) == 7  # earlier request keeps its pages


def _split_layout(batch, nkv, d, units=4096):
    target = max(16, units // (4 * nkv))
    max_chunks = target + batch  # the workspace below is large enough for the full budget
    align = lambda x: (x + 255) // 256 * 256
    hdr = 0
    chunk_indptr = 256
    work = align(chunk_indptr + 4 * (batch + 1))
    return hdr, chunk_indptr, work, max_chunks


@pytest.mark.parametrize("lens,pool,hq,hkv", [
    ([0, 1, 16, 17, 300, 5000, 32768, 4096, 77], 4000, 32, 4),
    # a small job whose item size falls strictly inside the search range (21 pages on 256 CUs)
    ([2000] * 20 + [0, 5], 3000, 32, 4),
    # a small job whose items cannot fit the slots at any size: the minimum chunk
    # (below the batch size that pairs kv-heads, which this plan model leaves out)
    ([1000] * 100, 7000, 24, 8),
])
def test_decode_plan_partition(gpu, lens, pool, hq, hkv):
    from gpu_helpers import custom_batch

    log(f"decode plan partition: {len(lens)} requests, {sum(lens)} tokens")
    qo, kv_indptr, kv_indices, last = custom_batch(lens, 16, pool, seed=2)
    d = 128
    ws = workspace(gpu, 256 << 20)
    loc = torch.full((len(lens), 2), -7, dtype=torch.long, device=gpu)
    ti = lambda x: torch.as_tensor(x).to(gpu)
    a, b_, c = ti(kv_indptr), ti(kv_indices), ti(last)
    _lib.check(_lib.lib().mi_decode_plan(None, a.data_ptr(), b_.data_ptr(), c.data_ptr(), len(lens), 16, hq, hkv, d,
                                         loc.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr()), "plan")
    torch.cuda.synchronize()
    hdr, ci, wk, max_chunks = _split_layout(len(lens), hkv, d)
    h = ws[hdr:hdr + 20].cpu().view(torch.int32).tolist()
    # a small job is cut for the CUs: two items per CU per kv-head at head_dim 128
    assert len(lens) < 128, "a paired-head plan has another split target"
    slots = min(torch.cuda.get_device_properties(0).multi_processor_count * 2 // hkv, max_chunks)
    cp, nchunks = P.split_chunks(kv_indptr, 16, 4096, hkv, slots=slots)
    log(f"  slots={slots} item pages: plan {h[3]}, oracle {cp}")
    assert h[0] == 0x4D494450 and h[1] == len(lens) and h[3] == cp and h[2] == int(nchunks.sum())
    cptr = ws[ci:ci + 4 * (len(lens) + 1)].cpu().view(torch.int32).numpy()
    assert cptr.tolist() == [0] + np.cumsum(nchunks).tolist()
    work = ws[wk:wk + 16 * h[2]].cpu().view(torch.int32).numpy().reshape(-1, 4)
    npages = np.diff(kv_indptr)
    # items: (request, index within request, end page, items of request); start page = index * cp
    sizes = [min(e, npages[r]) - k * cp for r, k, e, _ in work]
    nfull = sum(1 for z in sizes if z == cp)
    assert all(z == cp for z in sizes[:nfull]), f"full items come first: cp={cp} work={work.tolist()}"
    buckets = [(z * 64 - 1) // cp for z in sizes[nfull:]]
    assert buckets == sorted(buckets, reverse=True), "remainders ordered by descending size bucket"
    for r in range(len(lens)):
        rows = sorted((int(k), int(e)) for rr, k, e, n in work if rr == r)
        assert all(n == nchunks[r] for rr, _, _, n in work if rr == r)
        assert [k for k, _ in rows] == list(range(nchunks[r]))
        covered = [p for k, e in rows for p in range(k * cp, e)]
        assert covered == list(range(npages[r]))
    # locations: (last page, last_page_len - 1); (-1, -1) for a request without pages
    exp = []
    for r in range(len(lens)):
        if npages[r] == 0:
            exp.append([-1, -1])
        else:
            exp.append([int(kv_indices[kv_indptr[r + 1] - 1]), int(last[r]) - 1])
    assert loc.cpu().tolist() == exp


@pytest.mark.parametrize("with_plan", [True, False])
@pytest.mark.parametrize("nreq", [64, 200])
def test_pack_plan_host_matches_device_metadata(gpu, with_plan, nreq):
    """mi_pack_plan_host (metadata as the kernel argument) == mi_pack_plan / mi_pack with
    the same metadata in device memory: packed arrays, table rows and plan.  64 requests
    pass the metadata as given, 200 requests (more than MI_PACK_HOST_ARGS values) in the
    argument's compact form."""
    from mstar_amd.cache_manager import _step_tensors

    ps, hq, hkv, d = 16, 24, 8, 128
    rng = np.random.default_rng(11)
    lens = [0, 1, 16, 17] + rng.integers(1, 3000, size=nreq - 4).tolist()
    b = len(lens)
    npages = np.array([(t + ps - 1) // ps for t in lens], dtype=np.int32)
    # a decode step: all but the last page or two of each list are already in the table
    old = np.maximum(npages - rng.integers(0, 3, size=b), 0).astype(np.int32)
    stride = int(npages.max()) + 1
    pool = torch.randperm(int(npages.sum()) + 64, generator=torch.Generator().manual_seed(5)).numpy().astype(np.int32)
    rows = np.zeros((b, stride), dtype=np.int32)
    new_pages, off = [], 0
    for r in range(b):
        rows[r, :npages[r]] = pool[off:off + npages[r]]
        new_pages.append(rows[r, old[r]:npages[r]])
        off += npages[r]
    meta = np.empty((5, b), dtype=np.int32)
    meta[0] = rng.permutation(b)                 # slots
    meta[1] = np.maximum(np.array(lens) - 1, 0)  # seq_len before the step
    meta[2] = 1
    meta[3] = npages
    meta[4] = old
    flat = np.concatenate([meta.reshape(-1)] + new_pages).astype(np.int32)
    if nreq == 64:
        assert flat.size <= _lib.PACK_HOST_META
    else:  # beyond the argument as given, within its compact form
        assert flat.size > 896 and 3 * b + (flat.size - 5 * b) <= 896
    dmeta = torch.from_numpy(flat).to(gpu)
    base = dmeta.data_ptr()
    table0 = np.zeros((b, stride), dtype=np.int32)
    for r in range(b):
        table0[meta[0][r], :old[r]] = rows[r, :old[r]]
    outs = []
    for host in (False, True):
        ws = workspace(gpu, 64 << 20)
        ws.zero_()
        table = torch.from_numpy(table0).to(gpu)
        qo, ip, idx, last, loc = _step_tensors(b, int(npages.sum()), True, gpu)
        wsp, wsn = (ws.data_ptr(), ws.numel()) if with_plan else (None, 0)
        L = _lib.lib()
        if host:
            _lib.check(L.mi_pack_plan_host(flat.ctypes.data, flat.size, b, table.data_ptr(), stride, ps, qo.data_ptr(),
                                           ip.data_ptr(), idx.data_ptr(), last.data_ptr(), loc.data_ptr(), 3, hq, hkv,
                                           d, wsp, wsn, _lib.stream_ptr()), "pack_plan_host")
        else:
            args = [base, base + 4 * b, base + 8 * b, base + 12 * b, b, table.data_ptr(), stride, base + 16 * b,
                    base + 20 * b, ps, qo.data_ptr(), ip.data_ptr(), idx.data_ptr(), last.data_ptr(), loc.data_ptr(), 3]
            if with_plan:
                _lib.check(L.mi_pack_plan(*args, hq, hkv, d, wsp, wsn, _lib.stream_ptr()), "pack_plan")
            else:
                _lib.check(L.mi_pack(*args, _lib.stream_ptr()), "pack")
        torch.cuda.synchronize()
        outs.append(([t.cpu().tolist() for t in (qo, ip, idx, last, loc)], table.cpu().tolist(),
                     ws[:1 << 16].cpu().tolist() if with_plan else None))
    assert outs[0][:2] == outs[1][:2]
    if with_plan:
        # The plan: header and item offsets equal; the work list equal as a set
        # (items of one size bucket are placed by LDS atomics, whose order across
        # the plan workgroup's wavefronts varies from run to run).
        ws0, ws1 = (np.array(o[2], dtype=np.uint8).view(np.int32) for o in outs)
        assert ws0[:5].tolist() == ws1[:5].tolist()
        ci = 64  # item offsets at byte 256
        assert ws0[ci:ci + b + 1].tolist() == ws1[ci:ci + b + 1].tolist()
        wk = -(-(256 + 4 * (b + 1)) // 256) * 64  # work list, 256-byte aligned after the offsets
        n = int(ws0[2])
        w0, w1 = (sorted(map(tuple, w[wk:wk + 4 * n].reshape(-1, 4).tolist())) for w in (ws0, ws1))
        assert w0 == w1
    # and the packed page lists are the requests' lists
    ip_h, idx_h = np.array(outs[1][0][1]), np.array(outs[1][0][2])
    for r in range(b):
        assert idx_h[ip_h[r]:ip_h[r + 1]].tolist() == rows[r, :npages[r]].tolist()


@pytest.mark.parametrize("extra", [300, 1100])
def test_pack_plan_matches_pack_then_plan(gpu, extra):
    """mi_pack_plan (one launch) == mi_pack followed by mi_decode_plan on the packed arrays,
    and the packed arrays are the closed-form ones; 1108 requests take the pack's and the
    plan's loops over several 1024-request windows."""
    from mstar_amd.cache_manager import _step_tensors

    ps, hq, hkv, d = 16, 32, 4, 128
    rng = np.random.default_rng(7)
    lens = [0, 1, 17, 300, 5000, 32768, 4096, 77] + rng.integers(1, 20000 if extra < 1024 else 2000,
                                                                 size=extra).tolist()
    b = len(lens)
    npages = [(t + ps - 1) // ps for t in lens]
    pool = torch.randperm(sum(npages) + 64, generator=torch.Generator().manual_seed(3)).numpy().astype(np.int32)
    stride = max(npages) + 1
    table = torch.zeros(b, stride, dtype=torch.int32, device=gpu)
    meta = np.empty((5, b), dtype=np.int32)
    meta[0] = np.arange(b)                      # slots
    meta[1] = np.maximum(np.array(lens) - 1, 0)  # seq_len before the step
    meta[2] = 1                                  # one new token each
    meta[3] = npages
    meta[4] = 0                                  # nothing in the table yet: every page is new
    flat = np.concatenate([meta.reshape(-1), pool[:sum(npages)]])
    dmeta = torch.from_numpy(flat).to(gpu)
    base = dmeta.data_ptr()
    outs = []
    for fused in (False, True):
        ws = workspace(gpu, 64 << 20)
        ws.zero_()
        table.zero_()
        qo, ip, idx, last, loc = _step_tensors(b, sum(npages), True, gpu)
        args = [base, base + 4 * b, base + 8 * b, base + 12 * b, b, table.data_ptr(), stride, base + 16 * b,
                base + 20 * b, ps, qo.data_ptr(), ip.data_ptr(), idx.data_ptr(), last.data_ptr(), loc.data_ptr(), 7]
        L = _lib.lib()
        if fused:
            _lib.check(L.mi_pack_plan(*args, hq, hkv, d, ws.data_ptr(), ws.numel(), _lib.stream_ptr()), "pack_plan")
        else:
            _lib.check(L.mi_pack(*args, _lib.stream_ptr()), "pack")
            _lib.check(L.mi_decode_plan(None, ip.data_ptr(), idx.data_ptr(), last.data_ptr(), b, ps, hq, hkv, d, None,
                                        ws.data_ptr(), ws.numel(), _lib.stream_ptr()), "plan")
        torch.cuda.synchronize()
        hdr, ci, wk, _ = _split_layout(b, hkv, d)
        h = ws[hdr:hdr + 20].cpu().view(torch.int32).tolist()
        cptr = ws[ci:ci + 4 * (b + 1)].cpu().view(torch.int32).tolist()
        work = ws[wk:wk + 16 * h[2]].cpu().view(torch.int32).numpy().reshape(-1, 4)
        outs.append((h, cptr, sorted(map(tuple, work.tolist())), work[:, :2].tolist(),
                     [t.cpu().tolist() for t in (qo, ip, idx, last, loc)], table.cpu().tolist()))
    (h0, c0, w0, o0, p0, t0), (h1, c1, w1, o1, p1, t1) = outs
    assert h0 == h1 and c0 == c1 and w0 == w1 and p0 == p1 and t0 == t1
    # closed form (one new token per request; every page arrives with the step)
    T = np.maximum(np.array(lens) - 1, 0) + 1  # seq_len before the step + the new token
    np_ = np.array(npages)
    want_ip = np.concatenate([[0], np.cumsum(np_)]).tolist()
    want_last = np.where(T % ps == 0, ps, T % ps).tolist()
    want_loc = [[int(pool[want_ip[r + 1] - 1]), want_last[r] - 1] if np_[r] else [-1, -1] for r in range(b)]
    assert p0[0] == list(range(b + 1)) and p0[1] == want_ip and p0[2] == pool[:sum(npages)].tolist()
    assert p0[3] == want_last and p0[4] == want_loc
    nfull = sum(1 for r, k, e, n in w0 if e == (k + 1) * h0[3])
    assert o0[:nfull] and sorted(map(tuple, o0[:nfull])) == sorted(map(tuple, o1[:nfull]))  # full items first in both
