"""KV page transfer on the GPU against the CPU oracle (bit-exact bytes).

* ``mi_kv_copy_tokens`` between two device pools: random page-level records
  with partial token ranges and layer ranges, bf16 / fp16 / fp8 pools;
  records the kernel must skip (bad page ids or ranges) leave the pool
  untouched;
* wire format: pack equals the oracle's bytes, unpack restores exactly the
  covered rows, a layer range is a contiguous block, whole-page records, a
  pinned-host wire buffer;
* CPU offload / reload through ``PagedAllocationManager`` + ``CPUPagePool``:
  page bookkeeping equal to the oracle's, host pool contents, round trip;
* remote reads between a producer and a consumer manager
  (``start_async_retrieve`` / ``read_batched_async``): the consumer pool
  equals the oracle's after the read, and decode attention over the
  consumer's pages is bit-identical to attention over the producer's;
* a 32768-page copy at the north-star page shape (property check).
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import log
from mstar_amd import _lib
from mstar_amd import kv_transfer as KT
from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager
from oracle import transfer as T

pytestmark = pytest.mark.gpu

_BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float8_e4m3fn: torch.uint8}


def _pool(shape, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    bits = _BITS[dtype]
    x = torch.randint(-128 if bits == torch.uint8 else -(1 << 15), 128 if bits == torch.uint8 else 1 << 15,
                      shape, generator=g, dtype=torch.int32)
    x = x.to(torch.uint8) if bits == torch.uint8 else x.to(torch.int16)
    return x.view(dtype).to(device)


def _np(kv: torch.Tensor) -> np.ndarray:
    """[L, P, 2, ps, H*D] integer view of a pool (host copy)."""
    L, P, _, ps, H, D = kv.shape
    return kv.cpu().view(_BITS[kv.dtype]).reshape(L, P, 2, ps, H * D).numpy()


def _records(rng, n, ps, dst_pages, src_pages, partial=True):
    dst = rng.permutation(dst_pages)[:n]
    src = rng.permutation(src_pages)[:n]
    if not partial:
        return dst, src, None, None
    ts = rng.integers(0, ps, size=n)
    te = np.minimum(ps, ts + rng.integers(1, ps + 1, size=n))
    return dst, src, ts, te


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
def test_copy_tokens_matches_oracle(gpu, dtype):
    L, P, ps, H, D = 3, 64, 16, 2, 64
    src = _pool((L, P, 2, ps, H, D), dtype, 1, gpu)
    dst = _pool((L, P + 9, 2, ps, H, D), dtype, 2, gpu)
    rng = np.random.default_rng(5)
    for lb, le, partial in ((0, L, True), (1, 2, True), (0, L, False)):
        d0 = dst.clone()
        dp, sp, ts, te = _records(rng, 40, ps, P + 9, P, partial)
        KT.copy_tokens(src, d0, dp, sp, ts, te, lb, le)
        torch.cuda.synchronize()
        tsl = [0] * len(dp) if ts is None else ts
        tel = [ps] * len(dp) if te is None else te
        recs = list(zip(dp.tolist(), sp.tolist(), list(map(int, tsl)), list(map(int, tel))))
        exp = T.copy_tokens(_np(src), _np(dst), recs, lb, le)
        np.testing.assert_array_equal(_np(d0), exp)
        log(f"copy_tokens {dtype} layers [{lb},{le}) partial={partial}: {len(recs)} records ok")


def test_kernel_skips_malformed_records(gpu):
    """Records with page ids or token ranges out of bounds are skipped by the kernel."""
    L, P, ps, H, D = 2, 8, 16, 1, 64
    src = _pool((L, P, 2, ps, H, D), torch.bfloat16, 3, gpu)
    dst = _pool((L, P, 2, ps, H, D), torch.bfloat16, 4, gpu)
    before = dst.clone()
    recs = np.array([[1, 2, 0, 16], [P, 0, 0, 16], [3, -1, 0, 16], [4, 1, 5, 5], [5, 1, 3, 17], [6, 1, -2, 4]],
                    dtype=np.int32)
    dev = torch.from_numpy(np.ascontiguousarray(recs.T)).to(gpu)
    n = recs.shape[0]
    base = dev.data_ptr()
    sd, dd = KT.pool_desc(src), KT.pool_desc(dst)
    rc = _lib.lib().mi_kv_copy_tokens(ctypes.byref(sd), ctypes.byref(dd), base + 4 * n, base, base + 8 * n,
                                      base + 12 * n, n, 0, L, _lib.stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    exp = before.clone()
    exp[:, 1] = src[:, 2]
    assert torch.equal(dst.view(torch.int16), exp.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_wire_pack_unpack_matches_oracle(gpu, dtype):
    L, P, ps, H, D = 4, 50, 16, 2, 128
    pool = _pool((L, P, 2, ps, H, D), dtype, 7, gpu)
    ref = _np(pool)
    rng = np.random.default_rng(11)
    pages, _, ts, te = _records(rng, 23, ps, P, P)
    wire = KT.pack_wire(pool, pages, ts, te)
    exp = T.wire_pack(ref, pages, ts, te)
    np.testing.assert_array_equal(wire.cpu().numpy(), exp)
    # a layer range is one contiguous block of the full buffer
    rows = int((te - ts).sum())
    blk = 2 * rows * H * D * pool.element_size()
    sub = KT.pack_wire(pool, pages, ts, te, 1, 3)
    np.testing.assert_array_equal(sub.cpu().numpy(), exp[blk:3 * blk])
    # unpack into a fresh pool restores exactly the covered rows
    back = torch.zeros_like(pool)
    KT.unpack_wire(wire, back, pages, ts, te)
    np.testing.assert_array_equal(_np(back), T.wire_unpack(exp, np.zeros_like(ref), pages, ts, te))
    # whole pages, packed straight into pinned host memory, unpacked from there
    host = torch.empty(KT.wire_nbytes(pool, len(pages) * ps), dtype=torch.uint8, pin_memory=True)
    KT.pack_wire(pool, pages, out=host)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host.numpy(), T.wire_pack(ref, pages, [0] * len(pages), [ps] * len(pages)))
    back2 = torch.zeros_like(pool)
    KT.unpack_wire(host, back2, pages)
    torch.cuda.synchronize()
    exp2 = np.zeros_like(ref)
    exp2[:, pages] = ref[:, pages]
    np.testing.assert_array_equal(_np(back2), exp2)
    log(f"wire {dtype}: {len(pages)} records, {wire.numel()} bytes ok")


def _manager(pool_pages, L, ps, H, D, gpu, seed, labels=("main",), rids=()):
    cfg = KVCacheConfig(num_layers=L, num_kv_heads=H, head_dim=D, max_seq_len=8192, max_num_pages=pool_pages,
                        page_size=ps, num_qo_heads=4 * H)
    kv = _pool((L, pool_pages, 2, ps, H, D), torch.bfloat16, seed, gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    for r in rids:
        mgr.add_request(r, list(labels))
    return cfg, kv, mgr


def test_cpu_offload_reload_round_trip(gpu):
    L, ps, H, D, POOL, CPU = 3, 16, 2, 64, 96, 15
    cfg, kv, mgr = _manager(POOL, L, ps, H, D, gpu, 21, ("main", "cfg"), ["a", "b", "c"])
    lens = {("a", "main"): 70, ("a", "cfg"): 16, ("b", "main"): 3, ("c", "main"): 129}
    for (r, label), n in lens.items():  # GPU pages a/main 0-4, a/cfg 5, b 6, c 7-15
        mgr.alloc(r, label, n)
        st = mgr.get_state(r, label)
        st.seq_len, st.position_id_start = n, n + 7
    pages = {k: list(mgr.get_state(*k).page_indices) for k in lens}
    original = {k: kv[:, pages[k]].cpu() for k in lens}
    cpu_pool = KT.CPUPagePool(cfg, CPU, torch.bfloat16)
    ocpu = T.CpuPool(CPU, (L, 2, ps, H * D), np.int16)
    ogpu = _np(kv)

    assert mgr.offload_request("a", cpu_pool) == 6
    assert mgr.offload_request("c", cpu_pool) == 9
    assert mgr.offload_request("b", cpu_pool) == 1  # no CPU page left: freed but not kept (reference behaviour)
    for k in (("a", "main"), ("a", "cfg"), ("c", "main"), ("b", "main")):
        ocpu.offload(k[0], k[1], ogpu, pages[k], lens[k], lens[k] + 7)
    torch.cuda.synchronize()
    assert set(cpu_pool.offloaded) == set(ocpu.offloaded) == {"a", "c"}
    for r, labels in ocpu.offloaded.items():
        for label, (cpages, n, pos) in labels.items():
            got = cpu_pool.offloaded[r][label]
            assert (got.cpu_page_indices, got.seq_len, got.position_id_start) == (cpages, n, pos)
    np.testing.assert_array_equal(cpu_pool.cpu_kv_cache.view(torch.int16).reshape(L, CPU, 2, ps, H * D).numpy(),
                                  ocpu.data)
    for k in lens:
        assert mgr.get_state(*k).page_indices == [] and mgr.get_state(*k).seq_len == 0
    assert list(mgr.page_allocator.free_pages) == list(range(16, POOL)) + list(range(6)) + list(range(7, 16)) + [6]
    # freed GPU pages are taken by another request and overwritten before the reloads
    mgr.add_request("z", ["main"])
    mgr.alloc("z", "main", 81 * ps)
    kv[:, mgr.get_state("z", "main").page_indices] = 0
    mgr.add_request("y", ["main"])
    mgr.alloc("y", "main", 1)  # 14 GPU pages left: c (9) fits, then a (5 + 1) does not
    mgr.reload_request("c", cpu_pool)
    free_before = list(mgr.page_allocator.free_pages)
    with pytest.raises(RuntimeError):
        mgr.reload_request("a", cpu_pool)  # all-or-nothing: no label of "a" changes
    assert list(mgr.page_allocator.free_pages) == free_before
    assert cpu_pool.is_offloaded("a") and set(cpu_pool.offloaded["a"]) == {"main", "cfg"}
    assert mgr.get_state("a", "main").page_indices == [] and mgr.get_state("a", "cfg").page_indices == []
    mgr.remove_request("y")
    mgr.reload_request("a", cpu_pool)
    torch.cuda.synchronize()
    assert mgr.num_free_pages == 0
    for k in (("a", "main"), ("a", "cfg"), ("c", "main")):
        st = mgr.get_state(*k)
        assert (st.seq_len, st.position_id_start) == (lens[k], lens[k] + 7)
        assert torch.equal(kv[:, st.page_indices].cpu().view(torch.int16), original[k].view(torch.int16)), k
    assert not cpu_pool.is_offloaded("a") and cpu_pool.num_free_pages == CPU
    log("offload/reload round trip ok")


def test_remote_read_between_managers(gpu):
    from mstar_amd.paged_attention import FlashInferDecodeWrapper

    L, ps, H, D = 2, 16, 2, 128
    rids = ["r0", "r1", "r2", "r3"]
    _, kv_p, prod = _manager(200, L, ps, H, D, gpu, 31, rids=rids)
    _, kv_c, cons = _manager(260, L, ps, H, D, gpu, 32, rids=rids)
    cons.add_request("pad", ["main"])
    cons.alloc("pad", "main", 7 * ps)  # consumer page ids differ from the producer's
    want = [1, 200, 16, 333]
    have = [0, 37, 16, 32]
    for r, n in zip(rids, want):
        prod.alloc(r, "main", n)
        st = prod.get_state(r, "main")
        st.seq_len, st.position_id_start = n, 1000 + n
    # the consumer already holds a prefix (an earlier read)
    info = prod.get_per_label_seq_info("r0")["main"].latest_kv_transfer_info
    expect = _np(kv_c)
    src_np = _np(kv_p)
    for r, h in zip(rids, have):
        if h == 0:
            continue
        pinfo = prod.get_per_label_seq_info(r)["main"]
        cons.sync_retrieve(r, "main", KT.SequenceInfo(h, 1000 + h, info, pinfo.page_indices))
        recs = T.read_records(0, h, ps, cons.get_state(r, "main").page_indices, pinfo.page_indices)
        T.copy_tokens(src_np, expect, recs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(kv_c), expect)
    # then reads the rest asynchronously
    for r, h in zip(rids, have):
        pinfo = prod.get_per_label_seq_info(r)["main"]
        cons.start_async_retrieve(r, "main", pinfo)
        recs = T.read_records(h, pinfo.seq_len, ps, cons.get_state(r, "main").page_indices, pinfo.page_indices)
        T.copy_tokens(src_np, expect, recs)
    for r in rids:
        cons.wait_for_retrieves(r, "main")
        assert cons.check_retrieve_ready(r, "main")
        st = cons.get_state(r, "main")
        assert st.seq_len == prod.get_state(r, "main").seq_len and st.position_id_start == 1000 + st.seq_len
    np.testing.assert_array_equal(_np(kv_c), expect)

    # decode over the consumer's pages is bit-identical to decode over the producer's
    q = torch.randn(len(rids), 4 * H, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu)
    outs = []
    for mgr, kv in ((prod, kv_p), (cons, kv_c)):
        lists = [mgr.get_state(r, "main").page_indices for r in rids]
        indptr = torch.tensor(np.concatenate([[0], np.cumsum([len(x) for x in lists])]), dtype=torch.int32)
        idx = torch.tensor([p for x in lists for p in x], dtype=torch.int32)
        last = torch.tensor([(n % ps) or ps for n in want], dtype=torch.int32)
        w = FlashInferDecodeWrapper(torch.empty(32 << 20, dtype=torch.uint8, device=gpu), 4 * H, H, D, ps,
                                    device=gpu)
        w.plan(indptr, idx, last)
        outs.append(torch.stack([w.run(q, kv[layer]) for layer in range(L)]).cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))

    # the reference's per-(layer, page) list, one layer only for some records
    before = _np(kv_c)
    infos = [KT.KVReadInfo(0, 250, 3, 0, 16), KT.KVReadInfo(1, 250, 3, 0, 16), KT.KVReadInfo(1, 251, 4, 2, 9)]
    fut = cons.kv_transfer_engine.read_batched_async(info, infos)
    fut.result()
    T.copy_tokens(src_np, before, [(250, 3, 0, 16)])
    T.copy_tokens(src_np, before, [(251, 4, 2, 9)], 1, 2)
    np.testing.assert_array_equal(_np(kv_c), before)
    log("remote reads ok")


def test_large_copy_property(gpu):
    """32768 whole pages of the north-star shape (ps 16, 4 kv-heads, D 128, bf16)."""
    P, ps, H, D = 40000, 16, 4, 128
    src = torch.empty(1, P, 2, ps, H, D, dtype=torch.bfloat16, device=gpu)
    src.view(torch.int16).random_(-(1 << 15), 1 << 15)
    dst = torch.zeros_like(src)
    g = torch.Generator().manual_seed(9)
    sp = torch.randperm(P, generator=g)[:32768]
    dp = torch.randperm(P, generator=g)[:32768]
    KT.copy_tokens(src, dst, dp.numpy(), sp.numpy())
    torch.cuda.synchronize()
    assert torch.equal(dst[0, dp.to(gpu)].view(torch.int16), src[0, sp.to(gpu)].view(torch.int16))
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[dp] = False
    assert int(dst[0, untouched.to(gpu)].view(torch.int16).abs().sum()) == 0
