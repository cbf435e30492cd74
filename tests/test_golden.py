"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture exactly.
GPU: the product path reproduces them — packing metadata, token map, write
locations and fp8 codes bit for bit; attention within 2e-2 (max-abs, the
fixture holds the fp32 result rounded to fp16); RoPE within the bound of
``gpu_helpers.rope_bound``.
"""

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import rope as R

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.copy()).view(torch.bfloat16)


# ------------------------------------------------------------------ CPU
def test_oracle_reproduces_packing():
    ref = _load("packing.npz")
    got = _maker().packing()
    for key in ref.files:
        np.testing.assert_array_equal(got[key], ref[key], err_msg=key)


@pytest.mark.parametrize("name", ["decode_small.npz", "prefill_small.npz"])
def test_oracle_reproduces_attention(name):
    d = _load(name)
    out = A.paged_attention(_bf16(d["q"]), _bf16(d["cache"]), d["qo_indptr"], d["kv_indptr"], d["kv_indices"],
                            d["last_page_len"], causal=bool(d["causal"]))
    np.testing.assert_array_equal(out.numpy().astype(np.float16), d["out"])


def test_oracle_reproduces_rope_and_fp8():
    r = _load("rope_small.npz")
    q, k, pos = _bf16(r["q"]), _bf16(r["k"]), r["pos"]
    np.testing.assert_array_equal(R.rope(q, pos, rope_theta=1e4).numpy(), r["q_plain"])
    l31 = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)
    np.testing.assert_array_equal(R.rope(k, pos, rope_scale=8.0, rope_theta=5e5, llama31=l31).numpy(), r["k_l31"])
    f = _load("fp8_codes.npz")
    codes = A.quantize_e4m3(torch.from_numpy(f["x"]), torch.from_numpy(f["scale"])).view(torch.uint8).numpy()
    np.testing.assert_array_equal(codes, f["codes"])


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_gpu_packing_matches_golden(gpu):
    from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
    from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager

    g = _load("packing.npz")
    ps, pool, prompt = int(g["page_size"]), int(g["pool"]), g["prompt"].tolist()
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=1, head_dim=64, max_seq_len=1024, max_num_pages=pool,
                        page_size=ps, num_qo_heads=1)
    kv = torch.zeros(1, pool, 2, ps, 1, 64, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    bufs = WorkspaceBufferManager(64 << 20, gpu)
    rids = [f"r{i}" for i in range(len(prompt))]
    for r in rids:
        mgr.add_request(r, ["main"])
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, bufs, cfg, gpu)
    cm.plan_attention(prompt)
    qo, kv_indptr, kv_indices, last, _ = cm._last_pack
    w = cm._plan_states["main"].wrapper
    assert qo.cpu().numpy().tolist() == g["qo1"].tolist()
    assert kv_indptr.cpu().numpy().tolist() == g["kv1"].tolist()
    assert kv_indices.cpu().numpy().tolist() == g["idx1"].tolist()
    assert last.cpu().numpy().tolist() == g["last1"].tolist()
    n = int(g["qo1"][-1])
    assert w.token_to_page[:n].cpu().numpy().tolist() == g["t2p1"][:n].tolist()
    assert w.token_to_cache[:n].cpu().numpy().tolist() == g["t2c1"][:n].tolist()
    cm.advance_seq_lens()
    # request 4 finishes and a fresh request takes its place in the batch
    mgr.remove_request("r4")
    mgr.add_request("r4b", ["main"])
    rids2 = rids[:4] + ["r4b"] + rids[5:]
    cm2 = BatchedCacheManager(rids2, {r: "main" for r in rids2}, kv, mgr, bufs, cfg, gpu)
    cm2.plan_attention([1] * len(rids2))
    _, kv_indptr, kv_indices, last, loc = cm2._last_pack
    assert kv_indptr.cpu().numpy().tolist() == g["kv2"].tolist()
    assert kv_indices.cpu().numpy().tolist() == g["idx2"].tolist()
    assert last.cpu().numpy().tolist() == g["last2"].tolist()
    assert loc.cpu().numpy().tolist() == g["loc2"].tolist()
    assert list(mgr.page_allocator.free_pages) == g["free_after"].tolist()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["decode_small.npz", "prefill_small.npz"])
def test_gpu_attention_matches_golden(gpu, name):
    from mstar_amd.paged_attention import FlashInferDecodeWrapper, FlashInferPrefillWrapper

    d = _load(name)
    hkv = int(d["num_kv_heads"])
    q = _bf16(d["q"]).to(gpu)
    cache = _bf16(d["cache"]).to(gpu)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=gpu)
    idx = [torch.from_numpy(d[k].copy()) for k in ("qo_indptr", "kv_indptr", "kv_indices", "last_page_len")]
    if name.startswith("decode"):
        w = FlashInferDecodeWrapper(ws, q.shape[1], hkv, q.shape[2], cache.shape[2], device=gpu)
        w.plan(idx[1], idx[2], idx[3])
    else:
        w = FlashInferPrefillWrapper(ws, q.shape[1], hkv, q.shape[2], cache.shape[2], device=gpu)
        w.plan(idx[0], idx[1], idx[2], idx[3], causal=bool(d["causal"]))
    out = w.run(q, cache)
    err = (out.float().cpu() - torch.from_numpy(d["out"]).float()).abs().max().item()
    assert err <= 2e-2, err


@pytest.mark.gpu
def test_gpu_rope_and_fp8_match_golden(gpu):
    from gpu_helpers import rope_bound
    from mstar_amd import rope as MR
    from mstar_amd.paged_attention import FlashInferDecodeWrapper

    r = _load("rope_small.npz")
    pos = torch.from_numpy(r["pos"])
    l31 = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)
    for key, kw, fn in (("plain", dict(rope_theta=1e4), MR.apply_rope_pos_ids_inplace),
                        ("l31", dict(rope_scale=8.0, rope_theta=5e5, **l31), MR.apply_llama31_rope_pos_ids_inplace)):
        q, k = _bf16(r["q"]), _bf16(r["k"])
        qg, kg = q.to(gpu), k.to(gpu)
        fn(qg, kg, pos.to(gpu), **kw)
        ll = l31 if key == "l31" else None
        sc, th = (8.0, 5e5) if key == "l31" else (1.0, 1e4)
        for x, y, ref in ((q, qg, r[f"q_{key}"]), (k, kg, r[f"k_{key}"])):
            ref_t = torch.from_numpy(ref)
            err = (y.cpu().double() - ref_t.double()).abs()
            assert (err <= rope_bound(x, ref_t, r["pos"], x.shape[2], False, sc, th, ll)).all(), key

    # fp8 codes through the append kernel: token t goes to page t, slot 3
    f = _load("fp8_codes.npz")
    x = torch.from_numpy(f["x"])
    t, hkv, d = x.shape
    scale = torch.from_numpy(f["scale"]).to(gpu)
    cache = torch.zeros(t, 2, 16, hkv, d, dtype=torch.float8_e4m3fn, device=gpu)
    w = FlashInferDecodeWrapper(torch.empty(16 << 20, dtype=torch.uint8, device=gpu), hkv, hkv, d, 16, device=gpu)
    kv_indptr = torch.arange(t + 1, dtype=torch.int32)
    w.plan(kv_indptr, torch.arange(t, dtype=torch.int32), torch.full((t,), 4, dtype=torch.int32))
    w.set_kv_cache(cache, x.to(gpu), (-x).to(gpu), k_scale=scale, v_scale=scale)
    got = cache[:, 0, 3].view(torch.uint8).cpu().numpy()
    np.testing.assert_array_equal(got, f["codes"])
    neg = A.quantize_e4m3(-x, torch.from_numpy(f["scale"])).view(torch.uint8).numpy()
    np.testing.assert_array_equal(cache[:, 1, 3].view(torch.uint8).cpu().numpy(), neg)
