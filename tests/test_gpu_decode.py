"""GPU parity: decode wrapper (plan -> set_kv_cache -> run) against the CPU oracle.

Tolerance: max-abs 2e-2 for bf16/fp16 KV and 6e-2 for fp8-e4m3 KV against
fp32 attention over the same (dequantised) cache — the north-star bar.
The appended cache must equal the oracle's append bit for bit.
"""

import math

import numpy as np
import pytest
import torch

from gpu_helpers import A, P, S, custom_batch, decode_reference, log, max_abs, random_cache, workspace
from mstar_amd.paged_attention import FlashInferDecodeWrapper

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 6e-2


def _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, pool, seed, dtype=torch.bfloat16,
                fp8=False, cpu_index=True, ws_bytes=256 << 20, plan_header=None):
    b = len(last)
    g = torch.Generator().manual_seed(seed + 1000)
    cache_src = random_cache(pool, ps, hkv, d, seed, torch.float32)
    q = torch.randn(b, hq, d, generator=g).to(dtype)
    k_new = torch.randn(b, hkv, d, generator=g).to(dtype)
    v_new = torch.randn(b, hkv, d, generator=g).to(dtype)
    if fp8:
        ks = A.head_scales(cache_src[:, 0].reshape(-1, hkv, d))
        vs = A.head_scales(cache_src[:, 1].reshape(-1, hkv, d))
        cache_cpu = torch.empty(pool, 2, ps, hkv, d, dtype=torch.float8_e4m3fn)
        cache_cpu[:, 0] = A.quantize_e4m3(cache_src[:, 0].reshape(-1, hkv, d), ks).view(pool, ps, hkv, d)
        cache_cpu[:, 1] = A.quantize_e4m3(cache_src[:, 1].reshape(-1, hkv, d), vs).view(pool, ps, hkv, d)
        scales = (ks.to(gpu), vs.to(gpu))
    else:
        ks = vs = None
        cache_cpu = cache_src.to(dtype)
        scales = (None, None)
    cache = cache_cpu.to(gpu)
    # oracle: append then attend
    loc = P.decode_locations(kv_indptr, kv_indices, last)
    A.append(cache_cpu, loc[:, 0], loc[:, 1], k_new, v_new, ks, vs)
    ref = decode_reference(q, cache_cpu, kv_indptr, kv_indices, last, ks, vs)

    wrapper = FlashInferDecodeWrapper(workspace(gpu, ws_bytes), hq, hkv, d, ps, device=gpu)
    t = (lambda x: torch.as_tensor(x)) if cpu_index else (lambda x: torch.as_tensor(x).to(gpu))
    wrapper.plan(t(kv_indptr), t(kv_indices), t(last), dtype=dtype)
    wrapper.set_kv_cache(cache, k_new.to(gpu), v_new.to(gpu), *scales)
    out = wrapper.run(q.to(gpu), cache, *scales)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu().view(torch.uint8), cache_cpu.view(torch.uint8)), "append is not bit-exact"
    assert torch.equal(wrapper.kv_cache_locations.cpu(), torch.as_tensor(loc)), "write locations differ"
    if plan_header is not None:  # [magic, batch, items, item_pages, max_items] of the split-KV plan
        plan_header.extend(wrapper._workspace[:20].view(torch.int32).cpu().tolist())
    return out, ref


@pytest.mark.parametrize("name,nreq", [("c1", None), ("c2", 16), ("c3", 6)])
def test_decode_configs(gpu, name, nreq):
    bt = S.make_batch(name, batch=nreq)
    s = bt.spec
    idx, pool = (bt.kv_indices, s.pool_pages) if s.pool_pages <= 4096 else _compact(bt)
    log(f"decode {name} B={len(bt.kv_len)} pages={bt.total_pages} pool={pool}")
    out, ref = _run_decode(gpu, s.num_qo_heads, s.num_kv_heads, s.head_dim, s.page_size, bt.kv_indptr,
                           idx, bt.last_page_len, pool, s.seed)
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < TOL_BF16


def _compact(bt):
    """Renumber a batch's pages into a pool just large enough (keeps CPU memory small)."""
    uniq = np.unique(bt.kv_indices)
    remap = np.searchsorted(uniq, bt.kv_indices).astype(np.int32)
    rng = np.random.default_rng(0)
    perm = rng.permutation(len(uniq)).astype(np.int32)
    return perm[remap], len(uniq)


@pytest.mark.parametrize("name,nreq", [("c3", 6), ("c5", 6)])
def test_decode_long_context_split(gpu, name, nreq):
    bt = S.make_batch(name, batch=nreq)
    s = bt.spec
    idx, pool = _compact(bt)
    log(f"decode-long {name} B={nreq} max_T={bt.kv_len.max()} pool={pool}")
    out, ref = _run_decode(gpu, s.num_qo_heads, s.num_kv_heads, s.head_dim, s.page_size, bt.kv_indptr, idx,
                           bt.last_page_len, pool, s.seed, fp8=(s.kv_dtype == "fp8"))
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < (TOL_FP8 if s.kv_dtype == "fp8" else TOL_BF16)


@pytest.mark.parametrize(
    "hq,hkv,d,ps",
    [(8, 1, 256, 16), (8, 2, 64, 16), (24, 8, 128, 32), (28, 4, 128, 16), (16, 1, 128, 128), (4, 4, 128, 16),
     (32, 2, 64, 64), (8, 2, 128, 256), (32, 4, 128, 48), (8, 1, 256, 80), (20, 4, 128, 16),
     (48, 4, 128, 32)],
)
def test_decode_shapes(gpu, hq, hkv, d, ps):
    lens = [1, 15, 16, 17, 255, 256, 257, 1000, 3001]
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, 600, seed=hq + d + ps)
    log(f"decode-shape hq={hq} hkv={hkv} d={d} ps={ps}")
    out, ref = _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, 600, seed=7)
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("b,hq,hkv,max_len", [(1100, 8, 2, 64), (1300, 32, 4, 700)])
def test_decode_batch_over_1024(gpu, b, hq, hkv, max_len):
    """More requests than the plan workgroup's 1024 threads: the plan's scans, the
    small-job search and the partition run over several windows of requests (short
    contexts: a small job; longer ones: paired kv-heads and split requests)."""
    rng = np.random.default_rng(b)
    lens = rng.integers(1, max_len + 1, size=b).tolist()
    ps = 16
    pool = int(sum(-(-np.array(lens) // ps))) + 8
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, pool, seed=b)
    log(f"decode B={b} hq={hq} hkv={hkv} max_len={max_len}")
    hdr = []
    out, ref = _run_decode(gpu, hq, hkv, 128, ps, kv_indptr, kv_indices, last, pool, seed=b, plan_header=hdr)
    err = max_abs(out, ref)
    log(f"  items={hdr[2]} item_pages={hdr[3]} max_abs={err:.3e}")
    assert hdr[1] == b and err < TOL_BF16


def test_decode_fp16_and_device_indices(gpu):
    qo, kv_indptr, kv_indices, last = custom_batch([5, 70, 700], 16, 64, seed=3)
    out, ref = _run_decode(gpu, 8, 2, 128, 16, kv_indptr, kv_indices, last, 64, seed=3, dtype=torch.float16,
                           cpu_index=False)
    assert out.dtype == torch.float16
    assert max_abs(out, ref) < TOL_BF16


def test_decode_fp8_shapes(gpu):
    qo, kv_indptr, kv_indices, last = custom_batch([1, 17, 400, 5000], 16, 400, seed=11)
    for hq, hkv, d in [(32, 4, 128), (8, 1, 256), (8, 2, 64)]:
        out, ref = _run_decode(gpu, hq, hkv, d, 16, kv_indptr, kv_indices, last, 400, seed=11, fp8=True)
        err = max_abs(out, ref)
        log(f"decode-fp8 hq={hq} hkv={hkv} d={d} max_abs={err:.3e}")
        assert err < TOL_FP8


def test_decode_is_deterministic(gpu):
    qo, kv_indptr, kv_indices, last = custom_batch([3000, 20, 9000], 16, 1024, seed=5)
    cache = random_cache(1024, 16, 4, 128, 5).to(gpu)
    q = torch.randn(3, 32, 128, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu)
    w = FlashInferDecodeWrapper(workspace(gpu), 32, 4, 128, 16, device=gpu)
    w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last))
    a = w.run(q, cache)
    b = w.run(q, cache)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _ws_for_items(batch, hkv, d, items):
    """Workspace bytes whose split-KV plan holds at most ``items`` items: the
    plan header, item offsets and, per item, its work entry and fp32 partial
    (o, lse) of 16 rows per kv-head, plus alignment slack."""
    fixed = 256 + -(-4 * (batch + 1) // 256) * 256 + 3 * 256
    per_item = 16 + 4 * hkv * 16 + 4 * hkv * 16 * d
    return fixed + per_item * items


@pytest.mark.parametrize(
    "hq,hkv,d,ps,fp8",
    [(32, 4, 128, 16, False), (32, 4, 128, 32, False), (32, 4, 128, 16, True), (32, 4, 128, 32, True),
     (8, 1, 256, 16, False), (24, 8, 64, 64, False)],
)
def test_decode_long_items_walk_several_page_windows(gpu, hq, hkv, d, ps, fp8):
    """A workspace with room for batch + 2 items makes the plan cut long items
    (over 256 pages, more than 64 pages per wavefront): each wavefront reloads
    its window of page ids several times, at page sizes where a wavefront's
    first token falls mid-page, and the longest request is still split in two
    (partials + merge)."""
    lens = [40000, 3000, 17]
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, 3000, seed=ps + d)
    hdr = []
    out, ref = _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, 3000, seed=ps + d + 1, fp8=fp8,
                           ws_bytes=_ws_for_items(len(lens), hkv, d, len(lens) + 2), plan_header=hdr)
    err = max_abs(out, ref)
    log(f"decode long items hq={hq} hkv={hkv} d={d} ps={ps} fp8={fp8}: items={hdr[2]} item_pages={hdr[3]} "
        f"max_abs={err:.3e}")
    assert hdr[3] > 256 and hdr[2] == len(lens) + 1
    assert err < (TOL_FP8 if fp8 else TOL_BF16)


# Decode batches of at least 128 requests at head_dim 128 with at most 8 query
# heads per kv-head read two adjacent kv-heads as one 256-element row (the
# query rows of each head in their half, zeros in the other); smaller
# batches, fp8 and fp32 caches and pools whose heads are not adjacent run the
# per-head kernels on the same plan.
PAIR_B = 136
F32 = torch.float32


def _pair_batch(ps, seed, long_lens=(6000, 9001)):
    """PAIR_B requests: edge lengths, short contexts and long ones the plan splits."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 320, size=PAIR_B)
    lens[: 4 + len(long_lens)] = [1, 15, 16, 17, *long_lens]
    pool = int(((lens + ps - 1) // ps).sum()) + 8
    return (*custom_batch(lens, ps, pool, seed), pool)


@pytest.mark.parametrize(
    "hq,hkv,ps,dtype,fp8",
    [(32, 4, 16, torch.bfloat16, False), (24, 8, 32, torch.bfloat16, False), (8, 8, 16, torch.float16, False),
     (28, 4, 48, torch.bfloat16, False), (16, 2, 16, torch.bfloat16, False), (32, 4, 16, torch.bfloat16, True),
     (32, 4, 16, F32, False)],
)
def test_decode_paired_heads(gpu, hq, hkv, ps, dtype, fp8):
    qo, kv_indptr, kv_indices, last, pool = _pair_batch(ps, seed=hq + ps)
    out, ref = _run_decode(gpu, hq, hkv, 128, ps, kv_indptr, kv_indices, last, pool, seed=hq, dtype=dtype, fp8=fp8)
    err = max_abs(out, ref)
    log(f"decode paired heads hq={hq} hkv={hkv} ps={ps} {dtype} fp8={fp8}: max_abs={err:.3e}")
    assert err < (TOL_FP8 if fp8 else 2e-5 if dtype == F32 else TOL_BF16)


@pytest.mark.parametrize("ps", [16, 32])
def test_decode_paired_heads_long_items(gpu, ps):
    """Paired heads with a workspace for batch + 2 items: items of over 256
    pages, each wavefront walking several 64-page windows, and the longest
    request split in two (partials + merge of 256-element pair rows)."""
    qo, kv_indptr, kv_indices, last, pool = _pair_batch(ps, seed=ps, long_lens=(40000, 6000))
    hdr = []
    out, ref = _run_decode(gpu, 32, 4, 128, ps, kv_indptr, kv_indices, last, pool, seed=ps + 1,
                           ws_bytes=_ws_for_items(PAIR_B, 4, 128, PAIR_B + 2), plan_header=hdr)
    err = max_abs(out, ref)
    log(f"decode paired long items ps={ps}: items={hdr[2]} item_pages={hdr[3]} max_abs={err:.3e}")
    assert hdr[3] > 256 and hdr[2] == PAIR_B + 1
    assert err < TOL_BF16


def test_decode_paired_plan_with_padded_heads(gpu):
    """A pool view whose kv-heads are 160 elements apart (not adjacent) gets
    the per-head kernel on the paired plan; the padding stays untouched."""
    hq, hkv, d, ps = 32, 4, 128, 16
    qo, kv_indptr, kv_indices, last, pool = _pair_batch(ps, seed=21)
    b = len(last)
    g = torch.Generator().manual_seed(22)
    cache_cpu = random_cache(pool, ps, hkv, d, 23)
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16)
    k_new = torch.randn(b, hkv, d, generator=g).to(torch.bfloat16)
    v_new = torch.randn(b, hkv, d, generator=g).to(torch.bfloat16)
    padded = torch.zeros(pool, 2, ps, hkv, 160, dtype=torch.bfloat16, device=gpu)
    padded[..., :d].copy_(cache_cpu.to(gpu))
    view = padded[..., :d]
    loc = P.decode_locations(kv_indptr, kv_indices, last)
    A.append(cache_cpu, loc[:, 0], loc[:, 1], k_new, v_new, None, None)
    ref = decode_reference(q, cache_cpu, kv_indptr, kv_indices, last)
    w = FlashInferDecodeWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
    w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last))
    w.set_kv_cache(view, k_new.to(gpu), v_new.to(gpu))
    out = w.run(q.to(gpu), view)
    torch.cuda.synchronize()
    assert torch.equal(view.cpu().view(torch.uint8), cache_cpu.view(torch.uint8)), "append is not bit-exact"
    assert not padded[..., d:].any().item(), "padding was written"
    err = max_abs(out, ref)
    log(f"decode paired plan, padded heads: max_abs={err:.3e}")
    assert err < TOL_BF16


def _index_variants(arrays):
    """The same index arrays as the plan may receive them: int32 contiguous
    (the reference's), int64, int32 strided views, and device tensors."""
    def strided(a):
        wide = np.repeat(np.asarray(a, dtype=np.int32), 2)  # every element twice
        return torch.from_numpy(wide)[::2]
    return {
        "int32": [torch.as_tensor(np.asarray(a, dtype=np.int32)) for a in arrays],
        "int64": [torch.as_tensor(np.asarray(a, dtype=np.int64)) for a in arrays],
        "strided": [strided(a) for a in arrays],
        "device": None,  # filled per device by the caller
    }


def test_decode_plan_index_inputs(gpu):
    """plan() over int64, strided and device index tensors gives bit-identical
    outputs and write locations to int32 contiguous CPU tensors (the staging
    copy into pinned memory and the device conversion paths)."""
    hq, hkv, d, ps = 32, 4, 128, 16
    lens = [1, 17, 300, 1000, 2500, 64]
    _, kv_indptr, kv_indices, last = custom_batch(lens, ps, 400, seed=3)
    g = torch.Generator().manual_seed(11)
    cache0 = random_cache(400, ps, hkv, d, 3).to(gpu)
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.bfloat16).to(gpu)
    k_new = torch.randn(len(lens), hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    v_new = torch.randn(len(lens), hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    variants = _index_variants([kv_indptr, kv_indices, last])
    variants["device"] = [t.to(gpu) for t in variants["int32"]]
    results = {}
    for name, idx in variants.items():
        assert name != "strided" or not idx[1].is_contiguous()
        cache = cache0.clone()
        w = FlashInferDecodeWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
        w.plan(*idx, dtype=torch.bfloat16)
        w.set_kv_cache(cache, k_new, v_new)
        out = w.run(q, cache)
        torch.cuda.synchronize()
        results[name] = (out.cpu(), w.kv_cache_locations.cpu(), cache.cpu())
        log(f"decode plan index inputs: {name}")
    base = results["int32"]
    for name, (out, loc, cache) in results.items():
        assert torch.equal(out.view(torch.int16), base[0].view(torch.int16)), name
        assert torch.equal(loc, base[1]), name
        assert torch.equal(cache.view(torch.int16), base[2].view(torch.int16)), name
