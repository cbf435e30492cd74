"""GPU parity: ragged paged prefill wrapper (plan -> set_kv_cache -> run).

* the reference's own scenario, test/modular/test_pi05_reference_equivalence.py:645-719
  (1 request, page_size 16, 8 q / 1 kv head, head_dim 256, 24-token
  bidirectional prefix then a 4-token suffix; its tolerance 5e-2, ours 2e-2);
* small ragged causal / non-causal batches against the CPU oracle, including
  zero-length and one-token requests mixed with long chunks;
* the full BAGEL-shaped mixed batch (c4) against an fp32 torch reference on
  the GPU (the CPU oracle would take minutes at that size);
* the per-token page map and the append are bit-exact with the oracle.
"""

import math

import numpy as np
import pytest
import torch

from gpu_helpers import A, P, S, custom_batch, log, max_abs, random_cache, workspace
from mstar_amd import _lib
from mstar_amd.paged_attention import FlashInferPrefillWrapper

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_FP8 = 6e-2


def test_reference_scenario_prefix_then_suffix(gpu):
    torch.manual_seed(0)
    hq, hkv, d, ps, max_pages, prefix_len, suffix_len = 8, 1, 256, 16, 32, 24, 4
    dt = torch.bfloat16
    cache = torch.zeros(max_pages, 2, ps, hkv, d, device=gpu, dtype=dt)
    w = FlashInferPrefillWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
    qp = torch.randn(prefix_len, hq, d, device=gpu, dtype=dt)
    kp = torch.randn(prefix_len, hkv, d, device=gpu, dtype=dt)
    vp = torch.randn(prefix_len, hkv, d, device=gpu, dtype=dt)
    n_pref = (prefix_len + ps - 1) // ps
    last = prefix_len - (n_pref - 1) * ps
    w.plan(torch.tensor([0, prefix_len], dtype=torch.int32, device=gpu),
           torch.tensor([0, n_pref], dtype=torch.int32, device=gpu),
           torch.arange(n_pref, dtype=torch.int32, device=gpu),
           torch.tensor([last], dtype=torch.int32, device=gpu), causal=False, dtype=dt)
    w.set_kv_cache(cache, kp, vp)
    out = w.run(qp, cache)
    ref, _ = A.attend(qp.cpu(), kp.cpu(), vp.cpu(), causal=False, sm_scale=d ** -0.5)
    delta = max_abs(out, ref)
    log(f"reference scenario prefill: {delta:.3e}")
    assert delta < TOL

    qs = torch.randn(suffix_len, hq, d, device=gpu, dtype=dt)
    ks = torch.randn(suffix_len, hkv, d, device=gpu, dtype=dt)
    vs = torch.randn(suffix_len, hkv, d, device=gpu, dtype=dt)
    total = prefix_len + suffix_len
    n_after = (total + ps - 1) // ps
    last2 = total - (n_after - 1) * ps
    w.plan(torch.tensor([0, suffix_len], dtype=torch.int32, device=gpu),
           torch.tensor([0, n_after], dtype=torch.int32, device=gpu),
           torch.arange(n_after, dtype=torch.int32, device=gpu),
           torch.tensor([last2], dtype=torch.int32, device=gpu), causal=False, dtype=dt)
    w.set_kv_cache(cache, ks, vs)
    out2 = w.run(qs, cache)
    ref2, _ = A.attend(qs.cpu(), torch.cat([kp, ks]).cpu(), torch.cat([vp, vs]).cpu(), causal=False,
                       sm_scale=d ** -0.5)
    delta2 = max_abs(out2, ref2)
    log(f"reference scenario suffix: {delta2:.3e}")
    assert delta2 < TOL


def _run_prefill(gpu, hq, hkv, d, ps, kv_lens, new_lens, causal, seed, fp8=False, dtype=torch.bfloat16):
    qo, kv_indptr, kv_indices, last = custom_batch(kv_lens, ps, int(sum(-(-np.array(kv_lens) // ps))) + 4, seed,
                                                   new_lens=new_lens)
    pool = int(kv_indices.max()) + 1 if len(kv_indices) else 1
    g = torch.Generator().manual_seed(seed + 7)
    src = random_cache(pool, ps, hkv, d, seed, torch.float32)
    ntok = int(qo[-1])
    q = torch.randn(ntok, hq, d, generator=g).to(dtype)
    k = torch.randn(ntok, hkv, d, generator=g).to(dtype)
    v = torch.randn(ntok, hkv, d, generator=g).to(dtype)
    if fp8:
        ks = A.head_scales(src[:, 0].reshape(-1, hkv, d))
        vs = A.head_scales(src[:, 1].reshape(-1, hkv, d))
        cache_cpu = torch.empty(pool, 2, ps, hkv, d, dtype=torch.float8_e4m3fn)
        cache_cpu[:, 0] = A.quantize_e4m3(src[:, 0].reshape(-1, hkv, d), ks).view(pool, ps, hkv, d)
        cache_cpu[:, 1] = A.quantize_e4m3(src[:, 1].reshape(-1, hkv, d), vs).view(pool, ps, hkv, d)
        scales = (ks.to(gpu), vs.to(gpu))
    else:
        ks = vs = None
        cache_cpu = src.to(dtype)
        scales = (None, None)
    cache = cache_cpu.to(gpu)
    t2p, t2c = P.token_map(qo, kv_indptr, kv_indices, last, ps)
    A.append(cache_cpu, t2p, t2c, k, v, ks, vs)
    ref = A.paged_attention(q, cache_cpu, qo, kv_indptr, kv_indices, last, causal=causal, k_scale=ks, v_scale=vs)
    w = FlashInferPrefillWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
    w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last),
           causal=causal, dtype=dtype)
    w.set_kv_cache(cache, k.to(gpu), v.to(gpu), *scales)
    out = w.run(q.to(gpu), cache, *scales)
    torch.cuda.synchronize()
    assert w.token_to_page.cpu().tolist() == t2p.tolist() and w.token_to_cache.cpu().tolist() == t2c.tolist()
    assert torch.equal(cache.cpu().view(torch.uint8), cache_cpu.view(torch.uint8)), "append is not bit-exact"
    return out, ref


MIX_KV = [40, 1, 300, 17, 700, 33, 5, 260]
MIX_NEW = [40, 1, 120, 0, 300, 2, 5, 3]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv,d,ps", [(28, 4, 128, 16), (8, 8, 128, 16), (16, 2, 64, 32), (8, 1, 256, 16),
                                         (32, 2, 128, 64), (16, 2, 256, 32), (8, 2, 128, 128), (28, 4, 128, 48),
                                         (8, 1, 256, 80), (20, 4, 128, 16), (48, 4, 64, 32)])
def test_prefill_ragged_mix(gpu, causal, hq, hkv, d, ps):
    log(f"prefill mix causal={causal} hq={hq} hkv={hkv} d={d} ps={ps}")
    out, ref = _run_prefill(gpu, hq, hkv, d, ps, MIX_KV, MIX_NEW, causal, seed=hq + d)
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < TOL


def _paired_mix(seed, b=140):
    """A ragged batch of >= 128 requests at head_dim 128 (its short part reads
    kv-head pairs): single-token requests (paired decode), two- and
    three-token requests whose 14-21 rows no longer fit a paired column block
    (MFMA tiles), empty requests and two long chunks."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(2, 600, b)
    new = np.ones(b, dtype=np.int64)
    new[5:9] = [2, 3, 2, 0]
    kv[10:12] = [900, 700]
    new[10:12] = [300, 640]
    kv[20] = 5000  # a long single-token request: split items and a merge
    return kv.tolist(), new.tolist()


@pytest.mark.parametrize("dtype,fp8", [(torch.bfloat16, False), (torch.float16, False), (torch.bfloat16, True),
                                       (torch.float32, False)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_paired_short_queries(gpu, dtype, fp8, causal):
    """Short-query requests of a large ragged batch run on the paired kernel
    (bf16/fp16; fp8 and fp32 run the per-head kernels on the paired plan)."""
    kv, new = _paired_mix(7)
    assert _lib.lib().mi_prefill_short_rows(len(kv), 28, 4, 128) == 8
    out, ref = _run_prefill(gpu, 28, 4, 128, 16, kv, new, causal, seed=23, fp8=fp8, dtype=dtype)
    err = max_abs(out, ref)
    log(f"paired short queries {dtype} fp8={fp8} causal={causal}: max_abs={err:.3e}")
    assert err < (TOL_FP8 if fp8 else (2e-5 if dtype == torch.float32 else TOL))


def test_prefill_paired_short_queries_only(gpu):
    """Every request single-token: run() launches only the short half, paired."""
    rng = np.random.default_rng(3)
    kv = rng.integers(1, 900, 130).tolist()
    out, ref = _run_prefill(gpu, 32, 4, 128, 16, kv, [1] * 130, True, seed=29)
    assert max_abs(out, ref) < TOL


@pytest.mark.parametrize("kv_lens,new_lens,launches", [([40, 300, 17, 260], [1, 2, 0, 1], "short"),
                                                      ([40, 300, 700], [40, 3, 300], "tiles")])
def test_prefill_batch_needing_one_launch(gpu, kv_lens, new_lens, launches):
    """Batches whose requests all go to one of run()'s two kernels (the other
    launch is skipped when the host knows it has no work)."""
    out, ref = _run_prefill(gpu, 28, 4, 128, 16, kv_lens, new_lens, True, seed=11)
    err = max_abs(out, ref)
    log(f"prefill {launches}-only batch max_abs={err:.3e}")
    assert err < TOL


@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (8, 1, 256)])
def test_prefill_fp16_and_fp8(gpu, hq, hkv, d):
    log(f"prefill fp16 / fp8 hq={hq} hkv={hkv} d={d}")
    out, ref = _run_prefill(gpu, hq, hkv, d, 16, MIX_KV, MIX_NEW, True, seed=3, dtype=torch.float16)
    assert out.dtype == torch.float16 and max_abs(out, ref) < TOL
    out, ref = _run_prefill(gpu, hq, hkv, d, 16, MIX_KV, MIX_NEW, True, seed=4, fp8=True)
    err = max_abs(out, ref)
    log(f"prefill fp8 max_abs={err:.3e}")
    assert err < TOL_FP8


def _torch_ref_gpu(q, cache, qo, kv_indptr, kv_indices, last, causal, hq, hkv):
    """fp32 attention per request on the GPU (gathered pages, repeat_interleave GQA)."""
    ps = cache.shape[2]
    out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    for r in range(len(last)):
        q0, q1 = int(qo[r]), int(qo[r + 1])
        if q1 == q0:
            continue
        pages = torch.as_tensor(kv_indices[kv_indptr[r]:kv_indptr[r + 1]].astype(np.int64), device=q.device)
        kv_len = (len(pages) - 1) * ps + int(last[r])
        k = cache[pages, 0].reshape(-1, hkv, cache.shape[-1])[:kv_len].float().repeat_interleave(hq // hkv, 1)
        v = cache[pages, 1].reshape(-1, hkv, cache.shape[-1])[:kv_len].float().repeat_interleave(hq // hkv, 1)
        qr = q[q0:q1].float()
        kt = k.permute(1, 2, 0).contiguous()  # [H, D, kv]
        s = torch.matmul(qr.transpose(0, 1).contiguous(), kt) / math.sqrt(q.shape[-1])  # [H, qo, kv]
        if causal:
            qo_len = q1 - q0
            j = torch.arange(qo_len, device=q.device).view(-1, 1)
            i = torch.arange(kv_len, device=q.device).view(1, -1)
            s = s.masked_fill(i > kv_len - qo_len + j, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[q0:q1] = torch.matmul(p, v.transpose(0, 1).contiguous()).transpose(0, 1)
    return out


def test_prefill_c4_bagel_mixed_batch(gpu):
    bt = S.make_batch("c4")
    s = bt.spec
    log(f"c4: B={len(bt.kv_len)} q_tokens={bt.total_q_tokens} pages={bt.total_pages}")
    cache = torch.empty(s.pool_pages, 2, s.page_size, s.num_kv_heads, s.head_dim, dtype=torch.bfloat16, device=gpu)
    cache.normal_(generator=torch.Generator(device=gpu).manual_seed(s.seed))
    g = torch.Generator().manual_seed(s.seed + 1)
    ntok = bt.total_q_tokens
    q = torch.randn(ntok, s.num_qo_heads, s.head_dim, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(ntok, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(ntok, s.num_kv_heads, s.head_dim, generator=g).to(torch.bfloat16).to(gpu)
    w = FlashInferPrefillWrapper(workspace(gpu, 512 << 20), s.num_qo_heads, s.num_kv_heads, s.head_dim,
                                 s.page_size, device=gpu)
    w.plan(torch.as_tensor(bt.qo_indptr), torch.as_tensor(bt.kv_indptr), torch.as_tensor(bt.kv_indices),
           torch.as_tensor(bt.last_page_len), causal=True)
    w.set_kv_cache(cache, k, v)
    out = w.run(q, cache)
    ref = _torch_ref_gpu(q, cache, bt.qo_indptr, bt.kv_indptr, bt.kv_indices, bt.last_page_len, True,
                         s.num_qo_heads, s.num_kv_heads)
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    log(f"c4 max_abs={err:.3e}")
    assert err < TOL
    # appended tokens are where the oracle's page map puts them
    t2p, t2c = P.token_map(bt.qo_indptr, bt.kv_indptr, bt.kv_indices, bt.last_page_len, s.page_size)
    got = cache[torch.as_tensor(t2p, device=gpu), 0, torch.as_tensor(t2c, device=gpu)]
    assert torch.equal(got, k)


def test_prefill_graph_mode_tail_and_padding(gpu):
    hq, hkv, d, ps = 8, 2, 128, 16
    max_tok = 64
    w = FlashInferPrefillWrapper(workspace(gpu), hq, hkv, d, ps, batch_size=2, max_total_tokens=max_tok,
                                 max_num_pages=32, device=gpu, use_cuda_graph=True)
    qo, kv_indptr, kv_indices, last = custom_batch([30, 50], ps, 32, seed=9, new_lens=[10, 20])
    w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last))
    t2p, t2c = P.token_map(qo, kv_indptr, kv_indices, last, ps, tail_len=max_tok)
    torch.cuda.synchronize()
    assert w.token_to_page.cpu().tolist() == t2p.tolist() and w.token_to_cache.cpu().tolist() == t2c.tolist()
    # padding tokens beyond qo_indptr[-1] are not written (the reference would write page 0 slot 0)
    cache = torch.zeros(32, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    k = torch.ones(max_tok, hkv, d, dtype=torch.bfloat16, device=gpu)
    w._total_tokens = max_tok  # as a graph captured with a larger batch would replay
    w.set_kv_cache(cache, k, k)
    torch.cuda.synchronize()
    written = int((cache[:, 0].float().abs().sum(dim=(2, 3)) != 0).sum().item())
    assert written == 30


def test_prefill_plan_tiles_costs_and_queues(gpu):
    """The plan's tile list, cost prefix, per-XCD queue cuts and unit order, read from the
    workspace and checked against a host listing (more than 1024 requests and more than
    1024 tiles in one request, so both of the plan's loops take several rounds)."""
    hq, hkv, d, ps = 28, 4, 128, 16
    g_ = hq // hkv
    rng = np.random.default_rng(11)
    b = 1500
    new = np.ones(b, dtype=np.int64)
    kvl = rng.integers(1, 3000, size=b)
    for r, (qn, kn) in {3: (40000, 41000), 700: (513, 600), 1100: (3, 3), 1499: (2048, 9000)}.items():
        new[r], kvl[r] = qn, kn
    qo, kv_indptr, kv_indices, last = custom_batch(kvl, ps, int(sum(-(-kvl // ps))) + 4, 5, new_lens=new)
    w = FlashInferPrefillWrapper(workspace(gpu, 512 << 20), hq, hkv, d, ps, device=gpu)
    w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last),
           causal=True)
    torch.cuda.synchronize()
    # host listing: tiles of 256 rows, request order, last rows first; cost = 32-key steps to the causal limit
    short = _lib.lib().mi_prefill_short_rows(b, hq, hkv, d)
    assert short == 8  # 1500 requests, head_dim 128, 7 q-heads per kv-head: the short part reads kv-head pairs
    exp_tiles, exp_cost = [], []
    for r in range(b):
        rows = int(new[r]) * g_
        if rows <= short:
            continue
        n = -(-rows // 256)
        for i in range(n):
            row0 = (n - 1 - i) * 256
            last_row = min(row0 + 256, rows) - 1
            kv_end = min(int(kvl[r]), int(kvl[r]) - int(new[r]) + last_row // g_ + 1)
            exp_tiles.append((r, row0))
            exp_cost.append(-(-kv_end // 32) if kv_end > 0 else 0)
    nt = len(exp_tiles)
    assert max(-(-int(new[r]) * g_ // 256) for r in range(b)) > 1024
    max_tok = w._plan_max_tokens
    mt = -(-max_tok * g_ // 256) + b
    al = lambda x: -(-x // 256) * 256
    o_tiles = 256 + 9 * 32 * 4
    o_tcum = al(o_tiles + 8 * mt)
    o_order = al(o_tcum + 4 * (mt + 1))
    ws = w._workspace
    i32 = lambda off, n: ws[off:off + 4 * n].cpu().view(torch.int32).numpy().astype(np.int64)
    hdr = i32(0, 17)
    units = nt * hkv
    assert hdr[0] == nt and hdr[1] == units
    tiles = i32(o_tiles, 2 * nt).reshape(-1, 2)
    assert [tuple(t) for t in tiles.tolist()] == exp_tiles
    tcum = i32(o_tcum, nt + 1)
    assert tcum.tolist() == [0] + np.cumsum(exp_cost).tolist()
    ct = int(tcum[nt])
    total = ct * hkv
    prefix = np.array([h * ct + tcum[t] for h in range(hkv) for t in range(nt)] + [total])
    cuts = hdr[8:17].tolist()
    assert cuts[0] == 0 and cuts[8] == units and cuts == sorted(cuts)
    for x in range(1, 8):
        target = -(-x * total // 8)
        assert cuts[x] == int(np.argmax(prefix >= target))
    order = i32(o_order, units)
    cost_u = np.array([exp_cost[u % nt] for u in range(units)])
    for x in range(8):
        seg = order[cuts[x]:cuts[x + 1]]
        assert sorted(seg.tolist()) == list(range(cuts[x], cuts[x + 1]))
        keys = np.minimum(cost_u[seg], 1023)
        assert (np.diff(keys) <= 0).all(), f"queue {x} not heaviest first"


@pytest.mark.parametrize("hq,hkv,d,causal", [(28, 4, 128, True), (28, 4, 128, False), (8, 1, 256, True)])
def test_prefill_long_context_page_chunks(gpu, hq, hkv, d, causal):
    """Contexts longer than the 2048 page ids the kernel stages in LDS at once (several
    page chunks per tile), against fp32 attention on the GPU."""
    ps = 16
    kv_lens = [40000, 33000, 70000, 2100]
    new_lens = [64, 300, 5, 2100]
    qo, kv_indptr, kv_indices, last = custom_batch(kv_lens, ps, sum(-(-np.array(kv_lens) // ps)) + 8, 21,
                                                   new_lens=new_lens)
    pool = int(kv_indices.max()) + 1
    log(f"long context hq={hq} hkv={hkv} d={d} causal={causal}: kv={kv_lens} new={new_lens}")
    cache = torch.empty(pool, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    cache.normal_(generator=torch.Generator(device=gpu).manual_seed(5))
    g = torch.Generator().manual_seed(6)
    ntok = int(qo[-1])
    q = torch.randn(ntok, hq, d, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    w = FlashInferPrefillWrapper(workspace(gpu, 512 << 20), hq, hkv, d, ps, device=gpu)
    w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last),
           causal=causal)
    w.set_kv_cache(cache, k, v)
    out = w.run(q, cache)
    ref = _torch_ref_gpu(q, cache, qo, kv_indptr, kv_indices, last, causal, hq, hkv)
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    log(f"  max_abs={err:.3e}")
    assert err < TOL


def test_prefill_head_dim_256_full_batch(gpu):
    """The head_dim 256 batch the bench times, at full size: 8 requests of 2048 new
    tokens over 4096..7680-token contexts, 16 q / 2 kv heads, page 16, causal, pages
    in a random order, against fp32 attention on the GPU."""
    hq, hkv, d, ps = 16, 2, 256, 16
    kv_lens = [4096 + 512 * i for i in range(8)]
    new = [2048] * 8
    pages = [-(-n // ps) for n in kv_lens]
    pool = sum(pages) + 8
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    kv_indices = np.random.default_rng(0).permutation(pool)[: kv_indptr[-1]].astype(np.int32)
    last = np.array([n - (p - 1) * ps for n, p in zip(kv_lens, pages)], np.int32)
    qo = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    log(f"head_dim 256 full batch: kv={kv_lens} new={new}")
    g = torch.Generator(device=gpu).manual_seed(5)
    cache = torch.randn(pool, 2, ps, hkv, d, device=gpu, generator=g).to(torch.bfloat16)
    q = torch.randn(int(qo[-1]), hq, d, device=gpu, generator=g).to(torch.bfloat16)
    w = FlashInferPrefillWrapper(workspace(gpu, 512 << 20), hq, hkv, d, ps, device=gpu)
    w.plan(*(torch.from_numpy(a) for a in (qo, kv_indptr, kv_indices, last)), causal=True)
    out = w.run(q, cache)
    ref = _torch_ref_gpu(q, cache, qo, kv_indptr, kv_indices, last, True, hq, hkv)
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    log(f"  max_abs={err:.3e}")
    assert err < TOL


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_d256_chunk_remainders(gpu, causal):
    """Head_dim 256 (tiles loaded straight into LDS, page offsets staged 512 tiles at a time):
    contexts that leave 1, 2 and 3 tiles in their last chunk and a one-tile request, with NaN
    in every last page's slots past kv_len, against fp32 attention on the GPU."""
    hq, hkv, d, ps = 16, 2, 256, 16
    kv_lens = [16385, 16424, 16470, 31]   # 513, 514, 515 and 1 tiles of 32 keys
    new_lens = [37, 5, 64, 31]
    qo, kv_indptr, kv_indices, last = custom_batch(kv_lens, ps, sum(-(-np.array(kv_lens) // ps)) + 8, 23,
                                                   new_lens=new_lens)
    pool = int(kv_indices.max()) + 1
    log(f"d256 chunk remainders causal={causal}: kv={kv_lens} new={new_lens}")
    cache = torch.empty(pool, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    cache.normal_(generator=torch.Generator(device=gpu).manual_seed(7))
    g = torch.Generator().manual_seed(8)
    ntok = int(qo[-1])
    q = torch.randn(ntok, hq, d, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    w = FlashInferPrefillWrapper(workspace(gpu, 512 << 20), hq, hkv, d, ps, device=gpu)
    w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last),
           causal=causal)
    w.set_kv_cache(cache, k, v)
    for r in range(len(kv_lens)):  # after the append: slots past each request's last key
        page = int(kv_indices[kv_indptr[r + 1] - 1])
        cache[page, :, int(last[r]):] = float("nan")
    out = w.run(q, cache)
    ref = _torch_ref_gpu(q, cache, qo, kv_indptr, kv_indices, last, causal, hq, hkv)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    err = (out.float() - ref).abs().max().item()
    log(f"  max_abs={err:.3e}")
    assert err < TOL


def test_prefill_plan_index_inputs(gpu):
    """plan() over int64, strided and device index tensors gives bit-identical
    outputs and appended pages to int32 contiguous CPU tensors."""
    hq, hkv, d, ps = 28, 4, 128, 16
    kv_lens, new_lens = [40, 700, 1300, 33], [40, 1, 600, 2]
    qo, kv_indptr, kv_indices, last = custom_batch(kv_lens, ps, 200, seed=5, new_lens=new_lens)
    ntok = int(qo[-1])
    g = torch.Generator().manual_seed(13)
    cache0 = random_cache(200, ps, hkv, d, 5).to(gpu)
    q = torch.randn(ntok, hq, d, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(ntok, hkv, d, generator=g).to(torch.bfloat16).to(gpu)

    def strided(a):
        return torch.from_numpy(np.repeat(np.asarray(a, dtype=np.int32), 2))[::2]

    arrays = [qo, kv_indptr, kv_indices, last]
    variants = {
        "int32": [torch.as_tensor(np.asarray(a, dtype=np.int32)) for a in arrays],
        "int64": [torch.as_tensor(np.asarray(a, dtype=np.int64)) for a in arrays],
        "strided": [strided(a) for a in arrays],
    }
    variants["device"] = [t.to(gpu) for t in variants["int32"]]
    results = {}
    for name, idx in variants.items():
        cache = cache0.clone()
        w = FlashInferPrefillWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
        w.plan(*idx, causal=True, dtype=torch.bfloat16)
        w.set_kv_cache(cache, k, v)
        out = w.run(q, cache)
        torch.cuda.synchronize()
        results[name] = (out.cpu(), cache.cpu())
        log(f"prefill plan index inputs: {name}")
    base = results["int32"]
    for name, (out, cache) in results.items():
        assert torch.equal(out.view(torch.int16), base[0].view(torch.int16)), name
        assert torch.equal(cache.view(torch.int16), base[1].view(torch.int16)), name
