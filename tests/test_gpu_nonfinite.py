"""Non-finite values in the KV cache.

* **Heads stay apart.**  Decode batches of >= 128 requests at head_dim 128
  with at most 8 q-heads per kv-head and a 16-bit cache run the paired kernel
  (two kv-heads as one 256-element row).  An +Inf or NaN in one kv-head's keys
  or values, inside ``kv_len``, must leave the other head of its pair exactly
  as the per-head computation gives it (the reference's FlashInfer kernel
  keeps heads apart, ``flashinfer_utils.py:455-465``).  The poisoned head itself
  must follow a textbook fp32 softmax: a row with a +Inf or NaN score is NaN,
  a -Inf score drops its key, an Inf value makes the elements it reaches
  non-finite.  The same batch at 8 requests runs the per-head kernel.
* **Slots past the end are never read as data.**  The unwritten slots of a
  request's last page (past ``kv_len``) may hold anything; filled with NaN and
  Inf bit patterns they must give outputs bit-identical to finite filler, for
  the per-head, paired, fp8, fp32 and prefill kernels.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import A, P, custom_batch, decode_reference, log, random_cache, workspace
from mstar_amd.paged_attention import FlashInferDecodeWrapper, FlashInferPrefillWrapper

pytestmark = pytest.mark.gpu

TOL = 2e-2
HQ, HKV, D, PS = 32, 4, 128, 16
INT_OF = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
          torch.float8_e4m3fn: torch.uint8}
# NaN, +Inf, -Inf and a negative NaN of each format (e4m3fn has no Inf: its two NaNs)
PATTERNS = {
    torch.bfloat16: [0x7FC0, 0x7F80, -0x0080, -0x003F],  # 0x7FC0, 0x7F80, 0xFF80, 0xFFC1 as int16
    torch.float16: [0x7E00, 0x7C00, -0x0400, -0x01FF],
    torch.float32: [0x7FC00000, 0x7F800000, -0x00800000, -0x003FFFFF],
    torch.float8_e4m3fn: [0x7F, 0xFF],
}


def _batch(lens, seed, new_lens=None, pool_extra=8):
    npages = int(sum(-(-np.asarray(lens) // PS)))
    qo, kv_indptr, kv_indices, last = custom_batch(lens, PS, npages + pool_extra, seed, new_lens=new_lens)
    return qo, kv_indptr, kv_indices, last, npages + pool_extra


def _decode(gpu, cache_cpu, q, k_new, v_new, kv_indptr, kv_indices, last, scales=(None, None), hq=HQ, hkv=HKV):
    cache = cache_cpu.to(gpu)
    w = FlashInferDecodeWrapper(workspace(gpu, 64 << 20), hq, hkv, cache.shape[-1], PS, device=gpu)
    w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last), dtype=q.dtype)
    sc = tuple(s.to(gpu) if s is not None else None for s in scales)
    w.set_kv_cache(cache, k_new.to(gpu), v_new.to(gpu), *sc)
    out = w.run(q.to(gpu), cache, *sc)
    torch.cuda.synchronize()
    return out.cpu()


def _textbook(q, k, v):
    """fp32 softmax(q k^T / sqrt(D)) v for one request and kv-head, no special
    handling of non-finite values: q [G, D], k/v [kv, D] -> [G, D]."""
    s = (q.float() @ k.float().t()) * D ** -0.5
    return torch.softmax(s, dim=-1) @ v.float()


@pytest.mark.parametrize("batch", [128, 8])
def test_poisoned_kv_head_stays_in_its_head(gpu, batch):
    rng = np.random.default_rng(batch)
    lens = rng.integers(20, 400, batch)
    lens[:3] = [5000, 3100, 40]  # long requests are split into several items (merged partials)
    qo, kv_indptr, kv_indices, last, pool = _batch(lens, seed=batch)
    g = torch.Generator().manual_seed(batch + 1)
    cache_cpu = random_cache(pool, PS, HKV, D, batch + 2, torch.bfloat16)
    q = torch.randn(batch, HQ, D, generator=g).to(torch.bfloat16)
    k_new = torch.randn(batch, HKV, D, generator=g).to(torch.bfloat16)
    v_new = torch.randn(batch, HKV, D, generator=g).to(torch.bfloat16)
    inf, nan = float("inf"), float("nan")
    # (request, token, kv-head, K=0/V=1, element, value): odd heads of pairs (1, 3) and an even one (2)
    poison = [(0, 1234, 1, 0, 5, inf), (0, 4321, 1, 1, 77, inf), (1, 3000, 3, 0, 9, nan),
              (2, 10, 1, 0, 100, -inf), (3, 2, 2, 0, 0, inf), (4, 7, 3, 1, 127, -inf)]
    for r, tok, h, kv, e, val in poison:
        page = kv_indices[kv_indptr[r] + tok // PS]
        cache_cpu[page, kv, tok % PS, h, e] = val
    out = _decode(gpu, cache_cpu, q, k_new, v_new, kv_indptr, kv_indices, last)
    ref_cache = cache_cpu.clone()
    loc = P.decode_locations(kv_indptr, kv_indices, last)
    A.append(ref_cache, loc[:, 0], loc[:, 1], k_new, v_new)
    ref = decode_reference(q, ref_cache, kv_indptr, kv_indices, last)
    G = HQ // HKV
    bad = {(r, h) for r, _, h, _, _, _ in poison}
    for r in range(batch):
        kv_len = (kv_indptr[r + 1] - kv_indptr[r] - 1) * PS + last[r]
        for h in range(HKV):
            o = out[r, h * G:(h + 1) * G].float()
            if (r, h) not in bad:  # every other head, its pair neighbour included: finite and in tolerance
                assert torch.isfinite(o).all(), (r, h)
                assert (o - ref[r, h * G:(h + 1) * G]).abs().max().item() < TOL, (r, h)
                continue
            k, v = A.gather_request_kv(ref_cache, kv_indices[kv_indptr[r]:kv_indptr[r + 1]], kv_len)
            want = _textbook(q[r, h * G:(h + 1) * G], k[:, h], v[:, h])
            assert torch.equal(torch.isfinite(o), torch.isfinite(want)), (r, h)
            fin = torch.isfinite(want)
            if fin.any():
                assert (o[fin] - want[fin]).abs().max().item() < TOL, (r, h)
            log(f"B={batch} request {r} kv-head {h}: {int((~fin).sum())} non-finite elements, as the textbook")


def _poison_tails(cache_cpu, kv_indptr, kv_indices, last, dtype):
    """Fill the slots past kv_len of every request's last page (K and V) with
    the format's NaN/Inf patterns, cycling over elements."""
    it = INT_OF[dtype]
    raw = cache_cpu.view(it)
    pats = torch.tensor(PATTERNS[dtype], dtype=torch.int64)
    n = 0
    for r in range(len(last)):
        if kv_indptr[r + 1] == kv_indptr[r] or last[r] == PS:
            continue
        page = kv_indices[kv_indptr[r + 1] - 1]
        tail = raw[page, :, last[r]:]
        idx = torch.arange(tail.numel()) % len(pats)
        raw[page, :, last[r]:] = pats[idx].view(tail.shape).to(it) if it != torch.uint8 else \
            (pats[idx] & 0xFF).to(torch.uint8).view(tail.shape)
        n += tail.numel()
    return n


def _fp8_cache(src):
    pool, _, ps, hkv, d = src.shape
    ks = A.head_scales(src[:, 0].reshape(-1, hkv, d))
    vs = A.head_scales(src[:, 1].reshape(-1, hkv, d))
    c = torch.empty(pool, 2, ps, hkv, d, dtype=torch.float8_e4m3fn)
    c[:, 0] = A.quantize_e4m3(src[:, 0].reshape(-1, hkv, d), ks).view(pool, ps, hkv, d)
    c[:, 1] = A.quantize_e4m3(src[:, 1].reshape(-1, hkv, d), vs).view(pool, ps, hkv, d)
    return c, (ks, vs)


@pytest.mark.parametrize("batch,dtype", [(8, torch.bfloat16), (160, torch.bfloat16), (160, torch.float16),
                                         (8, torch.float8_e4m3fn), (160, torch.float8_e4m3fn),
                                         (8, torch.float32)])
def test_decode_ignores_slots_past_kv_len(gpu, batch, dtype):
    """batch 160 at 16-bit runs the paired kernel, the others per-head (fp8,
    fp32: their own kernels).  Decode appends one token, so the tails are the
    slots past it."""
    rng = np.random.default_rng(batch + 11)
    lens = rng.integers(2, 700, batch)
    lens[0] = 4000  # one split request
    qo, kv_indptr, kv_indices, last, pool = _batch(lens, seed=batch + 12)
    g = torch.Generator().manual_seed(batch + 13)
    src = random_cache(pool, PS, HKV, D, batch + 14, torch.float32)
    qdt = torch.bfloat16 if dtype == torch.float8_e4m3fn else dtype
    q = torch.randn(batch, HQ, D, generator=g).to(qdt)
    k_new = torch.randn(batch, HKV, D, generator=g).to(qdt)
    v_new = torch.randn(batch, HKV, D, generator=g).to(qdt)
    if dtype == torch.float8_e4m3fn:
        finite, scales = _fp8_cache(src)
    else:
        finite, scales = src.to(dtype), (None, None)
    poisoned = finite.clone()
    n = _poison_tails(poisoned, kv_indptr, kv_indices, last, dtype)
    a = _decode(gpu, finite, q, k_new, v_new, kv_indptr, kv_indices, last, scales)
    b = _decode(gpu, poisoned, q, k_new, v_new, kv_indptr, kv_indices, last, scales)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a.view(INT_OF[a.dtype]), b.view(INT_OF[b.dtype])), "non-finite tail slots changed the output"
    log(f"decode B={batch} {dtype}: {n} tail elements NaN/Inf, output bit-identical")


@pytest.mark.parametrize("dtype,causal,hq,hkv,d", [(torch.bfloat16, True, HQ, HKV, D), (torch.bfloat16, False, HQ, HKV, D),
                                                   (torch.float8_e4m3fn, True, HQ, HKV, D),
                                                   (torch.float32, True, HQ, HKV, D),
                                                   (torch.bfloat16, True, 8, 1, 256), (torch.bfloat16, False, 8, 1, 256),
                                                   (torch.float8_e4m3fn, True, 8, 1, 256)])
def test_prefill_ignores_slots_past_kv_len(gpu, dtype, causal, hq, hkv, d):
    """A ragged batch: long chunks (MFMA tiles; head_dim 256: the role-split
    tiles), short queries (decode kernel with qo_indptr) and single tokens;
    its appended tokens end mid-page."""
    kv_lens = [700, 1301, 33, 5, 250, 17, 900]
    new_lens = [300, 645, 2, 1, 250, 1, 9]
    qo, kv_indptr, kv_indices, last, pool = _batch(kv_lens, seed=31, new_lens=new_lens)
    g = torch.Generator().manual_seed(32)
    src = random_cache(pool, PS, hkv, d, 33, torch.float32)
    qdt = torch.bfloat16 if dtype == torch.float8_e4m3fn else dtype
    ntok = int(qo[-1])
    q = torch.randn(ntok, hq, d, generator=g).to(qdt)
    k = torch.randn(ntok, hkv, d, generator=g).to(qdt)
    v = torch.randn(ntok, hkv, d, generator=g).to(qdt)
    if dtype == torch.float8_e4m3fn:
        finite, scales = _fp8_cache(src)
    else:
        finite, scales = src.to(dtype), (None, None)
    poisoned = finite.clone()
    n = _poison_tails(poisoned, kv_indptr, kv_indices, last, dtype)
    outs = []
    for c in (finite, poisoned):
        cache = c.to(gpu)
        w = FlashInferPrefillWrapper(workspace(gpu, 64 << 20), hq, hkv, d, PS, device=gpu)
        w.plan(torch.as_tensor(qo), torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last),
               causal=causal, dtype=qdt)
        sc = tuple(s.to(gpu) if s is not None else None for s in scales)
        w.set_kv_cache(cache, k.to(gpu), v.to(gpu), *sc)
        outs.append(w.run(q.to(gpu), cache, *sc).cpu())
        torch.cuda.synchronize()
    a, b = outs
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a.view(INT_OF[a.dtype]), b.view(INT_OF[b.dtype])), "non-finite tail slots changed the output"
    log(f"prefill {dtype} causal={causal} heads {hq}/{hkv} d={d}: {n} tail elements NaN/Inf, output bit-identical")
