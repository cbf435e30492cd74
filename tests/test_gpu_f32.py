"""GPU parity of the fp32 KV path (fp32 pool, q and output) against the CPU oracle.

The reference allocates the KV pool in the autocast dtype, fp32 included
(``mstar/engine/kv_cache_engine.py:104-105, 132-136``); Pi0.5's real-weights
test runs with ``kv_cache_type=torch.float32``
(``test/integration/test_pi05_real_weights.py:1006-1011``) at 8 q / 1 kv
heads, head_dim 256, page_size 16.  Bars:

* append into an fp32 cache bit-exact (fp32 source copied, bf16 source
  widened), with the oracle's append;
* attention within max-abs 2e-5 of the oracle's fp32 attention over the same
  cache: both sides compute in fp32 and differ only in summation order and in
  the exponential (the kernel's exp2 against libm's exp); measured errors are
  0.5-2e-6, three orders of magnitude below the bf16 bar of 2e-2.
"""

import pytest
import torch

from gpu_helpers import A, custom_batch, log, max_abs, workspace
from mstar_amd.paged_attention import FlashInferPrefillWrapper
from test_gpu_decode import _run_decode, _ws_for_items
from test_gpu_prefill import MIX_KV, MIX_NEW, _run_prefill

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-5
F32 = torch.float32


@pytest.mark.parametrize("hq,hkv,d,ps", [(8, 1, 256, 16), (32, 4, 128, 16), (24, 8, 64, 32), (16, 16, 128, 16),
                                         (28, 4, 128, 16)])
def test_f32_decode_shapes(gpu, hq, hkv, d, ps):
    lens = [1, 15, 16, 17, 255, 256, 257, 1000, 3001, 20000]
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, 1600, seed=hq + d + ps)
    out, ref = _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, 1600, seed=3, dtype=F32)
    err = max_abs(out, ref)
    log(f"f32 decode hq={hq} hkv={hkv} d={d} ps={ps}: max_abs={err:.3e}")
    assert out.dtype == F32 and err < TOL_F32


@pytest.mark.parametrize("hq,hkv,d,ps", [(32, 4, 128, 16), (8, 1, 256, 32)])
def test_f32_decode_long_items(gpu, hq, hkv, d, ps):
    """Items of over 256 pages (several 64-page windows per wavefront) and a split request."""
    lens = [40000, 3000, 17]
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, 3000, seed=ps + d)
    hdr = []
    out, ref = _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, 3000, seed=ps, dtype=F32,
                           ws_bytes=_ws_for_items(len(lens), hkv, d, len(lens) + 2), plan_header=hdr)
    err = max_abs(out, ref)
    log(f"f32 decode long items hq={hq} d={d} ps={ps}: items={hdr[2]} item_pages={hdr[3]} max_abs={err:.3e}")
    assert hdr[3] > 256 and err < TOL_F32


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv,d,ps", [(28, 4, 128, 16), (8, 1, 256, 16), (16, 2, 64, 32), (8, 8, 128, 64)])
def test_f32_prefill_ragged_mix(gpu, causal, hq, hkv, d, ps):
    out, ref = _run_prefill(gpu, hq, hkv, d, ps, MIX_KV, MIX_NEW, causal, seed=hq + d, dtype=F32)
    err = max_abs(out, ref)
    log(f"f32 prefill causal={causal} hq={hq} hkv={hkv} d={d} ps={ps}: max_abs={err:.3e}")
    assert out.dtype == F32 and err < TOL_F32


def test_f32_prefill_long_chunks(gpu):
    """Several 256-row tiles per request, causal over a long prefix."""
    out, ref = _run_prefill(gpu, 28, 4, 128, 16, [5000, 1300, 64], [1200, 700, 64], True, seed=9, dtype=F32)
    err = max_abs(out, ref)
    log(f"f32 prefill long chunks: max_abs={err:.3e}")
    assert err < TOL_F32


def test_f32_reference_scenario_prefix_then_suffix(gpu):
    """The reference's paged-prefill scenario (test_pi05_reference_equivalence.py:645-719) on an fp32 cache."""
    torch.manual_seed(0)
    hq, hkv, d, ps, max_pages, prefix_len, suffix_len = 8, 1, 256, 16, 32, 24, 4
    cache = torch.zeros(max_pages, 2, ps, hkv, d, device=gpu, dtype=F32)
    w = FlashInferPrefillWrapper(workspace(gpu), hq, hkv, d, ps, device=gpu)
    qp, kp, vp = (torch.randn(prefix_len, h, d, device=gpu) for h in (hq, hkv, hkv))
    n_pref = (prefix_len + ps - 1) // ps
    w.plan(torch.tensor([0, prefix_len], dtype=torch.int32), torch.tensor([0, n_pref], dtype=torch.int32),
           torch.arange(n_pref, dtype=torch.int32), torch.tensor([prefix_len - (n_pref - 1) * ps], dtype=torch.int32),
           causal=False, dtype=F32)
    w.set_kv_cache(cache, kp, vp)
    out = w.run(qp, cache)
    ref, _ = A.attend(qp.cpu(), kp.cpu(), vp.cpu(), causal=False, sm_scale=d ** -0.5)
    assert torch.equal(cache[:n_pref, 0].reshape(-1, hkv, d)[:prefix_len], kp)
    e1 = max_abs(out, ref)
    qs, ks, vs = (torch.randn(suffix_len, h, d, device=gpu) for h in (hq, hkv, hkv))
    total = prefix_len + suffix_len
    n_after = (total + ps - 1) // ps
    w.plan(torch.tensor([0, suffix_len], dtype=torch.int32), torch.tensor([0, n_after], dtype=torch.int32),
           torch.arange(n_after, dtype=torch.int32), torch.tensor([total - (n_after - 1) * ps], dtype=torch.int32),
           causal=False, dtype=F32)
    w.set_kv_cache(cache, ks, vs)
    out2 = w.run(qs, cache)
    ref2, _ = A.attend(qs.cpu(), torch.cat([kp, ks]).cpu(), torch.cat([vp, vs]).cpu(), causal=False,
                       sm_scale=d ** -0.5)
    e2 = max_abs(out2, ref2)
    log(f"f32 reference scenario: prefix {e1:.3e} suffix {e2:.3e}")
    assert e1 < TOL_F32 and e2 < TOL_F32


def test_f32_append_from_bf16_widens_exactly(gpu):
    qo, kv_indptr, kv_indices, last = custom_batch([5, 70, 700], 16, 64, seed=3)
    from mstar_amd.paged_attention import FlashInferDecodeWrapper

    cache = torch.zeros(64, 2, 16, 2, 128, dtype=F32, device=gpu)
    w = FlashInferDecodeWrapper(workspace(gpu), 8, 2, 128, 16, device=gpu)
    w.plan(torch.as_tensor(kv_indptr), torch.as_tensor(kv_indices), torch.as_tensor(last), dtype=F32)
    k = torch.randn(3, 2, 128, device=gpu).to(torch.bfloat16)
    v = torch.randn(3, 2, 128, device=gpu).to(torch.bfloat16)
    w.set_kv_cache(cache, k, v)
    loc = w.kv_cache_locations
    assert torch.equal(cache[loc[:, 0], 0, loc[:, 1]], k.float())
    assert torch.equal(cache[loc[:, 0], 1, loc[:, 1]], v.float())
