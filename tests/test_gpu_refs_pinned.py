"""The GPU fp32 references of the full-size tests, pinned to the CPU oracle.

``test_gpu_fullsize._ref_decode`` and ``test_gpu_prefill._torch_ref_gpu``
compute fp32 attention on the GPU because the CPU oracle would take minutes at
c2-c5 size.  Here each is compared with ``oracle.attention.paged_attention``
(itself pinned against torch SDPA, a float64 loop and closed forms in
``test_oracle_attention.py``) on small batches of the same shapes and cache
formats, so the full-size checks rest on the oracle.  Both sides are fp32;
the bound covers their different summation orders only.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import A, custom_batch, log, random_cache
from test_gpu_fullsize import _ref_decode
from test_gpu_prefill import _torch_ref_gpu

pytestmark = pytest.mark.gpu

FP32_BOUND = 2e-4


@pytest.mark.parametrize("hq,hkv,d,fp8", [(32, 4, 128, False), (24, 8, 128, False), (32, 4, 128, True),
                                         (8, 1, 256, False)])
def test_ref_decode_matches_oracle(gpu, hq, hkv, d, fp8):
    ps = 16
    lens = [1, 15, 16, 17, 300, 1025, 4000, 77]
    _, kv_indptr, kv_indices, last = custom_batch(lens, ps, 400, seed=5)
    src = random_cache(400, ps, hkv, d, 6, torch.float32)
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    if fp8:
        ks = A.head_scales(src[:, 0].reshape(-1, hkv, d))
        vs = A.head_scales(src[:, 1].reshape(-1, hkv, d))
        cache = torch.empty(400, 2, ps, hkv, d, dtype=torch.float8_e4m3fn)
        cache[:, 0] = A.quantize_e4m3(src[:, 0].reshape(-1, hkv, d), ks).view(400, ps, hkv, d)
        cache[:, 1] = A.quantize_e4m3(src[:, 1].reshape(-1, hkv, d), vs).view(400, ps, hkv, d)
    else:
        ks = vs = None
        cache = src.to(torch.bfloat16)
    want = A.paged_attention(q, cache, None, kv_indptr, kv_indices, last, causal=False, k_scale=ks, v_scale=vs)
    got = _ref_decode(q.to(gpu), cache.to(gpu), kv_indptr, kv_indices, last, hq, hkv,
                      ks.to(gpu) if fp8 else None, vs.to(gpu) if fp8 else None)
    err = (got.cpu() - want).abs().max().item()
    log(f"_ref_decode vs oracle hq={hq} hkv={hkv} d={d} fp8={fp8}: {err:.2e}")
    assert err < FP32_BOUND


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (8, 1, 256)])
def test_torch_ref_gpu_matches_oracle(gpu, hq, hkv, d, causal):
    ps = 16
    kv_lens = [600, 33, 1, 130, 2000, 16]
    new_lens = [300, 2, 1, 0, 700, 16]
    qo, kv_indptr, kv_indices, last = custom_batch(kv_lens, ps, 300, seed=8, new_lens=new_lens)
    cache = random_cache(300, ps, hkv, d, 9, torch.bfloat16)
    q = torch.randn(int(qo[-1]), hq, d, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    want = A.paged_attention(q, cache, qo, kv_indptr, kv_indices, last, causal=causal)
    got = _torch_ref_gpu(q.to(gpu), cache.to(gpu), qo, kv_indptr, kv_indices, np.asarray(last), causal, hq, hkv)
    err = (got.cpu() - want).abs().max().item()
    log(f"_torch_ref_gpu vs oracle hq={hq} hkv={hkv} d={d} causal={causal}: {err:.2e}")
    assert err < FP32_BOUND
