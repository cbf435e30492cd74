"""GPU parity: paged KV append is bit-exact with the oracle's index_put cast."""

import numpy as np
import pytest
import torch

from gpu_helpers import A, log
from mstar_amd import _lib
from mstar_amd.paged_attention import _append

pytestmark = pytest.mark.gpu


def _case(seed, n, pool, ps, hkv, d):
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(pool * ps, generator=g)[:n]
    return (slots // ps).to(torch.long), (slots % ps).to(torch.long), g


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dst", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
def test_append_bit_exact(gpu, src, dst):
    pool, ps, hkv, d, n = 40, 16, 4, 128, 300
    page, slot, g = _case(1, n, pool, ps, hkv, d)
    k = (torch.randn(n, hkv, d, generator=g) * 3).to(src)
    v = (torch.randn(n, hkv, d, generator=g) * 3).to(src)
    # exercise special values: exact RNE ties, signed zero, large magnitudes
    k[0, 0, :4] = torch.tensor([0.0, -0.0, 1e4, -3e5]).to(src)
    if src == torch.float32:
        k[1, 0, :3] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, float("inf")])
    cache_cpu = torch.zeros(pool, 2, ps, hkv, d).to(dst)
    scales = (None, None)
    if dst == torch.float8_e4m3fn:
        ks = A.head_scales(k.float())
        vs = A.head_scales(v.float())
        scales = (ks, vs)
    A.append(cache_cpu, page, slot, k, v, *scales)
    cache = torch.zeros(pool, 2, ps, hkv, d).to(dst).to(gpu)
    pg, sl = page.to(gpu), slot.to(gpu)
    sc = tuple(x.to(gpu) if x is not None else None for x in scales)
    _append(cache, k.to(gpu), v.to(gpu), pg, sl.data_ptr(), 1, n, None, *sc)
    torch.cuda.synchronize()
    got = cache.cpu().view(torch.uint8)
    exp = cache_cpu.view(torch.uint8)
    log(f"append {src}->{dst}: mismatching bytes {(got != exp).sum().item()}")
    assert torch.equal(got, exp)


@pytest.mark.parametrize("hkv,d", [(3, 72), (6, 128), (4, 96), (1, 256)])
def test_append_head_shapes(gpu, hkv, d):
    """Thread-to-element mapping for head counts and head_dims whose 8-element groups
    per token are not a power of two (the append accepts any head_dim divisible by 8)."""
    pool, ps, n = 24, 16, 200
    page, slot, g = _case(2, n, pool, ps, hkv, d)
    k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
    cache_cpu = torch.zeros(pool, 2, ps, hkv, d, dtype=torch.bfloat16)
    A.append(cache_cpu, page, slot, k, v)
    cache = torch.zeros(pool, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    _append(cache, k.to(gpu), v.to(gpu), page.to(gpu), slot.to(gpu).data_ptr(), 1, n, None, None, None)
    torch.cuda.synchronize()
    log(f"append hkv={hkv} d={d}")
    assert torch.equal(cache.cpu().view(torch.uint8), cache_cpu.view(torch.uint8))


def test_append_skips_out_of_range_and_device_count(gpu):
    pool, ps, hkv, d = 8, 16, 2, 64
    k = torch.randn(5, hkv, d).to(torch.bfloat16).to(gpu)
    v = torch.randn(5, hkv, d).to(torch.bfloat16).to(gpu)
    page = torch.tensor([0, -1, 8, 3, 2], dtype=torch.long, device=gpu)
    slot = torch.tensor([0, 0, 0, 16, 5], dtype=torch.long, device=gpu)
    cache = torch.zeros(pool, 2, ps, hkv, d, dtype=torch.bfloat16, device=gpu)
    count = torch.tensor([4], dtype=torch.int32, device=gpu)  # only the first 4 tokens are real
    _append(cache, k, v, page, slot.data_ptr(), 1, 5, count.data_ptr(), None, None)
    torch.cuda.synchronize()
    written = (cache.float().abs().sum(dim=(1, 3, 4)) != 0).nonzero().tolist()
    assert written == [[0, 0]]  # token 0 only: -1, 8 and slot 16 are out of range, token 4 is padding
    assert torch.equal(cache[0, 0, 0], k[0]) and torch.equal(cache[0, 1, 0], v[0])


def test_append_from_strided_views(gpu):
    # k/v as views of a fused qkv projection: [tokens, (hq+2hkv), d]
    pool, ps, hkv, d = 16, 16, 2, 128
    qkv = torch.randn(7, 8 + 2 * hkv, d).to(torch.bfloat16)
    k, v = qkv[:, 8:8 + hkv], qkv[:, 8 + hkv:]
    page = torch.tensor([3, 3, 3, 4, 9, 9, 0])
    slot = torch.tensor([0, 1, 2, 15, 7, 8, 0])
    cache_cpu = torch.zeros(pool, 2, ps, hkv, d, dtype=torch.bfloat16)
    A.append(cache_cpu, page, slot, k, v)
    cache = torch.zeros_like(cache_cpu).to(gpu)
    qkv_g = qkv.to(gpu)
    pg, sl = page.to(gpu), slot.to(gpu)
    _append(cache, qkv_g[:, 8:8 + hkv], qkv_g[:, 8 + hkv:], pg, sl.data_ptr(), 1, 7, None, None, None)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), cache_cpu)
