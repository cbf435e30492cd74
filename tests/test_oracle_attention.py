"""Pin the attention / merge / fp8 / append oracle (oracle/attention.py).

Independent checks: torch's scaled_dot_product_attention (a library routine),
a float64 per-query loop written from positions (query at absolute position
prefix+j sees keys at positions <= its own), closed forms (zero query ->
mean of V; one key -> that V row), the merge identity (attention over split
key sets merged == attention over all keys), and an exhaustive
nearest-code search over the 256 e4m3fn code points.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A


def _rand(*shape, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 1), (4, 4), (28, 4)])
def test_attend_matches_sdpa_noncausal(hq, hkv):
    q = _rand(5, hq, 64, seed=1)
    k = _rand(37, hkv, 64, seed=2)
    v = _rand(37, hkv, 64, seed=3)
    out, _ = A.attend(q, k, v, causal=False, sm_scale=1 / 8)
    ref = F.scaled_dot_product_attention(
        q.transpose(0, 1), k.repeat_interleave(hq // hkv, 1).transpose(0, 1),
        v.repeat_interleave(hq // hkv, 1).transpose(0, 1), scale=1 / 8,
    ).transpose(0, 1)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)


def test_attend_causal_square_matches_sdpa():
    q = _rand(19, 4, 32, seed=4)
    k = _rand(19, 2, 32, seed=5)
    v = _rand(19, 2, 32, seed=6)
    out, _ = A.attend(q, k, v, causal=True, sm_scale=0.3)
    ref = F.scaled_dot_product_attention(
        q.transpose(0, 1), k.repeat_interleave(2, 1).transpose(0, 1), v.repeat_interleave(2, 1).transpose(0, 1),
        is_causal=True, scale=0.3,
    ).transpose(0, 1)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)


def test_attend_causal_with_prefix_against_position_loop():
    qo, kv, hq, hkv, d = 6, 23, 6, 3, 16
    q, k, v = _rand(qo, hq, d, seed=7), _rand(kv, hkv, d, seed=8), _rand(kv, hkv, d, seed=9)
    out, lse = A.attend(q, k, v, causal=True, sm_scale=0.25)
    prefix = kv - qo
    for j in range(qo):
        pos = prefix + j
        for h in range(hq):
            kh = h // (hq // hkv)
            s = np.array([0.25 * float((q[j, h].double() * k[i, kh].double()).sum()) for i in range(pos + 1)])
            w = np.exp(s - s.max())
            o = (w[:, None] * v[: pos + 1, kh].double().numpy()).sum(0) / w.sum()
            np.testing.assert_allclose(out[j, h].numpy(), o, atol=1e-5)
            np.testing.assert_allclose(float(lse[j, h]), s.max() + math.log(w.sum()), atol=1e-5)


def test_closed_forms():
    v = _rand(11, 1, 8, seed=10)
    k = _rand(11, 1, 8, seed=11)
    out, _ = A.attend(torch.zeros(1, 3, 8), k, v, causal=False, sm_scale=1.0)
    torch.testing.assert_close(out[0, 2], v[:, 0].mean(0), atol=1e-6, rtol=1e-6)
    out, _ = A.attend(_rand(1, 2, 8, seed=12), k[:1], v[:1], causal=False, sm_scale=1.0)
    torch.testing.assert_close(out[0, 1], v[0, 0])


def test_merge_of_split_keys_equals_full():
    q = _rand(3, 8, 32, seed=13)
    k = _rand(50, 2, 32, seed=14)
    v = _rand(50, 2, 32, seed=15)
    full, _ = A.attend(q, k, v, causal=False, sm_scale=0.2)
    cuts = [0, 7, 8, 31, 50]
    outs, lses = [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        o, l = A.attend(q, k[a:b], v[a:b], causal=False, sm_scale=0.2)
        outs.append(o)
        lses.append(l)
    # an empty part contributes nothing
    outs.append(torch.full_like(full, 123.0))
    lses.append(torch.full_like(lses[0], float("-inf")))
    torch.testing.assert_close(A.merge_states(outs, lses), full, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(A.merge_states(outs[:1], lses[:1]), outs[0])


def test_paged_gather_matches_contiguous():
    ps, hkv, d = 16, 2, 32
    g = torch.Generator().manual_seed(3)
    lens = [5, 16, 17, 40, 1]
    cache = torch.zeros(64, 2, ps, hkv, d)
    perm = torch.randperm(64, generator=g).tolist()
    kv_indptr, kv_indices, last = [0], [], []
    ks, vs = [], []
    for L in lens:
        npg = -(-L // ps)
        pages = [perm.pop() for _ in range(npg)]
        k = torch.randn(L, hkv, d, generator=g)
        v = torch.randn(L, hkv, d, generator=g)
        for t in range(L):
            cache[pages[t // ps], 0, t % ps] = k[t]
            cache[pages[t // ps], 1, t % ps] = v[t]
        kv_indices += pages
        kv_indptr.append(len(kv_indices))
        last.append(L - (npg - 1) * ps)
        ks.append(k)
        vs.append(v)
    q = torch.randn(len(lens), 4, d, generator=g)
    out = A.paged_attention(q, cache, None, kv_indptr, kv_indices, last, causal=False)
    for r in range(len(lens)):
        ref, _ = A.attend(q[r : r + 1], ks[r], vs[r], causal=False, sm_scale=1 / math.sqrt(d))
        torch.testing.assert_close(out[r : r + 1], ref)


def test_e4m3fn_cast_is_nearest_even_code():
    vals = A.e4m3fn_values()
    finite = np.where(~np.isnan(vals))[0]
    # every code decodes to its defined value through torch
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(codes), np.isnan(vals))
    np.testing.assert_array_equal(codes[finite], vals[finite])
    rng = np.random.default_rng(0)
    mags = np.concatenate([
        rng.uniform(-448, 448, 4000),
        rng.uniform(-0.02, 0.02, 2000),
        (vals[finite][:-1] + vals[finite][1:]) / 2,  # midpoints of neighbouring codes
        [0.0, -0.0, 448.0, -448.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11],
    ]).astype(np.float32)
    got = torch.from_numpy(mags).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    for x, c in zip(mags.astype(np.float64), got):
        if np.isnan(vals[c]):
            raise AssertionError(f"{x} -> NaN")
        err = np.abs(vals[finite] - x)
        best = finite[err == err.min()]
        if len(best) > 1:  # tie: even mantissa wins
            best = [b for b in best if (b & 1) == 0]
        # +0 / -0 both valid for x == 0
        assert vals[c] == vals[best[0]], (x, c, best)


def test_quantize_clamps_then_rounds():
    x = torch.tensor([[[1000.0, -1000.0, 1.0, 0.001]]])
    q = A.quantize_e4m3(x, torch.tensor([1.0]))
    assert q.float().tolist() == [[[448.0, -448.0, 1.0, 2.0 ** -9]]]  # 0.001 is nearest to the smallest subnormal
    s = A.head_scales(torch.tensor([[[2.0, -4.0]], [[1.0, 0.5]]]))
    assert s.tolist() == [float(np.float32(4.0) / np.float32(448.0))]


def test_append_casts_like_index_put():
    cache = torch.zeros(4, 2, 16, 1, 8, dtype=torch.bfloat16)
    k = _rand(3, 1, 8, seed=20)
    v = _rand(3, 1, 8, seed=21)
    A.append(cache, [2, 2, 0], [15, 0, 3], k, v)
    assert torch.equal(cache[2, 0, 15], k[0].to(torch.bfloat16))
    assert torch.equal(cache[0, 1, 3], v[2].to(torch.bfloat16))
    assert cache.float().abs().sum() == (k.to(torch.bfloat16).float().abs().sum() + v.to(torch.bfloat16).float().abs().sum())
