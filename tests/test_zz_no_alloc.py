"""mi_decode_noalloc (no workspace, static device scratch) against mi_decode_plan + mi_decode_run.

Bar: outputs and write locations bit-identical to the two-call path given a
workspace of MI_NOALLOC_SCRATCH_BYTES bytes (same split-KV plan, same
kernels), on two calls in a row, the second with a smaller batch that runs
over what the first left in the scratch; each output also within max-abs
2e-2 of the CPU oracle (fp32 attention).  All calls go through the C ABI.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from gpu_helpers import P, custom_batch, decode_reference, log, max_abs, random_cache
from mstar_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MI_NOALLOC_SCRATCH_BYTES
MI_ERR_WORKSPACE = -3


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _both(gpu, lens, new_lens, hq, hkv, d, ps, pool, seed, causal):
    """Run the two-call path and the no-alloc path on the same inputs."""
    L = _lib.lib()
    qo, kv_indptr, kv_indices, last = custom_batch(lens, ps, pool, seed=seed, new_lens=new_lens)
    b = len(lens)
    ntok = int(qo[-1])
    g = torch.Generator().manual_seed(seed + 77)
    cache_cpu = random_cache(pool, ps, hkv, d, seed)
    q_cpu = torch.randn(ntok, hq, d, generator=g).to(torch.bfloat16)
    cache = cache_cpu.to(gpu)
    q = q_cpu.to(gpu)
    ragged = new_lens is not None
    dev = lambda a: torch.as_tensor(a).to(gpu)
    t_qo, t_ip, t_idx, t_last = dev(qo), dev(kv_indptr), dev(kv_indices), dev(last)
    qo_ptr = t_qo.data_ptr() if ragged else None
    desc = _lib.paged_kv_desc(cache)
    scale = 1.0 / math.sqrt(d)
    stream = _lib.stream_ptr(gpu)
    outs, locs = [], []
    for noalloc in (False, True):
        out = torch.full((ntok, hq, d), float("nan"), dtype=torch.bfloat16, device=gpu)
        loc = torch.full((b, 2), -7, dtype=torch.long, device=gpu)
        if noalloc:
            st = L.mi_decode_noalloc(q.data_ptr(), _lib.MI_BF16, q.stride(0), q.stride(1), desc, qo_ptr,
                                     t_ip.data_ptr(), t_idx.data_ptr(), t_last.data_ptr(), b, hq, causal, scale,
                                     out.data_ptr(), out.stride(0), out.stride(1), loc.data_ptr(), stream)
            _lib.check(st, "mi_decode_noalloc")
        else:
            ws = torch.empty(SCRATCH_BYTES, dtype=torch.uint8, device=gpu)
            _lib.check(L.mi_decode_plan(qo_ptr, t_ip.data_ptr(), t_idx.data_ptr(), t_last.data_ptr(), b, ps, hq, hkv,
                                        d, loc.data_ptr(), ws.data_ptr(), SCRATCH_BYTES, stream), "mi_decode_plan")
            _lib.check(L.mi_decode_run(q.data_ptr(), _lib.MI_BF16, q.stride(0), q.stride(1), desc, qo_ptr,
                                       t_ip.data_ptr(), t_idx.data_ptr(), t_last.data_ptr(), b, hq, causal, scale,
                                       ws.data_ptr(), SCRATCH_BYTES, out.data_ptr(), out.stride(0), out.stride(1),
                                       stream), "mi_decode_run")
        torch.cuda.synchronize()
        outs.append(out.cpu())
        locs.append(loc.cpu())
    from oracle import attention as A

    ref = A.paged_attention(q_cpu, cache_cpu, qo if ragged else None, kv_indptr, kv_indices, last,
                            causal=bool(causal))
    return outs, locs, ref, (kv_indptr, kv_indices, last)


def test_noalloc_matches_workspace_path_twice(gpu):
    cases = [
        # long contexts force split-KV items (partials + merge) and several page windows per wave
        dict(lens=[20000, 17, 1, 4096, 9000, 300, 0, 12345], hq=32, hkv=4, d=128, ps=16, pool=4096, seed=1),
        # second call: smaller batch over the scratch the first one left behind
        dict(lens=[700, 5, 2500], hq=32, hkv=4, d=128, ps=16, pool=512, seed=2),
    ]
    for c in cases:
        log(f"noalloc decode B={len(c['lens'])} lens={c['lens']}")
        outs, locs, ref, (ip, idx, last) = _both(gpu, c["lens"], None, c["hq"], c["hkv"], c["d"], c["ps"], c["pool"],
                                                 c["seed"], 0)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), "outputs differ from the two-call path"
        assert torch.equal(locs[0], locs[1]), "write locations differ"
        held = np.diff(ip) > 0  # an empty page list gets (-1, -1), not a neighbour's page
        want = torch.as_tensor(P.decode_locations(ip, idx, last))
        assert torch.equal(locs[1][held], want[held])
        assert (locs[1][~held] == -1).all()
        err = max_abs(outs[1], ref)
        log(f"  max_abs vs oracle {err:.3e}")
        assert err < 2e-2


def test_noalloc_paired_plan_twice(gpu):
    """Batches of >= 128 requests at head_dim 128 with <= 8 q-heads per kv-head
    plan and run over kv-head pairs (a head_dim 256 plan over half the heads)
    through the same static scratch; two calls in a row, the second smaller,
    each bit-identical to the two-call path and within 2e-2 of the oracle."""
    rng = np.random.default_rng(12)
    for b, seed in ((160, 21), (128, 22)):
        lens = rng.integers(1, 900, b).tolist()
        lens[:2] = [9000, 4100]  # split requests: partials and merge in the scratch
        pool = int(sum(-(-np.array(lens) // 16))) + 16
        log(f"noalloc paired decode B={b}")
        outs, locs, ref, _ = _both(gpu, lens, None, 32, 4, 128, 16, pool, seed, 0)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), "outputs differ from the two-call path"
        assert torch.equal(locs[0], locs[1])
        err = max_abs(outs[1], ref)
        log(f"  max_abs vs oracle {err:.3e}")
        assert err < 2e-2


def test_noalloc_short_query_ragged(gpu):
    # two query tokens per request (qo_len * group = 16 rows), causal
    lens, new = [40, 3000, 17, 16], [2, 2, 2, 1]
    outs, locs, ref, _ = _both(gpu, lens, new, 16, 2, 128, 16, 256, 9, 1)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert max_abs(outs[1], ref) < 2e-2


def test_noalloc_rejects_batch_beyond_scratch(gpu):
    L = _lib.lib()
    cache = torch.zeros(4, 2, 16, 4, 128, dtype=torch.bfloat16, device=gpu)
    desc = _lib.paged_kv_desc(cache)
    dummy = torch.zeros(16, dtype=torch.int32, device=gpu)
    p = dummy.data_ptr()
    # 4 kv heads x head_dim 128: about 33 KB of partials per item; 4000 + 1 items do not fit 64 MiB
    st = L.mi_decode_noalloc(p, _lib.MI_BF16, 4096, 128, desc, None, p, p, p, 4000, 32, 0, 0.1, p, 4096, 128, None,
                             _lib.stream_ptr(gpu))
    assert st == MI_ERR_WORKSPACE
    assert L.mi_status_string(st)
