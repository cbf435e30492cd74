"""GPU parity sweep: seeded random decode and ragged prefill problems against the
CPU oracle, each drawn from the supported space (head_dim 64 / 128 / 256, page
sizes 16-128, group sizes 1-16, bf16 / fp16 / fp8-e4m3 / fp32 caches, one-token decode
contexts, empty prefill requests, batches large enough to pair kv-heads, prefill
chunks over long prefixes).  The draws are fixed by the seed, so a failure names a
reproducible case; every case logs its shape before it runs.

Same bars as the per-feature tests: append bit-exact, attention within 2e-2
(bf16 / fp16), 6e-2 (fp8) or 2e-5 (fp32) max-abs of fp32.
"""

import random

import numpy as np
import pytest
import torch

from gpu_helpers import custom_batch, log, max_abs
from test_gpu_decode import TOL_BF16, TOL_FP8, _run_decode
from test_gpu_prefill import _run_prefill

TOL_F32 = 2e-5  # fp32 caches: fp32 q, attention and output
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp8": torch.bfloat16, "fp32": torch.float32}
TOLS = {"bf16": TOL_BF16, "fp16": TOL_BF16, "fp8": TOL_FP8, "fp32": TOL_F32}

pytestmark = pytest.mark.gpu

HEADS = [(8, 8), (8, 2), (8, 1), (16, 1), (24, 8), (28, 4), (32, 4), (32, 2), (12, 4), (20, 4), (6, 2), (16, 16)]
PAGES = [16, 32, 48, 64, 128]


def _lens(rng: random.Random, n: int, hi: int) -> list[int]:
    out = []
    for _ in range(n):
        r = rng.random()
        out.append(0 if r < 0.05 else 1 if r < 0.1 else rng.choice([15, 16, 17]) if r < 0.2 else rng.randint(2, hi))
    return out


@pytest.mark.parametrize("seed", range(24))
def test_decode_sweep(gpu, seed):
    rng = random.Random(1000 + seed)
    d = rng.choice([64, 128, 128, 256])
    hq, hkv = rng.choice(HEADS)
    ps = rng.choice(PAGES)
    kind = rng.choice(["bf16", "bf16", "fp16", "fp8", "fp32"])
    # every fourth case is a batch that takes the paired-kv-head kernels (B >= 128, D = 128)
    big = seed % 4 == 3
    if big:
        d, (hq, hkv) = 128, rng.choice([(32, 4), (24, 8), (16, 2), (8, 2)])
    b = rng.randint(128, 160) if big else rng.randint(1, 12)
    # decode lengths count the appended token, so every request holds at least one
    lens = [max(x, 1) for x in _lens(rng, b, 600 if big else 3000)]
    pool = int(sum(-(-np.array(lens) // ps))) + 8
    log(f"decode sweep seed={seed}: hq={hq} hkv={hkv} d={d} ps={ps} {kind} B={b} max_len={max(lens)}")
    _, kv_indptr, kv_indices, last = custom_batch(lens, ps, pool, seed)
    out, ref = _run_decode(gpu, hq, hkv, d, ps, kv_indptr, kv_indices, last, pool, seed, dtype=DTYPES[kind],
                           fp8=kind == "fp8")
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < TOLS[kind]


@pytest.mark.parametrize("seed", range(16))
def test_prefill_sweep(gpu, seed):
    rng = random.Random(2000 + seed)
    d = rng.choice([64, 128, 128, 256])
    hq, hkv = rng.choice(HEADS)
    ps = rng.choice(PAGES)
    kind = rng.choice(["bf16", "bf16", "fp16", "fp8", "fp32"])
    causal = rng.random() < 0.75
    b = rng.randint(1, 8)
    new_lens, kv_lens = [], []
    for _ in range(b):
        r = rng.random()
        n = 0 if r < 0.1 else 1 if r < 0.3 else rng.randint(2, 12) if r < 0.5 else rng.randint(13, 300)
        prefix = rng.choice([0, 0, rng.randint(1, 64), rng.randint(65, 1200)])
        new_lens.append(n)
        kv_lens.append(prefix + n)
    if sum(new_lens) == 0:
        new_lens[0] = kv_lens[0] = kv_lens[0] + 5
    log(f"prefill sweep seed={seed}: hq={hq} hkv={hkv} d={d} ps={ps} {kind} causal={causal} "
        f"new={new_lens} kv={kv_lens}")
    out, ref = _run_prefill(gpu, hq, hkv, d, ps, kv_lens, new_lens, causal, seed, fp8=kind == "fp8",
                            dtype=DTYPES[kind])
    err = max_abs(out, ref)
    log(f"  max_abs={err:.3e}")
    assert err < TOLS[kind]
