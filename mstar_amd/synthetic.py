"""Seeded synthetic ragged batches for the benchmark configurations.

Each configuration draws request lengths and page assignments from a CPU
``torch.Generator`` (so CPU and GPU runs see identical metadata):

* ``c1`` — seed 0, B=8, T~U{16..512}, 8 q / 2 kv heads, pool of 512 pages.
* ``c2`` — seed 1, B=64, T log-uniform [128, 4096], 24 q / 8 kv heads, 32768 pages.
* ``c3`` — seed 2, B=256, T log-uniform [512, 32768], 32 q / 4 kv heads, 262144 pages.
* ``c4`` — seed 3, 28 q / 4 kv heads, causal: 8 prefill chunks of U{512..2048}
  new tokens over prefixes U{0..8192} plus 120 decode requests, T log-uniform
  [1024, 16384], packed in one ragged batch.
* ``c5`` — seed 4, as c3 with T log-uniform [1024, 32768] and an fp8-e4m3 cache.

All use head_dim 128 and page_size 16.  Every request's page list is a
consecutive slice of one ``randperm(pool)``, in request order.  T is the
length after this step's append; decode requests append one token.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class Spec:
    name: str
    seed: int
    batch: int
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    pool_pages: int
    ctx: tuple  # ("uniform"|"loguniform", lo, hi)
    kv_dtype: str = "bf16"
    prefill_chunks: int = 0  # c4: leading requests that are prefill chunks


SPECS = {
    "c1": Spec("c1", 0, 8, 8, 2, 128, 16, 512, ("uniform", 16, 512)),
    "c2": Spec("c2", 1, 64, 24, 8, 128, 16, 32768, ("loguniform", 128, 4096)),
    "c3": Spec("c3", 2, 256, 32, 4, 128, 16, 262144, ("loguniform", 512, 32768)),
    "c4": Spec("c4", 3, 128, 28, 4, 128, 16, 65536, ("loguniform", 1024, 16384), prefill_chunks=8),
    "c5": Spec("c5", 4, 256, 32, 4, 128, 16, 262144, ("loguniform", 1024, 32768), kv_dtype="fp8"),
}


@dataclass
class Batch:
    spec: Spec
    kv_len: np.ndarray        # int64 [B], tokens after the append
    new_len: np.ndarray       # int64 [B], tokens appended this step (qo_len)
    qo_indptr: np.ndarray     # int32 [B+1]
    kv_indptr: np.ndarray     # int32 [B+1]
    kv_indices: np.ndarray    # int32 [sum pages]
    last_page_len: np.ndarray  # int32 [B]
    generator: torch.Generator

    @property
    def total_pages(self) -> int:
        return int(self.kv_indptr[-1])

    @property
    def total_kv_tokens(self) -> int:
        return int(self.kv_len.sum())

    @property
    def total_q_tokens(self) -> int:
        return int(self.qo_indptr[-1])


def _draw_lengths(g: torch.Generator, n: int, kind: str, lo: int, hi: int) -> np.ndarray:
    if kind == "uniform":
        return torch.randint(lo, hi + 1, (n,), generator=g).numpy().astype(np.int64)
    u = torch.rand(n, generator=g, dtype=torch.float64).numpy()
    t = np.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
    return np.clip(np.rint(t), lo, hi).astype(np.int64)


def make_batch(name_or_spec, batch: int | None = None) -> Batch:
    """Draw the metadata of one step of configuration ``name_or_spec``.

    ``batch`` truncates the batch to its first requests (same draws).
    """
    spec = SPECS[name_or_spec] if isinstance(name_or_spec, str) else name_or_spec
    g = torch.Generator().manual_seed(spec.seed)
    b = spec.batch
    if spec.prefill_chunks:
        npf = spec.prefill_chunks
        new_pf = torch.randint(512, 2049, (npf,), generator=g).numpy().astype(np.int64)
        prefix = torch.randint(0, 8193, (npf,), generator=g).numpy().astype(np.int64)
        dec = _draw_lengths(g, b - npf, *spec.ctx)
        kv_len = np.concatenate([prefix + new_pf, dec])
        new_len = np.concatenate([new_pf, np.ones(b - npf, dtype=np.int64)])
    else:
        kv_len = _draw_lengths(g, b, *spec.ctx)
        new_len = np.ones(b, dtype=np.int64)
    ps = spec.page_size
    npages = (kv_len + ps - 1) // ps
    if int(npages.sum()) > spec.pool_pages:
        raise ValueError(f"{spec.name}: {int(npages.sum())} pages needed, pool holds {spec.pool_pages}")
    perm = torch.randperm(spec.pool_pages, generator=g).numpy().astype(np.int32)
    kv_indptr = np.zeros(b + 1, dtype=np.int32)
    kv_indptr[1:] = np.cumsum(npages)
    kv_indices = perm[: kv_indptr[-1]].copy()
    qo_indptr = np.zeros(b + 1, dtype=np.int32)
    qo_indptr[1:] = np.cumsum(new_len)
    last = (kv_len - (npages - 1) * ps).astype(np.int32)
    bt = Batch(spec, kv_len, new_len, qo_indptr, kv_indptr, kv_indices, last, g)
    if batch is not None and batch < b:
        bt = truncate(bt, batch)
    return bt


def truncate(bt: Batch, n: int) -> Batch:
    """The first ``n`` requests of ``bt`` (same pages)."""
    kv_indptr = bt.kv_indptr[: n + 1].copy()
    qo_indptr = bt.qo_indptr[: n + 1].copy()
    return Batch(bt.spec, bt.kv_len[:n].copy(), bt.new_len[:n].copy(), qo_indptr, kv_indptr,
                 bt.kv_indices[: kv_indptr[-1]].copy(), bt.last_page_len[:n].copy(), bt.generator)


def algorithmic_decode_bytes(bt: Batch, kv_elem_bytes: int = 2, q_elem_bytes: int = 2) -> int:
    """HBM bytes one decode step must move: KV read + q read + o write + new K/V
    read+write + index arrays (split-KV partials excluded)."""
    s = bt.spec
    b = len(bt.kv_len)
    kv = bt.total_kv_tokens * s.num_kv_heads * s.head_dim * 2 * kv_elem_bytes
    qo = b * s.num_qo_heads * s.head_dim * q_elem_bytes * 2
    new = b * s.num_kv_heads * s.head_dim * 2 * (q_elem_bytes + kv_elem_bytes)
    idx = 4 * (bt.total_pages + 3 * b)
    return kv + qo + new + idx
