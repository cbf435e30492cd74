"""Shared builders for the GPU parity tests (seeded, CPU-generated inputs)."""

from __future__ import annotations

import sys

import numpy as np
import torch

from mstar_amd import synthetic as S
from oracle import attention as A
from oracle import packing as P


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def random_cache(pool: int, ps: int, hkv: int, d: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(pool, 2, ps, hkv, d, generator=g).to(dtype)


def custom_batch(kv_lens, ps: int, pool: int, seed: int, new_lens=None):
    """Metadata for explicit lengths with pages drawn from randperm(pool)."""
    kv_lens = np.asarray(kv_lens, dtype=np.int64)
    b = len(kv_lens)
    new_lens = np.ones(b, dtype=np.int64) if new_lens is None else np.asarray(new_lens, dtype=np.int64)
    g = torch.Generator().manual_seed(seed)
    npages = (kv_lens + ps - 1) // ps
    perm = torch.randperm(pool, generator=g).numpy().astype(np.int32)
    kv_indptr = np.zeros(b + 1, dtype=np.int32)
    kv_indptr[1:] = np.cumsum(npages)
    qo = np.zeros(b + 1, dtype=np.int32)
    qo[1:] = np.cumsum(new_lens)
    last = np.where(npages > 0, kv_lens - (npages - 1) * ps, ps).astype(np.int32)
    return qo, kv_indptr, perm[: kv_indptr[-1]].copy(), last


def workspace(device, nbytes: int = 256 << 20) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def decode_reference(q, cache_cpu, kv_indptr, kv_indices, last, k_scale=None, v_scale=None):
    return A.paged_attention(q.cpu(), cache_cpu, None, kv_indptr, kv_indices, last, causal=False,
                             k_scale=k_scale, v_scale=v_scale)


__all__ = ["S", "A", "P", "log", "random_cache", "custom_batch", "workspace", "max_abs", "decode_reference"]
