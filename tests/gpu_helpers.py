"""Shared builders for the GPU parity tests (seeded, CPU-generated inputs)."""

from __future__ import annotations

import sys

import numpy as np
import torch

from mstar_amd import synthetic as S
from oracle import attention as A
from oracle import packing as P
from oracle import rope as R


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


# RoPE tolerance: output rounding of both sides plus one fp32 ulp of the
# frequency at the token's position (pos * f * 2^-23 rad, doubled for margin)
# times the pair magnitude.
ROPE_REL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10}


def rope_bound(x, ref, pos, rd, interleave, scale, theta, llama31):
    """Per-element tolerance (see module docstring)."""
    half = rd // 2
    f = R.frequencies(rd, scale, theta, llama31).double()
    ang_err = torch.as_tensor(np.asarray(pos, dtype=np.float64))[:, None] * f[None, :] * 2.0 ** -21  # [T, half]
    xf = x.double()
    if interleave:
        mag = torch.sqrt(xf[..., 0:rd:2] ** 2 + xf[..., 1:rd:2] ** 2)
    else:
        mag = torch.sqrt(xf[..., :half] ** 2 + xf[..., half:rd] ** 2)
    pair = mag * ang_err[:, None, :]
    b = ROPE_REL[x.dtype] * ref.double().abs() + 1e-6
    if interleave:
        b[..., 0:rd:2] += pair
        b[..., 1:rd:2] += pair
    else:
        b[..., :half] += pair
        b[..., half:rd] += pair
    return b


__all__ = ["S", "A", "P", "log", "random_cache", "custom_batch", "workspace", "max_abs", "decode_reference", "rope_bound"]
