"""CPU fp32 paged attention, append and fp8 (de)quantisation.

Test infrastructure only (see ``oracle/__init__.py``).

Attention follows the FlashInfer semantics M* relies on, restated the way the
reference's tests compute their expected values: gather the request's pages,
expand KV heads with ``repeat_interleave`` (q head h reads kv head
h // (Hq/Hkv)), fp32 ``softmax(q k^T * sm_scale) v``
(``test/modular/test_pi05_reference_equivalence.py:158-185, 625-640``).
Defaults: sm_scale = 1/sqrt(head_dim) (the reference never passes one);
causal masks are aligned to the end of the KV: query j of a request with
qo_len queries and kv_len keys sees keys i <= kv_len - qo_len + j.
"""

from __future__ import annotations

import math

import numpy as np
import torch

FP8_MAX = 448.0


def gather_request_kv(kv_cache_layer: torch.Tensor, pages: np.ndarray, kv_len: int):
    """Contiguous K, V ``[kv_len, Hkv, D]`` of one request from its page list."""
    ps = kv_cache_layer.shape[2]
    idx = torch.as_tensor(np.asarray(pages, dtype=np.int64))
    kp = kv_cache_layer[idx, 0]  # [npages, ps, Hkv, D]
    vp = kv_cache_layer[idx, 1]
    k = kp.reshape(-1, *kp.shape[2:])[:kv_len]
    v = vp.reshape(-1, *vp.shape[2:])[:kv_len]
    assert k.shape[0] == kv_len or len(pages) * ps < kv_len
    return k, v


def dequant(x: torch.Tensor, scale: torch.Tensor | None) -> torch.Tensor:
    """fp32 value of a cache slice; fp8 entries times their per-head scale."""
    xf = x.float()
    if x.dtype == torch.float8_e4m3fn:
        xf = xf * scale.float().view(1, -1, 1)
    return xf


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, sm_scale: float):
    """fp32 GQA attention of ``q [qo, Hq, D]`` over ``k, v [kv, Hkv, D]``.

    Returns (out ``[qo, Hq, D]`` fp32, lse ``[qo, Hq]`` natural-log fp32).
    Rows with no visible key give zeros and lse = -inf.
    """
    qo, hq, _ = q.shape
    kv, hkv, _ = k.shape
    rep = hq // hkv
    kf = k.float().repeat_interleave(rep, dim=1)
    vf = v.float().repeat_interleave(rep, dim=1)
    s = torch.einsum("qhd,khd->hqk", q.float(), kf) * sm_scale
    if causal:
        j = torch.arange(qo).view(-1, 1)
        i = torch.arange(kv).view(1, -1)
        s = s.masked_fill((i > kv - qo + j).unsqueeze(0), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)  # [H, qo]
    p = torch.exp(s - torch.where(torch.isinf(lse), torch.zeros_like(lse), lse).unsqueeze(-1))
    p = torch.nan_to_num(p, nan=0.0)
    out = torch.einsum("hqk,khd->qhd", p, vf)
    return out, lse.transpose(0, 1)


def paged_attention(q: torch.Tensor, kv_cache_layer: torch.Tensor, qo_indptr, kv_indptr, kv_indices,
                    last_page_len, causal: bool = True, sm_scale: float | None = None,
                    k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Ragged paged attention over a CPU cache layer; fp32 output ``[tokens, Hq, D]``.

    ``qo_indptr=None`` means decode: one query row per request.
    """
    d = q.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    kv_indptr = np.asarray(kv_indptr, dtype=np.int64)
    kv_indices = np.asarray(kv_indices, dtype=np.int64)
    last_page_len = np.asarray(last_page_len, dtype=np.int64)
    b = len(last_page_len)
    if qo_indptr is None:
        qo_indptr = np.arange(b + 1)
    qo_indptr = np.asarray(qo_indptr, dtype=np.int64)
    ps = kv_cache_layer.shape[2]
    out = torch.zeros(q.shape[0], q.shape[1], d, dtype=torch.float32)
    for r in range(b):
        q0, q1 = int(qo_indptr[r]), int(qo_indptr[r + 1])
        if q1 == q0:
            continue
        pages = kv_indices[kv_indptr[r]:kv_indptr[r + 1]]
        kv_len = (len(pages) - 1) * ps + int(last_page_len[r]) if len(pages) else 0
        if kv_len <= 0:
            continue
        k, v = gather_request_kv(kv_cache_layer, pages, kv_len)
        k = dequant(k, k_scale)
        v = dequant(v, v_scale)
        o, _ = attend(q[q0:q1], k, v, causal, sm_scale)
        out[q0:q1] = o
    return out


def merge_states(outs: list[torch.Tensor], lses: list[torch.Tensor]) -> torch.Tensor:
    """Log-sum-exp merge of partial attention states (natural-log lse).

    lse = log sum_k exp(lse_k); o = sum_k exp(lse_k - lse) o_k; an empty part
    has lse = -inf and contributes nothing.
    """
    lse = torch.stack(lses)  # [K, ...]
    m = lse.max(dim=0).values
    m_safe = torch.where(torch.isinf(m), torch.zeros_like(m), m)
    w = torch.exp(lse - m_safe)
    w = torch.nan_to_num(w, nan=0.0)
    tot = w.sum(dim=0)
    o = sum(wk.unsqueeze(-1) * ok for wk, ok in zip(w, outs))
    return torch.where(tot.unsqueeze(-1) > 0, o / tot.clamp_min(1e-30).unsqueeze(-1), torch.zeros_like(o))


# ------------------------------------------------------------------ append
def append(kv_cache_layer: torch.Tensor, token_to_page, token_to_cache, k: torch.Tensor, v: torch.Tensor,
           k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
    """``cache[page, 0/1, slot] = k/v`` cast to the cache dtype, in place (``flashinfer_utils.py:284-288``)."""
    page = torch.as_tensor(np.asarray(token_to_page, dtype=np.int64))
    slot = torch.as_tensor(np.asarray(token_to_cache, dtype=np.int64))
    n = page.shape[0]
    if kv_cache_layer.dtype == torch.float8_e4m3fn:
        kv_cache_layer[page, 0, slot] = quantize_e4m3(k[:n], k_scale)
        kv_cache_layer[page, 1, slot] = quantize_e4m3(v[:n], v_scale)
    else:
        kv_cache_layer[page, 0, slot] = k[:n].to(kv_cache_layer.dtype)
        kv_cache_layer[page, 1, slot] = v[:n].to(kv_cache_layer.dtype)


def quantize_e4m3(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Per-kv-head fp8 e4m3fn quantisation of ``x [tokens, Hkv, D]``.

    q = e4m3fn_RNE(clamp(x_fp32 * (1/scale[h]), -448, 448)), ``1/scale`` in fp32.
    """
    inv = (1.0 / scale.float()).view(1, -1, 1)
    return (x.float() * inv).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


def head_scales(x: torch.Tensor) -> torch.Tensor:
    """Per-kv-head scale amax/448 of ``x [tokens, Hkv, D]`` (1.0 for an all-zero head)."""
    amax = x.float().abs().amax(dim=(0, 2))
    return torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))


# ----------------------------------------------------------- e4m3fn codec
def e4m3fn_values() -> np.ndarray:
    """fp64 value of each of the 256 e4m3fn codes, from the format definition.

    Sign bit 7, exponent bits 6-3 (bias 7), mantissa bits 2-0; exponent 0 is
    subnormal (m * 2^-9); 0x7F / 0xFF are NaN; no infinities.
    """
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * m * 2.0 ** -9
        else:
            vals[c] = s * (1 + m / 8) * 2.0 ** (e - 7)
    return vals
