"""Rotary position embedding on the packed batch (gfx950 kernels).

Mirrors the two ``flashinfer.rope`` calls M* makes from
``BatchedCacheManager.apply_rope`` (``mstar/engine/cache_manager.py:702-760``):
``apply_rope_pos_ids_inplace`` and ``apply_llama31_rope_pos_ids_inplace``, same
argument names and defaults.  q ``[tokens, Hq, D]`` and k ``[tokens, Hkv, D]``
(bf16 or fp16, last dim contiguous) are rotated in place by ``mi_rope_apply``;
there is no CPU fallback.  ``rope_append`` fuses the rotation with the paged
K/V append that follows it in ``run_attention`` (``mi_rope_append``).
"""

from __future__ import annotations

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.MI_BF16, torch.float16: _lib.MI_F16}
_POS = {torch.int32: _lib.MI_I32, torch.int64: _lib.MI_I64}


def _check(x: torch.Tensor, name: str) -> None:
    if x.dim() != 3:
        raise ValueError(f"{name} must be [tokens, heads, head_dim], got {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise ValueError(f"{name}: RoPE runs on bf16 or fp16 tensors, got {x.dtype}")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")
    if x.stride(2) != 1:
        raise ValueError(f"{name}: head_dim must be contiguous")


def _apply(q, k, pos_ids, rotary_dim, interleave, rope_scale, rope_theta, llama31, low, high, old) -> None:
    _check(q, "q")
    _check(k, "k")
    if q.dtype != k.dtype or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2] or q.device != k.device:
        raise ValueError("q and k must agree on dtype, device, token count and head_dim")
    d = q.shape[2]
    rd = d if rotary_dim is None else int(rotary_dim)
    if rd <= 0 or rd > d or rd % 8 or d % 8:
        raise ValueError(f"rotary_dim {rd} and head_dim {d} must be multiples of 8 with rotary_dim <= head_dim")
    if pos_ids.dtype not in _POS or pos_ids.dim() != 1 or pos_ids.shape[0] < q.shape[0]:
        raise ValueError("pos_ids must be an int32/int64 vector with one position per token")
    pos_ids = pos_ids.to(q.device).contiguous()
    _lib.check(
        _lib.lib().mi_rope_apply(
            q.data_ptr(), q.stride(0), q.stride(1), q.shape[1], k.data_ptr(), k.stride(0), k.stride(1), k.shape[1],
            _DTYPES[q.dtype], d, rd, pos_ids.data_ptr(), _POS[pos_ids.dtype], q.shape[0], 1 if interleave else 0,
            float(rope_scale), float(rope_theta), 1 if llama31 else 0, float(low), float(high), float(old),
            _lib.stream_ptr(q.device),
        ),
        "mi_rope_apply",
    )


def apply_rope_pos_ids_inplace(q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                               rotary_dim: int | None = None, interleave: bool = False,
                               rope_scale: float = 1, rope_theta: float = 1e4) -> None:
    """Rotate q and k in place at the given positions (flashinfer.rope semantics)."""
    _apply(q, k, pos_ids, rotary_dim, interleave, rope_scale, rope_theta, False, 1.0, 4.0, 8192.0)


def apply_llama31_rope_pos_ids_inplace(q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                                       rotary_dim: int | None = None, interleave: bool = False,
                                       rope_scale: float = 8, rope_theta: float = 5e5,
                                       low_freq_factor: float = 1, high_freq_factor: float = 4,
                                       old_context_len: int = 8192) -> None:
    """Llama-3.1 frequency-smoothed RoPE in place (flashinfer.rope semantics)."""
    _apply(q, k, pos_ids, rotary_dim, interleave, rope_scale, rope_theta, True, low_freq_factor,
           high_freq_factor, old_context_len)


def rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_cache_layer: torch.Tensor,
                pos_ids: torch.Tensor, page_idx: torch.Tensor, slot_idx_ptr: int, idx_stride: int,
                num_append: int, num_append_device_ptr: int | None, *, rotary_dim: int | None = None,
                interleave: bool = False, rope_scale: float = 1, rope_theta: float = 1e4,
                k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None, keep_k: bool = True,
                llama31: dict | None = None) -> None:
    """Rotate q (and k) in place and write the rotated k and v to the paged cache, in one launch.

    The result equals ``apply_rope_pos_ids_inplace`` (or the Llama-3.1 variant
    when ``llama31`` holds its factors) followed by the wrapper's
    ``set_kv_cache`` on the same page map: token ``t < num_append`` (and below
    the device count at ``num_append_device_ptr`` when given) goes to page
    ``page_idx[t * idx_stride]``, slot ``slot_idx[t * idx_stride]``.  With
    ``keep_k=False`` the rotated k only reaches the cache and ``k`` keeps its
    input values.
    """
    _check(q, "q")
    _check(k, "k")
    _check(v, "v")
    if q.dtype != k.dtype or v.dtype != k.dtype:
        raise ValueError("q, k and v must share one dtype")
    if q.shape[0] != k.shape[0] or v.shape != k.shape or q.shape[2] != k.shape[2]:
        raise ValueError(f"shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not agree")
    desc = _lib.paged_kv_desc(kv_cache_layer, k_scale, v_scale)
    if k.shape[1:] != (desc.num_kv_heads, desc.head_dim):
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match the cache heads/head_dim")
    if num_append > k.shape[0]:
        raise ValueError(f"k/v hold {k.shape[0]} tokens, {num_append} planned")
    for name, x in (("k", k), ("v", v)):
        if x.stride(0) % 8 or x.stride(1) % 8 or x.data_ptr() % 16:
            raise ValueError(f"{name}: rows must be 16-byte aligned")
    d = q.shape[2]
    rd = d if rotary_dim is None else int(rotary_dim)
    if rd <= 0 or rd > d or rd % 8 or d % 8:
        raise ValueError(f"rotary_dim {rd} and head_dim {d} must be multiples of 8 with rotary_dim <= head_dim")
    if pos_ids.dtype not in _POS or pos_ids.dim() != 1 or pos_ids.shape[0] < q.shape[0]:
        raise ValueError("pos_ids must be an int32/int64 vector with one position per token")
    pos_ids = pos_ids.to(q.device).contiguous()
    l31 = llama31 or {}
    _lib.check(
        _lib.lib().mi_rope_append(
            q.data_ptr(), q.stride(0), q.stride(1), q.shape[1], k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), _DTYPES[q.dtype], 1 if keep_k else 0, desc,
            page_idx.data_ptr(), slot_idx_ptr, idx_stride, num_append, num_append_device_ptr, rd,
            pos_ids.data_ptr(), _POS[pos_ids.dtype], q.shape[0], 1 if interleave else 0, float(rope_scale),
            float(rope_theta), 1 if llama31 else 0, float(l31.get("low_freq_factor", 1.0)),
            float(l31.get("high_freq_factor", 4.0)), float(l31.get("old_context_len", 8192.0)),
            _lib.stream_ptr(q.device),
        ),
        "mi_rope_append",
    )


def rope_positions(qo_indptr: torch.Tensor, position_id_start: torch.Tensor, out: torch.Tensor,
                   num_tokens: int) -> torch.Tensor:
    """``out[t] = position_id_start[r] + t - qo_indptr[r]`` for t < num_tokens (int64, on the GPU)."""
    batch = position_id_start.shape[0]
    if qo_indptr.dtype != torch.int32 or position_id_start.dtype != torch.int32 or out.dtype != torch.int64:
        raise ValueError("qo_indptr/position_id_start must be int32 and out int64")
    if out.shape[0] < num_tokens or qo_indptr.shape[0] != batch + 1:
        raise ValueError("rope_positions: inconsistent sizes")
    _lib.check(
        _lib.lib().mi_rope_positions(qo_indptr.data_ptr(), position_id_start.data_ptr(), batch, out.data_ptr(),
                                     num_tokens, _lib.stream_ptr(out.device)),
        "mi_rope_positions",
    )
    return out
