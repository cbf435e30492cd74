"""CPU rotary position embedding and RoPE position ids.

Test infrastructure only (see ``oracle/__init__.py``).

``positions`` restates ``BatchedCacheManager._plan_rope_impl``
(``mstar/engine/cache_manager.py:480-492``): request r contributes positions
``position_id_start[r] .. position_id_start[r] + seq_len[r] - 1``, in batch
order.

``rope`` restates what ``BatchedCacheManager.apply_rope``
(``cache_manager.py:702-760``) asks of FlashInfer's
``apply_rope_pos_ids_inplace`` / ``apply_llama31_rope_pos_ids_inplace``,
computed like the reference's own check of that call
(``test/modular/test_pi05_reference_equivalence.py:559-589``, the HF
Gemma/Llama formula): in fp32, dims ``[0, rotary_dim)`` rotate in pairs,
either (i, i + rotary_dim/2) ("half split", ``interleave=False``) or
(2i, 2i+1) (``interleave=True``); pair i turns by the angle
``pos * f_i`` with ``f_i = theta^(-2i/rotary_dim) / rope_scale``; dims past
``rotary_dim`` are unchanged.  With Llama-3.1 parameters the frequency is
blended between ``f_i`` (scaled) and the unscaled ``theta^(-2i/rotary_dim)``
by ``smooth = clamp(old_context_len * g / (2 pi (high - low)) - low / (high - low), 0, 1)``
where g is the unscaled frequency: long wavelengths (smooth = 0) are
divided by ``rope_scale``, short ones (smooth = 1) are kept.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def positions(seq_lens, position_id_start) -> np.ndarray:
    """Per-new-token RoPE positions (int64), request by request."""
    out = [np.arange(s0, s0 + sl, dtype=np.int64) for s0, sl in zip(position_id_start, seq_lens)]
    return np.concatenate(out) if out else np.zeros(0, dtype=np.int64)


def frequencies(rotary_dim: int, rope_scale: float = 1.0, rope_theta: float = 1e4,
                llama31: dict | None = None) -> torch.Tensor:
    """fp32 angular frequency of each of the rotary_dim/2 pairs."""
    half = rotary_dim // 2
    g = 1.0 / (rope_theta ** (torch.arange(0, half, dtype=torch.float32) * 2.0 / rotary_dim))
    if not llama31:
        return g / rope_scale
    lo = float(llama31["low_freq_factor"])
    hi = float(llama31["high_freq_factor"])
    old = float(llama31["old_context_len"])
    smooth = (g * (old / (2 * math.pi * (hi - lo))) - lo / (hi - lo)).clamp(0.0, 1.0)
    return (1.0 - smooth) * (g / rope_scale) + smooth * g


def rope(x: torch.Tensor, pos_ids, rotary_dim: int | None = None, interleave: bool = False,
         rope_scale: float = 1.0, rope_theta: float = 1e4, llama31: dict | None = None) -> torch.Tensor:
    """Rotated copy (fp32) of ``x [tokens, heads, head_dim]``."""
    d = x.shape[-1]
    rd = d if rotary_dim is None else rotary_dim
    half = rd // 2
    f = frequencies(rd, rope_scale, rope_theta, llama31)
    ang = torch.as_tensor(np.asarray(pos_ids)).to(torch.float32)[:, None] * f[None, :]  # [T, half]
    c = torch.cos(ang)[:, None, :]
    s = torch.sin(ang)[:, None, :]
    xf = x.float()
    out = xf.clone()
    if interleave:
        a, b = xf[..., 0:rd:2], xf[..., 1:rd:2]
        out[..., 0:rd:2] = a * c - b * s
        out[..., 1:rd:2] = b * c + a * s
    else:
        a, b = xf[..., :half], xf[..., half:rd]
        out[..., :half] = a * c - b * s
        out[..., half:rd] = b * c + a * s
    return out
