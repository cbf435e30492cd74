"""Tracing ranges around the phases of planning and running, for profilers.

The reference brackets its planning and decode phases with NVTX ranges when
``enable_nvtx`` is set (``mstar/utils/profiler.py``; range names in
``mstar/engine/cache_manager.py:192-227, 269-325, 397-418, 443-512`` and
``mstar/utils/flashinfer_utils.py:387-449``).  On ROCm, ``torch.cuda.nvtx``
is backed by roctx, so the same calls give ranges that ``rocprofv3
--marker-trace`` records beside the kernels.  The names are the reference's,
so a trace from either build reads the same; a phase that this build does not
have (the reference's host-side list building, say) is pushed around the step
that replaces it.

Ranges are host-side markers only: no device synchronisation.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Iterator

import torch


def range_push(name: str) -> None:
    torch.cuda.nvtx.range_push(name)


def range_pop() -> None:
    torch.cuda.nvtx.range_pop()


@contextmanager
def trace_range(enabled: bool, name: str) -> Iterator[None]:
    """``range_push(name)`` ... ``range_pop()`` around the block when ``enabled``."""
    if not enabled:
        yield
        return
    range_push(name)
    try:
        yield
    finally:
        range_pop()
