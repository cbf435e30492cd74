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

import torch


def range_push(name: str) -> None:
    torch.cuda.nvtx.range_push(name)


def range_pop() -> None:
    torch.cuda.nvtx.range_pop()


class _Range:
    """``range_push(name)`` on entry, ``range_pop()`` on exit."""

    __slots__ = ("name",)

    def __init__(self, name: str):
        self.name = name

    def __enter__(self) -> None:
        range_push(self.name)

    def __exit__(self, *exc) -> bool:
        range_pop()
        return False


class _NoRange:
    """The disabled range: nothing on entry or exit (one shared instance, so a
    disabled range costs a call and two no-op methods per phase)."""

    __slots__ = ()

    def __enter__(self) -> None:
        return None

    def __exit__(self, *exc) -> bool:
        return False


_NO_RANGE = _NoRange()


def trace_range(enabled: bool, name: str):
    """Context manager: ``range_push(name)`` ... ``range_pop()`` around the block when ``enabled``."""
    return _Range(name) if enabled else _NO_RANGE
