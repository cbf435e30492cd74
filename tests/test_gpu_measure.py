"""GPU: the HBM read probe behind the benchmark's read ceiling reads every
16-byte piece of its buffer exactly once (the XOR of its sink words is the XOR
of the buffer's words, which a skipped or doubled piece would change)."""

import numpy as np
import pytest
import torch

from gpu_helpers import log
from mstar_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096, 3), (1 << 20, 7), ((1 << 24) + 48, 64), (3 << 20, 2048)])
def test_hbm_read_covers_buffer_once(gpu, nbytes, grid):
    g = torch.Generator().manual_seed(nbytes % 1000 + grid)
    host = torch.randint(-(1 << 31), 1 << 31, (nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)
    buf = host.to(gpu)
    sink = torch.full((4 * grid,), -1, dtype=torch.int32, device=gpu)
    _lib.check(_lib.lib().mi_hbm_read(buf.data_ptr(), nbytes, sink.data_ptr(), grid, _lib.stream_ptr(gpu)),
               "mi_hbm_read")
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    log(f"hbm_read bytes={nbytes} grid={grid} xor={got:#x}")
    assert got == want


def test_hbm_read_rejects_bad_arguments(gpu):
    buf = torch.zeros(64, dtype=torch.int32, device=gpu)
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    s = _lib.stream_ptr(gpu)
    assert _lib.lib().mi_hbm_read(buf.data_ptr(), 20, sink.data_ptr(), 1, s) == -1  # not a multiple of 16
    assert _lib.lib().mi_hbm_read(buf.data_ptr() + 4, 16, sink.data_ptr(), 1, s) == -1  # misaligned
    assert _lib.lib().mi_hbm_read(buf.data_ptr(), 16, sink.data_ptr(), 0, s) == -1
