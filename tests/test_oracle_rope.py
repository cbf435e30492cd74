"""Pin the RoPE oracle (oracle/rope.py) against independent derivations.

* rotation as complex multiplication in float64 (pair i of token t times
  exp(1j * pos_t * f_i));
* position 0 is the identity, pair norms are kept, and scores depend only on
  the position difference (the property RoPE exists for);
* interleaved pairs are the half-split pairs under a fixed permutation;
* dims past rotary_dim are untouched;
* the Llama-3.1 frequencies against the published piecewise rule written
  with explicit wavelength branches;
* positions against a hand-computed list (cache_manager.py:480-492).
"""

import math

import numpy as np
import pytest
import torch

from oracle import rope as R


def test_positions_known_answer():
    assert R.positions([3, 0, 1], [5, 9, 0]).tolist() == [5, 6, 7, 0]
    assert R.positions([], []).tolist() == []


@pytest.mark.parametrize("d,rd", [(64, 64), (128, 128), (128, 64), (256, 256)])
def test_half_split_is_complex_rotation(d, rd):
    g = torch.Generator().manual_seed(d + rd)
    x = torch.randn(5, 3, d, generator=g)
    pos = np.array([0, 1, 17, 4096, 32767])
    out = R.rope(x, pos, rotary_dim=rd, rope_theta=10000.0).double()
    half = rd // 2
    # the fp32 frequencies are pinned separately (test_frequencies_match_float64);
    # here the angle is the same fp32 product pos * f, and the rotation is checked
    f = R.frequencies(rd, 1.0, 10000.0).numpy()
    z = x[..., :half].double().numpy() + 1j * x[..., half:rd].double().numpy()
    ang = (pos.astype(np.float32)[:, None] * f[None, :]).astype(np.float64)
    zr = z * np.exp(1j * ang)[:, None, :]
    np.testing.assert_allclose(out[..., :half].numpy(), zr.real, atol=2e-5)
    np.testing.assert_allclose(out[..., half:rd].numpy(), zr.imag, atol=2e-5)
    np.testing.assert_array_equal(out[..., rd:].numpy(), x[..., rd:].double().numpy())


@pytest.mark.parametrize("rd,theta", [(64, 10000.0), (128, 1000000.0), (256, 10000.0)])
def test_frequencies_match_float64(rd, theta):
    f = R.frequencies(rd, 1.0, theta).double().numpy()
    ref = theta ** (-np.arange(rd // 2) * 2.0 / rd)
    np.testing.assert_allclose(f, ref, rtol=3e-7)


def test_identity_at_zero_and_norms_kept():
    x = torch.randn(4, 2, 128, generator=torch.Generator().manual_seed(1))
    np.testing.assert_allclose(R.rope(x, [0, 0, 0, 0]).numpy(), x.numpy(), atol=0)
    y = R.rope(x, [1, 100, 1000, 30000])
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n1.numpy(), n0.numpy(), rtol=1e-5, atol=1e-5)


def test_scores_depend_on_position_difference():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 1, 128, generator=g)
    k = torch.randn(1, 1, 128, generator=g)
    ref = (R.rope(q, [37]) * R.rope(k, [0])).sum().item()
    for p in (50, 300, 1000):
        s = (R.rope(q, [p + 37]) * R.rope(k, [p])).sum().item()
        assert abs(s - ref) < 1e-3 * max(1.0, abs(ref))


def test_interleave_is_permuted_half_split():
    d = 64
    x = torch.randn(3, 2, d, generator=torch.Generator().manual_seed(3))
    perm = torch.cat([torch.arange(0, d, 2), torch.arange(1, d, 2)])  # interleaved -> half split
    pos = [0, 5, 999]
    a = R.rope(x, pos, interleave=True)
    b = R.rope(x[..., perm], pos, interleave=False)
    np.testing.assert_allclose(a[..., perm].numpy(), b.numpy(), atol=1e-6)


def test_rope_scale_divides_frequency():
    x = torch.randn(2, 1, 64, generator=torch.Generator().manual_seed(4))
    a = R.rope(x, [40, 400], rope_scale=4.0)
    b = R.rope(x, [10, 100])
    np.testing.assert_allclose(a.numpy(), b.numpy(), atol=1e-4)


def _llama31_reference(rd, theta, factor, lo, hi, old):
    """Llama 3.1 rope scaling, written with explicit wavelength branches."""
    out = []
    for i in range(rd // 2):
        g = 1.0 / theta ** (2.0 * i / rd)
        wavelen = 2 * math.pi / g
        if wavelen < old / hi:
            out.append(g)
        elif wavelen > old / lo:
            out.append(g / factor)
        else:
            smooth = (old / wavelen - lo) / (hi - lo)
            out.append((1 - smooth) * g / factor + smooth * g)
    return np.array(out)


@pytest.mark.parametrize("rd,theta", [(128, 500000.0), (64, 10000.0)])
def test_llama31_frequencies(rd, theta):
    p = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)
    f = R.frequencies(rd, 8.0, theta, p).double().numpy()
    ref = _llama31_reference(rd, theta, 8.0, 1.0, 4.0, 8192.0)
    np.testing.assert_allclose(f, ref, rtol=2e-6)
    # both regimes occur for these parameters
    g = 1.0 / theta ** (np.arange(rd // 2) * 2.0 / rd)
    assert np.isclose(f[0], g[0], rtol=1e-6) and np.isclose(f[-1], g[-1] / 8.0, rtol=1e-6)
