"""CPU checks of the test helper that classifies MX writeback differences (helpers.
mx_boundary_sites): every encoding of a state perturbed elementwise by at most eps * mag differs
from the encoding of the unperturbed state only at flagged sites, in every rounding mode; and
constructed threshold cases are flagged while states far from every threshold are not."""
import numpy as np
import pytest
import torch

from helpers import mx_boundary_sites
from oracle import mx_state as omx


def _state(seed, shape=(4, 8, 128)):
    g = np.random.default_rng(seed)
    h = g.standard_normal(shape) * np.exp(g.standard_normal(shape[:-1] + (1,)))
    return h.astype(np.float32)


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_perturbed_encodings_differ_only_at_flagged_sites(fb, mode):
    eps = 2.0 ** -9  # large, so that many decisions sit inside the interval
    for seed in range(6):
        h = _state(seed)
        mag = np.abs(h) * (1.0 + np.random.default_rng(100 + seed).random(h.shape)) + 1e-3
        uni = torch.rand(h.shape, generator=torch.Generator().manual_seed(seed)) if mode == 2 else None
        kw = dict(uniform=uni, seed=7, rng_offset=16 * seed)
        values, pairs, blocks = mx_boundary_sites(h, mag, fb, mode, eps=eps, **kw)
        ref = omx.mx_encode(h, fb, mode, **kw)
        assert 0 < values.sum() < values.size
        for trial in range(8):
            t = np.random.default_rng(1000 * seed + trial).uniform(-1, 1, h.shape)
            pert = (h + t * eps * mag).astype(np.float32)
            q, e, m = omx.mx_encode(pert, fb, mode, **kw)
            assert not np.any((e != ref[1]) & ~blocks)
            assert not np.any((m != ref[2]) & ~pairs)
            assert not np.any((q != ref[0]) & ~values)


def test_constructed_thresholds_are_flagged():
    fb, m_max = 4, 7.0
    h = np.full((1, 1, 32), 0.01, dtype=np.float32)
    h[0, 0, 3] = np.float32(2 * m_max * 2.0 ** -3)      # block absmax / 14 exactly 2^-3
    h[0, 0, 16 + 5] = 1.0                                # second block: absmax 1 -> base 2^-3
    h[0, 0, 16 + 9] = np.float32(m_max * 2.0 ** -3)     # pair absmax exactly M * base
    h[0, 0, 16 + 12] = np.float32(2.5 * 2.0 ** -3)      # qa = 2.5: half-up tie
    mag = np.abs(h).astype(np.float64)
    values, pairs, blocks = mx_boundary_sites(h, mag, fb, omx.ROUND_HALF_UP)
    assert blocks[0, 0, 0] and not blocks[0, 0, 1]
    assert pairs[0, 0, 8 + 4] and values[0, 0, 16 + 12]
    assert not values[0, 0, 16 + 14]                     # 0.01 / 2^-3 = 0.08: far from 0.5


def test_far_from_thresholds_nothing_flagged():
    h = np.full((2, 2, 16), 0.3, dtype=np.float32)      # amax/14: 0.0214 (not near 2^k)
    h[..., ::2] = -0.3
    values, pairs, blocks = mx_boundary_sites(h, np.abs(h), 4, omx.ROUND_HALF_UP)
    assert not values.any() and not pairs.any() and not blocks.any()
