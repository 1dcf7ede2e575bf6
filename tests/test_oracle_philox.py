"""Pins oracle/philox.py, the restatement of Triton's tl.rand stream that the reference's
stochastic writeback draws (hybrid_quant/mamba_state_8b_kernel.py:198, 405, 479, 529): Philox4x32-10
against the Random123 known-answer vectors, tl.randint / tl.rand against Triton's own outputs
(tests/golden/philox_tl_rand.json), the scalar restatement against the vectorized one, the
float conversion's end points, and the MX encoder's ROUND_SR_PHILOX offsets against a per-element
loop."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import mx_state as mx
from oracle import philox

GOLDEN = Path(__file__).parent / "golden"

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key, output)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox4x32_known_answers(ctr, key, want):
    assert philox.philox4x32_scalar(ctr, key) == want
    got = philox.philox4x32(*[np.array([c], dtype=np.uint32) for c in ctr], *key)
    assert tuple(int(g[0]) for g in got) == want


def test_tl_rand_matches_triton_outputs():
    """Triton's own tl.randint / tl.rand bits (its CPU interpreter), int32 and int64 offsets,
    seeds 0, 1234, 2^32 - 1, 2^32 + 7 and 2^62 + 12345, offsets up to 2^62 + 10."""
    data = json.loads((GOLDEN / "philox_tl_rand.json").read_text())
    assert len(data["cases"]) >= 40
    forms = set()
    for case in data["cases"]:
        offs = np.array(case["offsets"], dtype=np.uint64)
        assert philox.randint(case["seed"], offs).tolist() == case["bits"], case
        u = philox.rand(case["seed"], offs)
        assert u.view(np.uint32).tolist() == case["uniform_f32_bits"], case
        forms.add(case["form"])
    assert forms == {"constexpr", "int64"}


def test_scalar_restatement_matches_vectorized():
    gen = np.random.default_rng(7)
    offs = np.concatenate([gen.integers(0, 2**63, 200, dtype=np.uint64),
                           np.arange(2**32 - 5, 2**32 + 5, dtype=np.uint64)])
    for seed in (1234, 2**40 + 3):
        bits = philox.randint(seed, offs)
        u = philox.rand(seed, offs)
        for o, b, uu in zip(offs.tolist(), bits.tolist(), u.tolist()):
            c = philox.philox4x32_scalar((o & 0xFFFFFFFF, o >> 32, 0, 0),
                                         (seed & 0xFFFFFFFF, seed >> 32))
            assert c[0] == b
            assert philox.to_uniform_scalar(b) == uu


def test_uniform_conversion_end_points():
    bits = np.array([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, 0xFFFFFFFE], dtype=np.uint32)
    u = philox.to_uniform(bits)
    # 0 and -1 both map to 0; INT_MAX and INT_MIN to fp32(2^31) * scale = 1 - 2^-24
    assert u.tolist() == [0.0, float(np.float32(philox.SCALE)), 1.0 - 2.0**-24, 1.0 - 2.0**-24,
                          0.0, float(np.float32(philox.SCALE))]
    assert float(philox.SCALE).hex() == "0x1.fffffe0000000p-32"
    assert (u < 1.0).all()


def test_uniforms_are_uniform():
    u = philox.rand(1234, np.arange(1 << 16, dtype=np.uint64))
    hist = np.histogram(u, bins=16, range=(0.0, 1.0))[0]
    expected = (1 << 16) / 16
    chi2 = (((hist - expected) ** 2) / expected).sum()
    assert chi2 < 40.0  # 15 degrees of freedom: p ~ 5e-4 at 40


@pytest.mark.parametrize("fb", [8, 4])
def test_encode_philox_offsets_per_element(fb):
    """ROUND_SR_PHILOX equals ROUND_SR_UNIFORM fed with tl.rand(seed, rng_offset + flat index),
    the flat index of element (b, h, p, n) built here by an explicit loop."""
    gen = np.random.default_rng(fb)
    shape = (2, 3, 4, 32)
    v = (gen.standard_normal(shape) * 3).astype(np.float32)
    seed, off = 1234, (1 << 32) - 100
    u = np.empty(shape, dtype=np.float32)
    for b in range(shape[0]):
        for h in range(shape[1]):
            for p in range(shape[2]):
                for n in range(shape[3]):
                    idx = ((b * shape[1] + h) * shape[2] + p) * shape[3] + n
                    u[b, h, p, n] = philox.rand(seed, [off + idx])[0]
    got = mx.mx_encode(v, fb, mx.ROUND_SR_PHILOX, seed=seed, rng_offset=off)
    want = mx.mx_encode(v, fb, mx.ROUND_SR_UNIFORM, uniform=u)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    # the draws change the levels (not a deterministic mode in disguise)
    half_up = mx.mx_encode(v, fb, mx.ROUND_HALF_UP)
    assert not np.array_equal(got[0], half_up[0])
