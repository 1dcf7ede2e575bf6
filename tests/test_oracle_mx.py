"""Pins the CPU oracle of the MX state path (oracle/mx_state.py, oracle/rng.py): the exact
ceil(log2) rule against 60-digit arithmetic, encoder invariants and special cases, the update's
closed forms against an independent float64 evaluation, and the counter generator against a
scalar implementation and committed known-answer vectors."""
import json
import math
from fractions import Fraction
from pathlib import Path

import mpmath
import numpy as np
import pytest
import torch

from oracle import mx_state as mx
from oracle import rng

GOLDEN = Path(__file__).parent / "golden"


def _f32_round(x: mpmath.mpf) -> mpmath.mpf:
    m, e = mpmath.frexp(x)
    return mpmath.nint(m * mpmath.mpf(2) ** 24) * mpmath.mpf(2) ** (e - 24)


def test_ceil_log2_threshold_table_against_mpmath():
    mpmath.mp.dps = 60
    ts, want = [], []
    for e in range(-126, 128):
        for j in list(range(0, 96)) + [2**22, 2**23 - 2, 2**23 - 1]:
            ts.append(np.ldexp(np.float64(1 + j * 2.0 ** -23), e))
            exact = mpmath.mpf(e) + mpmath.log(1 + mpmath.mpf(j) * mpmath.mpf(2) ** -23, 2)
            want.append(int(mpmath.ceil(_f32_round(exact))))
    got = mx.ceil_log2_f32(np.array(ts, dtype=np.float32))
    assert np.array_equal(got, np.array(want))


def test_ceil_log2_matches_exact_ceiling_outside_rounding_band():
    gen = np.random.default_rng(0)
    t = (gen.random(20000) * 2 + 0.01).astype(np.float32) * np.float32(2.0) ** gen.integers(
        -100, 100, 20000).astype(np.float32)
    got = mx.ceil_log2_f32(t)
    for ti, gi in zip(t[:2000], got[:2000]):
        fr = Fraction(float(ti))
        k = int(np.floor(np.log2(float(ti))))
        while Fraction(2) ** k < fr:
            k += 1
        while Fraction(2) ** (k - 1) >= fr:
            k -= 1
        near = abs(float(fr / Fraction(2) ** (k - 1)) - 1.0) < 2.0 ** -16
        if not near:
            assert gi == k, (ti, gi, k)


def test_ceil_log2_agrees_with_torch_log2_at_boundaries():
    vals = [np.ldexp(np.float64(1 + j * 2.0 ** -23), e) for e in range(-126, 128)
            for j in list(range(0, 64)) + list(range(2**23 - 32, 2**23))]
    v = np.array(vals, dtype=np.float32)
    torch_ceil = torch.ceil(torch.log2(torch.from_numpy(v))).numpy().astype(np.int64)
    assert np.array_equal(torch_ceil, mx.ceil_log2_f32(v))


@pytest.mark.parametrize("fb", [8, 4])
def test_encode_invariants_and_error_bound(fb):
    gen = torch.Generator().manual_seed(10 + fb)
    v = torch.randn(64, 128, generator=gen) * torch.exp(torch.randn(64, 1, generator=gen) * 3)
    v[3, :16] = 0.0
    q, e, m = mx.mx_encode(v.numpy(), fb)
    M = mx.MANTISSA_MAX[fb]
    assert np.abs(q.astype(int)).max() <= M
    assert e.min() >= 1 and e.max() <= 254
    assert set(np.unique(m)) <= {0, 1}
    assert np.all(e[3, 0] == 28) and np.all(q[3, :16] == 0)
    deq = mx.mx_decode(q, e, m)
    ps = mx.exp2_scale(np.repeat(e.astype(np.uint32), 16, -1) + np.repeat(m.astype(np.uint32), 2, -1))
    err = np.abs(deq - v.numpy())
    assert np.all(err <= 0.5 * ps * (1 + 1e-6))


def test_encode_power_of_two_and_half_up_double_rounding():
    # absmax 126 * 2^-7 -> amax/126 = 2^-7 exactly -> e = 120; base = 2^-7
    v = np.zeros((1, 16), np.float32)
    v[0, 0] = 126 * 2.0 ** -7
    q, e, m = mx.mx_encode(v, 8)
    assert e[0, 0] == 120 and m[0, 0] == 1 and q[0, 0] == 63
    # absmax 31.5 -> t = 0.25 -> base 0.25; element with qa = 0.5 - 2^-25
    v = np.zeros((1, 16), np.float32)
    v[0, 0] = 31.5
    v[0, 2] = np.float32((0.5 - 2.0 ** -25) * 0.25)
    q_rne, e_rne, _ = mx.mx_encode(v, 8, mx.ROUND_NEAREST_EVEN)
    q_hu, _, _ = mx.mx_encode(v, 8, mx.ROUND_HALF_UP)
    assert e_rne[0, 0] == 125
    assert q_rne[0, 2] == 0 and q_hu[0, 2] == 1


def test_stochastic_rounding_extremes_and_unbiasedness():
    gen = torch.Generator().manual_seed(11)
    v = (torch.randn(256, 16, generator=gen)).numpy()
    q_floor, e, m = mx.mx_encode(v, 4, mx.ROUND_SR_UNIFORM, uniform=np.full(v.shape, 1 - 2**-24,
                                                                            np.float32))
    q_ceil, _, _ = mx.mx_encode(v, 4, mx.ROUND_SR_UNIFORM, uniform=np.zeros(v.shape, np.float32))
    ps = mx.exp2_scale(np.repeat(e.astype(np.uint32), 16, -1) + np.repeat(m.astype(np.uint32), 2, -1))
    qa = np.minimum(np.abs(v) / ps, 7)
    assert np.array_equal(np.abs(q_floor), np.floor(qa).astype(np.int8))
    assert np.array_equal(np.abs(q_ceil), np.ceil(qa).astype(np.int8))
    # mean of many stochastic encodes recovers the value
    acc = np.zeros_like(v, dtype=np.float64)
    n = 400
    for i in range(n):
        u = np.random.default_rng(i).random(v.shape, dtype=np.float32)
        qs, es, ms = mx.mx_encode(v, 4, mx.ROUND_SR_UNIFORM, uniform=u)
        acc += mx.mx_decode(qs, es, ms)
    bias = np.abs(acc / n - v) / ps
    assert bias.mean() < 0.03 and bias.max() < 0.2


def _grid_round(x: Fraction) -> Fraction:
    """x rounded to the nearest multiple of 2^-16, ties to the even multiple."""
    y = x * 65536
    lo = y.numerator // y.denominator
    r = y - lo
    k = lo + (1 if r > Fraction(1, 2) or (r == Fraction(1, 2) and lo % 2 == 1) else 0)
    return Fraction(k, 65536)


def _counter_level(qs: Fraction, u16: int, m: int) -> int:
    """The counter mode's level in exact rational arithmetic: qs + u16 * 2^-16 on the 2^-16
    grid, clamped to [-M, M + 1 - 2^-16], floored."""
    t = _grid_round(qs + Fraction(u16, 65536))
    t = min(max(t, Fraction(-m)), Fraction(m + 1) - Fraction(1, 65536))
    return t.numerator // t.denominator


def test_counter_dither_enumerates_to_the_rounded_fraction():
    """All 2^16 draws for one value: with F = frac(qa) * 2^16, |v| rounds up for floor(F + 1/2)
    draws when v > 0 and ceil(F - 1/2) when v < 0 (F to the nearest integer, a tie going to the
    even grid point), checked against exact rational arithmetic; the pair (7, x) of a block with
    absmax 7 has scale 1, so qa = |x|."""
    u = np.arange(1 << 16, dtype=np.uint32)
    xs = (2.3, 0.7, 6.99999, 1.0 + 2.0**-20, 5.0, 0.0, 3.0 + 2.0**-16 + 2.0**-17,
          4.0 + 2.0**-17, 2.0 - 2.0**-18, 1.0 + 3 * 2.0**-17)
    for x in xs:
        for sign in (1.0, -1.0):
            xv = np.float32(sign * x)
            v = np.zeros((u.size, 16), np.float32)
            v[:, 0] = 7.0
            v[:, 1] = xv
            draws = np.zeros(v.shape, np.uint32)
            draws[:, 1] = u
            q, e, m = mx.mx_encode(v, 4, mx.ROUND_SR_COUNTER, u16=draws)
            assert (e == 126).all() and (m[:, 0] == 1).all()
            mag = Fraction(float(abs(xv)))
            fl = int(mag)
            f16 = (mag - fl) * 65536
            half = Fraction(1, 2)
            if sign > 0:
                want_up = int(math.floor(f16 + half))
            else:
                want_up = int(math.ceil(f16 - half))
            lv = np.abs(q[:, 1].astype(np.int64))
            assert set(np.unique(lv)) <= {fl, fl + 1}
            assert int((lv == fl + 1).sum()) == want_up, (x, sign)
            if xv != 0:
                assert (np.sign(q[:, 1][lv > 0]) == np.sign(xv)).all()
            # level by level against the rational restatement (every 97th draw)
            for k in range(0, 1 << 16, 97):
                assert q[k, 1] == _counter_level(Fraction(float(xv)), k, 7), (x, sign, k)


def test_counter_dither_random_values_against_rationals():
    """Random blocks (both formats, many binades, micro pairs) level by level against the
    rational restatement, with the oracle's exponents and micro flags."""
    rs = np.random.default_rng(5)
    for fb, mant in ((4, 7), (8, 63)):
        v = (rs.standard_normal((64, 16)) * np.exp2(rs.integers(-30, 30, (64, 1)))).astype(np.float32)
        v[::7, 3] *= 3.0  # wide pairs: micro flags set
        draws = rs.integers(0, 1 << 16, v.shape).astype(np.uint32)
        q, e, m = mx.mx_encode(v, fb, mx.ROUND_SR_COUNTER, u16=draws)
        for i in range(v.shape[0]):
            for j in range(16):
                se = int(e[i, 0]) + int(m[i, j // 2])
                qs = Fraction(float(v[i, j])) / Fraction(2) ** (se - 127)
                assert q[i, j] == _counter_level(qs, int(draws[i, j]), mant), (fb, i, j)


def test_counter_dither_clamps_at_the_mantissa_limit():
    """A block whose rounded absmax/14 sits 20 ulps above 2^-80 keeps e = -80 (inside the
    correctly rounded log2 band), so the micro pair's qa = 7 + 140*2^-23 exceeds M = 7 by more
    than half the 2^-16 grid: without the clamp the largest draws would give level 8."""
    amax = np.float32(2.0**-77 * (1.75 + 35 * 2.0**-23))
    assert float(amax) / 14 == 2.0**-80 * (1 + 20 * 2.0**-23)
    u = np.arange(1 << 16, dtype=np.uint32)
    for sign in (1.0, -1.0):
        v = np.zeros((u.size, 16), np.float32)
        v[:, 0] = sign * amax
        draws = np.zeros(v.shape, np.uint32)
        draws[:, 0] = u
        q, e, m = mx.mx_encode(v, 4, mx.ROUND_SR_COUNTER, u16=draws)
        assert (e == 127 - 80).all() and (m[:, 0] == 1).all()
        assert (q[:, 0] == int(sign * 7)).all()
    qa = Fraction(float(amax)) * 2**79
    t = _grid_round(qa + Fraction(65535, 65536))
    assert t.numerator // t.denominator == 8


def _independent_update(h, x, dt, A, B, C, D, z, dt_bias, softplus):
    """float64 loop over heads, written without the oracle's broadcasting."""
    bsz, nh, p_, n = h.shape
    ratio = nh // B.shape[1]
    h2 = torch.empty_like(h, dtype=torch.float64)
    y = torch.empty(bsz, nh, p_, dtype=torch.float64)
    for hh in range(nh):
        g = hh // ratio
        d = dt[:, hh].double() + (dt_bias[hh].double() if dt_bias is not None else 0)
        if softplus:
            d = torch.where(d <= 20, torch.log1p(torch.exp(d)), d)
        decay = torch.exp(A[hh].double()[None] * d[..., None])
        h2[:, hh] = h[:, hh].double() * decay + B[:, g].double()[:, None, :] * (d * x[:, hh].double())[..., None]
        y[:, hh] = (h2[:, hh] * C[:, g].double()[:, None, :]).sum(-1)
        if D is not None:
            y[:, hh] += x[:, hh].double() * D[hh].double()
        if z is not None:
            y[:, hh] *= z[:, hh].double()
    return h2, y


def _inputs(bsz=2, nh=8, p_=4, n=32, ng=2, seed=12):
    g = torch.Generator().manual_seed(seed)
    return dict(
        h=torch.randn(bsz, nh, p_, n, generator=g) * 0.5,
        x=torch.randn(bsz, nh, p_, generator=g),
        dt=torch.nn.functional.softplus(torch.randn(bsz, nh, p_, generator=g)),
        A=-torch.exp(torch.rand(nh, p_, n, generator=g) * 2),
        B=torch.randn(bsz, ng, n, generator=g),
        C=torch.randn(bsz, ng, n, generator=g),
        D=torch.randn(nh, p_, generator=g),
        z=torch.randn(bsz, nh, p_, generator=g),
        dt_bias=torch.randn(nh, p_, generator=g) * 0.1,
    )


@pytest.mark.parametrize("softplus", [False, True])
def test_update_math_against_float64_loop(softplus):
    t = _inputs()
    h2, y = mx.update_math(t["h"], t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["z"],
                           t["dt_bias"], softplus)
    h2r, yr = _independent_update(t["h"], t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["z"],
                                  t["dt_bias"], softplus)
    assert torch.allclose(h2.double(), h2r, rtol=1e-5, atol=1e-6)
    assert torch.allclose(y.double(), yr, rtol=1e-4, atol=1e-5)


def test_update_closed_forms():
    t = _inputs()
    zero_dt = torch.zeros_like(t["dt"])
    h2, _ = mx.update_math(t["h"], t["x"], zero_dt, t["A"], t["B"], t["C"])
    assert torch.equal(h2, t["h"])  # dt = 0: the writeback is a pure re-encode
    h2, _ = mx.update_math(t["h"], t["x"], t["dt"], torch.zeros_like(t["A"]), t["B"], t["C"])
    ratio = 4
    Bh = t["B"].repeat_interleave(ratio, 1)
    assert torch.allclose(h2, t["h"] + (Bh[:, :, None, :] * t["dt"][..., None]) * t["x"][..., None])
    sp = mx.softplus_ref(torch.tensor([20.0, 20.5, -30.0]))
    assert sp[0] == torch.log(1 + torch.exp(torch.tensor(20.0))) and sp[1] == 20.5
    assert sp[2] >= 0


def test_mx_update_dt_zero_is_reencode():
    t = _inputs()
    q, e, m = mx.mx_encode(t["h"].numpy(), 8)
    q2, e2, m2, _, h2 = mx.mx_update(q, e, m, t["x"], torch.zeros_like(t["dt"]), t["A"], t["B"],
                                     t["C"], format_bits=8, round_mode=mx.ROUND_HALF_UP)
    assert torch.equal(h2, torch.from_numpy(mx.mx_decode(q, e, m)))
    q3, e3, m3 = mx.mx_encode(mx.mx_decode(q, e, m), 8, mx.ROUND_HALF_UP)
    assert np.array_equal(q2, q3) and np.array_equal(e2, e3) and np.array_equal(m2, m3)


def test_rng_vectorized_matches_scalar_and_golden():
    counters = np.array([0, 1, 2, 3, 1234567, (1 << 33) - 2, (1 << 33) - 1, 1 << 33,
                         (1 << 40) + 17, 2**63 + 5], dtype=np.uint64)
    for seed in (0, 1234, 2**40 + 7):
        vec = rng.uniforms(seed, counters)
        sca = np.array([rng.uniform_scalar(seed, int(c)) for c in counters], dtype=np.float32)
        assert np.array_equal(vec, sca)
    golden = json.loads((GOLDEN / "rng_vectors.json").read_text())
    for case in golden["cases"]:
        got = rng.uniforms(case["seed"], np.array(case["counters"], dtype=np.uint64))
        assert got.tolist() == case["uniforms"]
    assert rng.lowbias32_scalar(0) == golden["lowbias32"]["0"]
    assert rng.lowbias32_scalar(1) == golden["lowbias32"]["1"]


def test_rng_adjacent_draws_uncorrelated():
    """Draws of neighbouring counters -- the two halves of one hashed word, adjacent pairs and
    pairs further apart -- show no correlation: lag correlations within 5 sigma of zero and a
    2-D chi-square of (u_n, u_{n+lag}) on a 16x16 grid within its 0.9999 quantile."""
    n = 1 << 21
    u = rng.uniforms_u16(1234, np.arange(n, dtype=np.uint64) + np.uint64(7 << 20)).astype(np.float64)
    z = (u - u.mean()) / u.std()
    for lag in (1, 2, 3, 8, 15, 16, 17, 32):
        r = float(np.mean(z[:-lag] * z[lag:]))
        assert abs(r) < 5 / np.sqrt(n), (lag, r)
        a = (u[:-lag] / 4096).astype(np.int64)
        b = (u[lag:] / 4096).astype(np.int64)
        hist = np.bincount(a * 16 + b, minlength=256)
        expected = hist.sum() / 256
        chi2 = float(((hist - expected) ** 2 / expected).sum())
        assert chi2 < 360, (lag, chi2)  # 255 dof: the 0.9999 quantile is about 351-360
    # the draws at each position of a 16-value block, over many blocks, are uniform
    u16 = u.reshape(-1, 16)
    for j in range(16):
        hist = np.bincount((u16[:, j] / 4096).astype(np.int64), minlength=16)
        expected = hist.sum() / 16
        assert float(((hist - expected) ** 2 / expected).sum()) < 50, j


def test_rng_bijective_and_uniform():
    x = np.arange(1 << 20, dtype=np.uint32)
    y = rng.lowbias32(x)
    assert np.unique(y).size == x.size
    u = rng.state_uniforms(1234, 0, (16, 64, 128))
    assert 0.49 < u.mean() < 0.51 and u.min() >= 0 and u.max() < 1
    hist = np.bincount((u * 16).astype(int).ravel(), minlength=16)
    expected = u.size / 16
    chi2 = ((hist - expected) ** 2 / expected).sum()
    assert chi2 < 60  # 15 dof


def test_algorithmic_bytes_headline_figure():
    assert mx.update_algorithmic_bytes(64, 128, 64, 128, 8) == 212_092_416


def test_package_byte_counts_match_the_oracle():
    from layer_quant_amd import traffic

    for b in (1, 8, 64):
        assert traffic.mx_update_bytes(b, 128, 64, 128, 8) == mx.update_algorithmic_bytes(b, 128, 64, 128, 8)
    # the unquantized update moves 2 bytes per state element each way
    assert traffic.ssm_update_bytes(64, 128, 64, 128, 8) - traffic.mx_update_bytes(64, 128, 64, 128, 8) \
        == 2 * 64 * 128 * 64 * 128 * (2 - (1 + 1 / 16 + 1 / 2))


def test_compact_layout_bit_positions_and_round_trip():
    """to_compact against a per-element loop over the documented bit layout (nibble of value n
    at bits 4*(n%2) of byte n//2; micro bit of pair k at bit k%8 of byte k//8), and exact round
    trips for encoded MX4 and MX8 states."""
    rs = np.random.default_rng(3)
    for fb in (4, 8):
        h = (rs.standard_normal((2, 3, 5, 64)) * 0.5).astype(np.float32)
        q, e, m = mx.mx_encode(h, fb, mx.ROUND_NEAREST_EVEN)
        qc, ec, mc = mx.to_compact(q, e, m, fb)
        assert np.array_equal(ec, e)
        for idx in np.ndindex(*q.shape[:3]):
            row_q, row_m = q[idx], m[idx]
            for n in range(64):
                if fb == 4:
                    nib = (int(qc[idx][n // 2]) >> (4 * (n % 2))) & 0xF
                    assert (nib - 16 if nib > 7 else nib) == int(row_q[n])
                else:
                    assert int(qc[idx][n]) == int(row_q[n])
            for k in range(32):
                assert ((int(mc[idx][k // 8]) >> (k % 8)) & 1) == int(row_m[k])
        q2, e2, m2 = mx.from_compact(qc, ec, mc, fb)
        assert np.array_equal(q2, q) and np.array_equal(e2, e) and np.array_equal(m2, m)
        assert qc.shape[-1] == (32 if fb == 4 else 64) and mc.shape[-1] == 4
        assert np.array_equal(mx.mx_decode(q2, e2, m2), mx.mx_decode(q, e, m))
    with pytest.raises(ValueError):
        mx.to_compact(np.full((1, 1, 1, 16), 9, np.int8), np.zeros((1, 1, 1, 1), np.uint8),
                      np.zeros((1, 1, 1, 8), np.uint8), 4)
