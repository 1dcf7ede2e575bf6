"""CPU restatement of the reference's MX8/MX4 Mamba2 state path -- TEST INFRASTRUCTURE ONLY.

Reference: hybrid_quant/mamba_state_8b_kernel.py (cited as ms.py:line below).

MX block format (ms.py:11-25): 16-value blocks along d_state; one biased 8-bit shared exponent
per block (127 = 2^0); one micro-exponent bit per pair of values; signed integer mantissas
|q| <= M with M = 63 (MX8) or 7 (MX4), stored one int8 per value in both formats.
Encode of a block with absmax a (ms.py:168-203, 512-534, 557-571):
    e     = clamp(ceil(log2(max(a / (2M), 1e-30))) + 127, 1, 254)
    base  = 1 if a == 0 else 2^(e - 127)
    micro = pair_absmax > M * base
    qa    = min(|v| / (base * 2^micro), M)
    level = round(qa)  (one of the modes below), min(level, M), negated when v < 0
Rounding modes: nearest-even (torch.round, initial encode ms.py:568), half-up floor(qa + 0.5)
(deterministic writeback ms.py:201, 482, 531), stochastic floor(qa) + (u < qa - floor(qa))
(ms.py:196-199, 528-530) with u from a supplied tensor (ROUND_SR_UNIFORM, the reference's
formula) or from the reference's own generator (ROUND_SR_PHILOX: u = tl.rand(seed, rng_offset +
index), oracle.philox), and the counter mode ROUND_SR_COUNTER, which replaces the reference's
Triton tl.rand draw by oracle.rng's 16-bit draws u16 used as a dither on a 2^-16 grid:
    qs    = v / (base * 2^micro)                                  (signed, exact)
    t     = fp32(192 + u16 * 2^-16 + qs)                          (one rounding: the kernel's fma)
    level = floor(clamp(t, 192 - M, 193 + M - 2^-16)) - 192
t lies in [128, 256), where the fp32 spacing is 2^-16, so t is qs + u16 * 2^-16 rounded to that
grid (ties to even) plus 192. For v >= 0 it rounds |v| up for floor(F + 1/2) of the 2^16 draws,
for v < 0 for ceil(F - 1/2), F = frac(|qs|) * 2^16: F rounded to the nearest integer, so the
bias stays within half a grid step (2^-17 of a level step), on both signs; the clamp (a no-op
unless |qs| > M, which only a block inside the exponent's rounding band can give) keeps the
level in [-M, M].

ceil(log2(t)) is defined as the ceiling of the correctly rounded fp32 log2 of t. For a t with
unbiased exponent E and mantissa field j, that ceiling is E when j == 0, E when the fp32 value
of E + log2(1 + j*2^-23) rounds back to E, and E + 1 otherwise. The rounding back to E happens
exactly for 0 < j <= T(E), where T depends only on the fp32 spacing around E and is tabulated
below; torch's fp32 log2 agrees with it wherever it is correctly rounded.

Pinning (tests/test_oracle_mx.py): the T table against a 60-digit mpmath evaluation for every
reachable E; ceil_log2 against exact integer comparisons away from the rounding band; encode
invariants (|q| <= M, e in [1, 254], micro in {0,1}); half-step error bound of the nearest-even
decode; the all-zero block (e = 28, q = 0); exact powers of two; the floor(q + 0.5) double
rounding case; stochastic rounding with u = 0 (ceil) and u -> 1 (floor) and its unbiasedness;
the counter dither by enumerating all 2^16 draws (the round-up count against exact rational
arithmetic on the 2^-16 grid, for both signs, ties included) and its clamp, and random values
against a Fraction restatement;
the update's closed forms (dt = 0 leaves h unchanged so the writeback is a pure re-encode;
A = 0 gives h + dt*B*x; softplus threshold at 20) against an independent float64 evaluation.
bf16_state_update (drift baseline) restates mamba_ssm's selective_state_update, a dependency
(mamba-ssm 2.3.2.post1) that is not installed. It is pinned (tests/test_oracle_bf16_state.py) in
fp32 against an independent implementation of the same semantics that is installed:
transformers' modeling_nemotron_h.mamba2_selective_state_update (dt_bias, softplus with the
identity above 20, the decay/input update and the silu(z) gate); its bf16 store by torch's
round-to-nearest-even conversion. Only bit parity with mamba-ssm's own Triton kernel (its
approximate exp and operation order) stays unpinned.

Compact layout (this build's opt-in cache layout, no reference counterpart): to_compact /
from_compact convert the reference layout to micro-exponent bits (bit k of byte j = pair 8j + k
of the row) and, for MX4, two's-complement nibble mantissas (byte p = value 2p in the low
nibble, 2p + 1 in the high); pinned by a per-element loop over the bit layout and round trips.
"""
from __future__ import annotations

import numpy as np
import torch

from . import philox, rng

BLOCK = 16
PAIR = 2
MANTISSA_MAX = {8: 63.0, 4: 7.0}
EXP_FLOOR = np.float32(1.0e-30)

ROUND_NEAREST_EVEN = 0
ROUND_HALF_UP = 1
ROUND_SR_UNIFORM = 2
ROUND_SR_COUNTER = 3
ROUND_SR_PHILOX = 4

# T(kk) for kk = -1..8, where the half spacing of fp32 around E is 2^(kk - 24).
# T(kk) = largest j with log2(1 + j*2^-23) < 2^(kk-24)  (= floor(2^(kk-1) * ln 2) here).
CEIL_LOG2_T = np.array([0, 0, 0, 1, 2, 5, 11, 22, 44, 88], dtype=np.int64)


def _spacing_class(e: np.ndarray) -> np.ndarray:
    """kk such that half the fp32 spacing at the value E + log2(1 + tiny) is 2^(kk - 24)."""
    a = np.abs(e).astype(np.int64)
    a_safe = np.maximum(a, 1)
    fl = np.floor(np.log2(a_safe.astype(np.float64))).astype(np.int64)
    # guard the float64 floor(log2) at exact powers of two
    fl = np.where((np.int64(1) << (fl + 1)) <= a_safe, fl + 1, fl)
    fl = np.where((np.int64(1) << fl) > a_safe, fl - 1, fl)
    pow2 = (a_safe & (a_safe - 1)) == 0
    return np.where((e < 0) & pow2, fl - 1, fl)


def ceil_log2_f32(t: np.ndarray) -> np.ndarray:
    """ceil(fp32 correctly rounded log2(t)) for positive normal (or +inf) float32 t."""
    t = np.asarray(t, dtype=np.float32)
    bits = t.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127
    mant = bits & 0x7FFFFF
    kk = _spacing_class(e)
    thr = CEIL_LOG2_T[np.clip(kk + 1, 0, len(CEIL_LOG2_T) - 1)]
    thr = np.where(e == 0, 0, thr)
    return np.where(mant == 0, e, np.where(mant <= thr, e, e + 1)).astype(np.int64)


def exp2_scale(biased: np.ndarray) -> np.ndarray:
    """2^(biased - 127) as float32 built from the exponent bits (biased 255 -> +inf)."""
    b = np.asarray(biased, dtype=np.uint32)
    return (b << np.uint32(23)).view(np.float32)


def mx_encode(state, format_bits: int, round_mode: int = ROUND_NEAREST_EVEN,
              uniform: np.ndarray | None = None, seed: int = 0,
              rng_offset: int = 0, u16: np.ndarray | None = None
              ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Encode a float state [..., N] -> (q int8 [..., N], shared_exp u8 [..., N/16],
    micro_exp u8 [..., N/2]). `u16` overrides the counter draws of ROUND_SR_COUNTER."""
    if isinstance(state, torch.Tensor):
        state = state.detach().float().cpu().numpy()
    v = np.asarray(state, dtype=np.float32)
    n = v.shape[-1]
    if n % BLOCK != 0:
        raise ValueError(f"MX{format_bits} state dim must be divisible by {BLOCK}, got {n}")
    m = np.float32(MANTISSA_MAX[format_bits])
    blocks = v.reshape(*v.shape[:-1], n // BLOCK, BLOCK)
    amax = np.abs(blocks).max(axis=-1)
    t = np.maximum(amax / np.float32(2.0 * MANTISSA_MAX[format_bits]), EXP_FLOOR)
    raw = ceil_log2_f32(t)
    biased = np.clip(raw + 127, 1, 254)
    base = np.where(amax == 0, np.float32(1.0), exp2_scale(biased)).astype(np.float32)
    pairs = blocks.reshape(*blocks.shape[:-1], BLOCK // PAIR, PAIR)
    pair_amax = np.abs(pairs).max(axis=-1)
    micro = pair_amax > (m * base)[..., None]
    pair_scale = (base[..., None] * np.where(micro, np.float32(2.0), np.float32(1.0))).astype(
        np.float32)
    if round_mode == ROUND_SR_COUNTER:
        # dither on the 2^-16 grid: qs = v / pair_scale exactly (the pair scale is a power of two,
        # 2^(se-127) with se = exponent + micro and exponent 127 for a zero block);
        # t = fp32(192 + u16 * 2^-16 + qs), level = floor(t) - 192 after the clamp. The float64
        # sum is exact for |qs| >= 2^-22 (at most 53 bits from 2^7 down to qs's last bit); below
        # that qs is under a quarter of the fp32 spacing of t, so either way t = 192 + u16 * 2^-16.
        se = np.where(amax == 0, 127, biased)[..., None] + micro.astype(np.int64)
        qs = np.ldexp(pairs.astype(np.float64), (127 - se)[..., None].astype(np.int32))
        if u16 is None:
            u16 = rng.state_u16(seed, rng_offset, v.shape)
        u16 = np.asarray(u16).reshape(pairs.shape).astype(np.float64)
        with np.errstate(invalid="ignore"):
            t = (192.0 + u16 * 2.0**-16 + qs).astype(np.float32)
        t = np.clip(t, np.float32(192.0) - m, np.float32(193.0 - 2.0**-16) + m)
        level = np.floor(t).astype(np.int64) - 192
        q = level.reshape(v.shape).astype(np.int8)
        shared = biased.astype(np.uint8)
        micro_u8 = micro.astype(np.uint8).reshape(*v.shape[:-1], n // PAIR)
        return q, shared, micro_u8
    qa = np.minimum(np.abs(pairs) / pair_scale[..., None], m)
    if round_mode == ROUND_NEAREST_EVEN:
        level = np.rint(qa)
    elif round_mode == ROUND_HALF_UP:
        level = np.floor(qa + np.float32(0.5))
    elif round_mode in (ROUND_SR_UNIFORM, ROUND_SR_PHILOX):
        if round_mode == ROUND_SR_PHILOX:  # the reference's own draws: tl.rand per element
            uniform = philox.state_uniforms(seed, rng_offset, v.shape)
        if uniform is None:
            raise ValueError("ROUND_SR_UNIFORM needs a uniform tensor")
        if isinstance(uniform, torch.Tensor):
            uniform = uniform.detach().float().cpu().numpy()
        u = np.asarray(uniform, dtype=np.float32).reshape(pairs.shape)
        fl = np.floor(qa)
        level = fl + (u < (qa - fl)).astype(np.float32)
    else:
        raise ValueError(f"unknown round_mode {round_mode}")
    level = np.minimum(level, m)
    q = np.where(pairs < 0, -level, level).reshape(v.shape).astype(np.int8)
    shared = biased.astype(np.uint8)
    micro_u8 = micro.astype(np.uint8).reshape(*v.shape[:-1], n // PAIR)
    return q, shared, micro_u8


def mx_decode(q, shared_exp, micro_exp) -> np.ndarray:
    """h = q * 2^(e - 127 + micro) in float32 (ms.py:132, 322)."""
    q = np.asarray(q.cpu().numpy() if isinstance(q, torch.Tensor) else q)
    e = np.asarray(shared_exp.cpu().numpy() if isinstance(shared_exp, torch.Tensor) else shared_exp)
    mi = np.asarray(micro_exp.cpu().numpy() if isinstance(micro_exp, torch.Tensor) else micro_exp)
    n = q.shape[-1]
    e_full = np.repeat(e.astype(np.uint32), BLOCK, axis=-1)
    m_full = np.repeat(mi.astype(np.uint32), PAIR, axis=-1)
    scale = exp2_scale(e_full + m_full)
    assert scale.shape[-1] == n
    return (q.astype(np.float32) * scale).astype(np.float32)


def to_compact(q: np.ndarray, shared_exp: np.ndarray, micro_exp: np.ndarray, format_bits: int):
    """Reference layout -> compact layout (q nibbles for MX4, micro bits)."""
    q = np.asarray(q, dtype=np.int8)
    m = np.asarray(micro_exp, dtype=np.uint8)
    *lead, n = q.shape
    if format_bits == 4:
        if np.abs(q.astype(np.int16)).max(initial=0) > 7:
            raise ValueError("MX4 mantissas must lie in [-7, 7]")
        u = q.view(np.uint8) & np.uint8(0x0F)
        qc = (u[..., 0::2] | (u[..., 1::2] << np.uint8(4))).astype(np.uint8)
    else:
        qc = q.copy()
    bits = m.reshape(*lead, n // BLOCK, 8).astype(np.uint32) & np.uint32(1)
    mc = (bits << np.arange(8, dtype=np.uint32)).sum(axis=-1).astype(np.uint8)
    return qc, np.asarray(shared_exp, dtype=np.uint8).copy(), mc


def from_compact(qc: np.ndarray, shared_exp: np.ndarray, mc: np.ndarray, format_bits: int):
    """Compact layout -> reference layout."""
    qc = np.asarray(qc)
    mc = np.asarray(mc, dtype=np.uint8)
    *lead, nb = mc.shape
    n = nb * BLOCK
    if format_bits == 4:
        u = qc.view(np.uint8) if qc.dtype == np.int8 else qc.astype(np.uint8)
        lo = (u & np.uint8(0x0F)).astype(np.int16)
        hi = (u >> np.uint8(4)).astype(np.int16)
        q = np.empty((*lead, n), dtype=np.int16)
        q[..., 0::2] = np.where(lo > 7, lo - 16, lo)
        q[..., 1::2] = np.where(hi > 7, hi - 16, hi)
        q = q.astype(np.int8)
    else:
        q = qc.astype(np.int8)
    m = ((mc[..., None].astype(np.uint32) >> np.arange(8, dtype=np.uint32)) & np.uint32(1))
    return q, np.asarray(shared_exp, dtype=np.uint8).copy(), m.reshape(*lead, n // PAIR).astype(np.uint8)


def softplus_ref(x: torch.Tensor) -> torch.Tensor:
    """ms.py:28-30: x <= 20 ? log(1 + exp(x)) : x."""
    return torch.where(x <= 20.0, torch.log(1.0 + torch.exp(x)), x)


def update_math(h: torch.Tensor, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                dt_softplus: bool = False, dtype=torch.float32):
    """Dequantized-state update and output (ms.py:134-166, 324-368).

    h [B,H,P,N]; x, dt [B,H,P]; A [H,P,N]; B, C [B,G,N]; D, dt_bias [H,P]; z [B,H,P].
    Returns (h' [B,H,P,N], y [B,H,P]) computed in `dtype`.
    """
    bsz, nheads, dim, dstate = h.shape
    ratio = nheads // B.shape[1]
    hf = h.to(dtype)
    xf = x.to(dtype)
    dtf = dt.to(dtype)
    if dt_bias is not None:
        dtf = dtf + dt_bias.to(dtype)[None]
    if dt_softplus:
        dtf = softplus_ref(dtf)
    grp = torch.arange(nheads) // ratio
    Bh = B.to(dtype)[:, grp]  # [B,H,N]
    Ch = C.to(dtype)[:, grp]
    dA = torch.exp(A.to(dtype)[None] * dtf[..., None])
    h2 = hf * dA + (Bh[:, :, None, :] * dtf[..., None]) * xf[..., None]
    y = (h2 * Ch[:, :, None, :]).sum(dim=-1)
    if D is not None:
        y = y + xf * D.to(dtype)[None]
    if z is not None:
        y = y * z.to(dtype)
    return h2, y


def mx_update(q, shared_exp, micro_exp, x, dt, A, B, C, D=None, z=None, dt_bias=None,
              dt_softplus: bool = False, format_bits: int = 8,
              round_mode: int = ROUND_SR_COUNTER, uniform=None, seed: int = 1234,
              rng_offset: int = 0):
    """One fused MX update (ms.py:97-222 for MX8; :289-443 then :494-544 for MX4).

    Returns (q', shared_exp', micro_exp', y f32, h' f32) with h' the fp32 updated state that
    the writeback encodes.
    """
    h = torch.from_numpy(mx_decode(q, shared_exp, micro_exp))
    h2, y = update_math(h, x.cpu(), dt.cpu(), A.cpu(), B.cpu(), C.cpu(),
                        None if D is None else D.cpu(), None if z is None else z.cpu(),
                        None if dt_bias is None else dt_bias.cpu(), dt_softplus)
    q2, e2, m2 = mx_encode(h2.numpy(), format_bits, round_mode, uniform=uniform, seed=seed,
                           rng_offset=rng_offset)
    return q2, e2, m2, y, h2


def bf16_state_update(state: torch.Tensor, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                      dt_softplus: bool = False):
    """bf16-state baseline: fp32 update of a bf16 state, stored back as bf16 (round to nearest
    even), y from the fp32 updated state; z gates with silu as mamba_ssm does.
    Returns (new_state bf16, y f32)."""
    h2, y_nogate = update_math(state.float(), x, dt, A, B, C, D, None, dt_bias, dt_softplus)
    if z is not None:
        zf = z.float()
        y_nogate = y_nogate * (zf * torch.sigmoid(zf))
    return h2.to(torch.bfloat16), y_nogate


def update_algorithmic_bytes(batch: int, nheads: int, dim: int, dstate: int, ngroups: int,
                             x_bytes: int = 2, out_bytes: int = 2, dt_bytes: int = 2) -> int:
    """Unique bytes of one MX update call in the reference layout (state read + write once)."""
    elems = batch * nheads * dim * dstate
    state = 2 * (elems + elems // BLOCK + elems // PAIR)
    io = batch * nheads * dim * (x_bytes + out_bytes)
    bc = 2 * batch * ngroups * dstate * 2
    scalars = batch * nheads * dt_bytes + 3 * nheads * 4
    return state + io + bc + scalars
