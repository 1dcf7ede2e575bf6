"""Shared checks of the test suite."""
from __future__ import annotations

import numpy as np
import torch

RTOL = 2e-3  # the attention output / updated state tolerance, fp32 accumulation

# lines that tests register for the session's terminal summary (conftest.py prints them)
REPORT: list[str] = []


def require_env(name: str, on: bool = True):
    """Turn the library's diagnostic switch `name` on for the block (when `on`): with
    LQ_ATTN_REQUIRE_FAST, LQ_PREFILL_REQUIRE_MFMA, LQ_MX_REQUIRE_ROWS or LQ_SSM_REQUIRE_ROWS on, a
    call that would take the general kernel fails instead."""
    from layer_quant_amd import _abi

    return _abi.diagnostic(name, on=on)


def fast_attention_expected(q_dtype, head_dim: int, group_size: int, nrep: int) -> bool:
    """The decode attention's MFMA gate for a contiguous packed cache: bf16 queries, head_dim
    128, group 32/64/128, 1-16 query heads per KV head (a power of two) with
    nrep * (128 / group) <= 16 MFMA columns."""
    return (q_dtype == torch.bfloat16 and head_dim == 128 and group_size in (32, 64, 128)
            and nrep in (1, 2, 4, 8, 16) and nrep * (128 // group_size) <= 16)


def prefill_mfma_expected(q_dtype, head_dim: int, group_size: int) -> bool:
    """The prefill's MFMA gate for a contiguous packed cache: bf16 queries, head_dim 128, group
    32/64/128."""
    return q_dtype == torch.bfloat16 and head_dim == 128 and group_size in (32, 64, 128)


def to_device(t: torch.Tensor | None, device) -> torch.Tensor | None:
    """t on `device` with its broadcast (stride-0) dimensions kept. Tensor.to copies an expanded
    tensor into a contiguous one, which would hand the library another layout than the model's
    (dt, A, D and dt_bias expanded along head_dim select the state updates' row kernels)."""
    if t is None:
        return None
    bcast = [s == 0 and n > 1 for s, n in zip(t.stride(), t.shape)]
    if not any(bcast):
        return t.to(device)
    base = t[tuple(slice(0, 1) if b else slice(None) for b in bcast)]
    return base.to(device).expand(t.shape)


def assert_close_rel(out: torch.Tensor, ref: torch.Tensor, rtol: float = RTOL, what: str = ""):
    """|out - ref| <= rtol * (|ref| + mean|ref|) elementwise, and the relative Frobenius error
    <= rtol. The mean|ref| term keeps outputs that cancel to nearly zero from demanding a
    tighter absolute error than the bulk of the tensor."""
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    err = (out - ref).abs()
    bound = rtol * (ref.abs() + ref.abs().mean())
    worst = (err / bound.clamp_min(1e-300)).max().item()
    fro = (err.norm() / ref.norm().clamp_min(1e-300)).item()
    print(f"[close] {what}: max err/bound {worst:.3g}, relative Frobenius {fro:.3g}")
    assert worst <= 1.0, f"{what}: max err/bound {worst:.3g} (max abs err {err.max().item():.3g})"
    assert fro <= rtol, f"{what}: relative Frobenius error {fro:.3g}"


def update_term_magnitudes(h, x, dt, A, B, C, dt_bias=None, dt_softplus=False):
    """|h * dA| + |dt * B * x| per state element (float64 numpy) from the oracle's update math:
    the scale of the difference between two fp32 evaluations of h' = h * dA + dt * B * x that
    differ in fused multiply-adds and in the exp/log approximations (about 1e-6 of it)."""
    from oracle import mx_state as omx

    h = torch.as_tensor(h).float()
    decay, _ = omx.update_math(h, x.float() * 0, dt, A, B, C, None, None, dt_bias, dt_softplus)
    drive, _ = omx.update_math(h * 0, x, dt, A, B, C, None, None, dt_bias, dt_softplus)
    return (decay.abs() + drive.abs()).double().numpy()


def mx_boundary_sites(h2, mag, format_bits, round_mode, uniform=None, seed=0, rng_offset=0,
                      eps=2.0 ** -20):
    """Where an updated state within eps * mag (elementwise) of the oracle's h2 may encode
    differently from the oracle's encoding of h2: (values [..., N], pairs [..., N/2],
    blocks [..., N/16]) boolean flags.

    Every encoder decision is monotone in the magnitudes it reads -- the block exponent in the
    block absmax, a pair's micro-exponent in the pair absmax, a value's level in the value at a
    fixed scale and random draw -- so encoding the magnitudes shrunk and grown by eps * mag
    brackets every encoding reachable inside the interval: a decision that agrees at both ends
    cannot change. Values with |h2| <= eps * mag may change sign and are always flagged."""
    from oracle import mx_state as omx

    h = np.asarray(h2, dtype=np.float64)
    d = eps * np.asarray(mag, dtype=np.float64)
    a = np.abs(h)
    sgn = np.where(h < 0, -1.0, 1.0)
    lo = (sgn * np.maximum(a - d, 0.0)).astype(np.float32)
    hi = (sgn * (a + d)).astype(np.float32)
    kw = dict(uniform=uniform, seed=seed, rng_offset=rng_offset)
    ql, el, ml = omx.mx_encode(lo, format_bits, round_mode, **kw)
    qh, eh, mh = omx.mx_encode(hi, format_bits, round_mode, **kw)
    blocks = el != eh
    pairs = (ml != mh) | np.repeat(blocks, 8, -1)
    values = (ql != qh) | np.repeat(pairs, 2, -1) | (a <= d)
    return values, pairs, blocks


def assert_mx_writeback(got, ref, h2, mag, format_bits, round_mode, uniform=None, seed=0,
                        rng_offset=0, what=""):
    """An MX writeback of a state updated in fp32 against the oracle's (got, ref = (q, e, m)
    numpy triples): equal everywhere except at encoder decision boundaries, i.e. where the
    oracle's h2 lies within 2^-20 * (|h*dA| + |dt*B*x|) of a block-exponent, micro-exponent or
    rounding threshold (mx_boundary_sites); there the kernel's h', which differs from the
    oracle's by fused multiply-adds and the hardware exp/log (about 1e-6 of those terms), may
    fall on the other side. In addition >= 99.9% of the mantissas are identical and every
    dequantized value is within one quantization step (of the larger scale) of the oracle's."""
    from oracle import mx_state as omx

    q, e, m = (np.asarray(t) for t in got)
    rq, re_, rm = (np.asarray(t) for t in ref)
    values, pairs, blocks = mx_boundary_sites(h2, mag, format_bits, round_mode, uniform, seed,
                                              rng_offset)
    dq, de, dm = q != rq, e != re_, m != rm
    print(f"[mx] {what}: {dq.sum()} of {dq.size} mantissas, {dm.sum()} micro bits, {de.sum()} "
          f"exponents differ; boundary sites: {values.sum()} values, {pairs.sum()} pairs, "
          f"{blocks.sum()} blocks")
    assert not np.any(de & ~blocks), f"{what}: exponents differ off a boundary at " \
        f"{np.argwhere(de & ~blocks)[:5].tolist()}"
    assert not np.any(dm & ~pairs), f"{what}: micro bits differ off a boundary at " \
        f"{np.argwhere(dm & ~pairs)[:5].tolist()}"
    assert not np.any(dq & ~values), f"{what}: mantissas differ off a boundary at " \
        f"{np.argwhere(dq & ~values)[:5].tolist()}"
    assert np.mean(~dq) > 0.999, f"{what}: only {np.mean(~dq):.5f} of mantissas identical"
    g = omx.mx_decode(q, e, m).astype(np.float64)
    w = omx.mx_decode(rq, re_, rm).astype(np.float64)
    step = lambda e_, m_: omx.exp2_scale(np.repeat(e_.astype(np.uint32), 16, -1)
                                         + np.repeat(m_.astype(np.uint32), 2, -1))
    bound = np.maximum(step(e, m), step(re_, rm)).astype(np.float64)
    assert np.all(np.abs(g - w) <= bound * (1 + 1e-6)), f"{what}: a value moved by more than " \
        "one level"
