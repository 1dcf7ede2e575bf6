"""Shared checks of the test suite."""
from __future__ import annotations

import torch

RTOL = 2e-3  # the attention output / updated state tolerance, fp32 accumulation


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
    assert worst <= 1.0, f"{what}: max err/bound {worst:.3g} (max abs err {err.max().item():.3g})"
    assert fro <= rtol, f"{what}: relative Frobenius error {fro:.3g}"
