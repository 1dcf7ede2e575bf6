"""Pins oracle.mx_state.bf16_state_update -- the restatement of mamba-ssm 2.3.2.post1's
selective_state_update, the update the reference runs for unregistered layers and as its
bf16-state baseline (hybrid_quant/mamba_state_8b_kernel.py:738-747) -- against an independent
implementation of the same semantics that is installed here: transformers'
models.nemotron_h.modeling_nemotron_h.mamba2_selective_state_update (its torch fallback, used
when mamba-ssm is absent). Both run in fp32 on an fp32 state with dt_bias, softplus and a silu(z)
gate; the oracle's only addition, the round-to-nearest-even store to bf16, is pinned by torch's
own bf16 conversion of the fp32 result."""
import pytest
import torch

from oracle import mx_state as omx

hf = pytest.importorskip("transformers.models.nemotron_h.modeling_nemotron_h")


def _inputs(seed, bsz=3, nh=8, p_=16, n=64, ng=2):
    g = torch.Generator().manual_seed(seed)
    return dict(
        state=torch.randn(bsz, nh, p_, n, generator=g) * 0.5,
        x=torch.randn(bsz, nh, p_, generator=g),
        dt=torch.randn(bsz, nh, 1, generator=g).expand(bsz, nh, p_) * 2,
        A=(-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n),
        B=torch.randn(bsz, ng, n, generator=g),
        C=torch.randn(bsz, ng, n, generator=g),
        D=torch.randn(nh, generator=g)[:, None].expand(nh, p_),
        z=torch.randn(bsz, nh, p_, generator=g),
        dt_bias=(torch.randn(nh, generator=g) * 0.5)[:, None].expand(nh, p_),
    )


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("gate", [True, False])
def test_bf16_state_update_matches_transformers_fallback(seed, gate):
    t = _inputs(seed)
    z = t["z"] if gate else None
    hf_state = t["state"].clone()
    y_hf = hf.mamba2_selective_state_update(hf_state, t["x"], t["dt"], t["A"], t["B"], t["C"],
                                            D=t["D"], dt_bias=t["dt_bias"], dt_softplus=True, z=z)
    h2, _ = omx.update_math(t["state"], t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], None,
                            t["dt_bias"], True)
    new_bf16, y = omx.bf16_state_update(t["state"], t["x"], t["dt"], t["A"], t["B"], t["C"],
                                        D=t["D"], z=z, dt_bias=t["dt_bias"], dt_softplus=True)
    # the updated state: same fp32 formula, evaluated in a different operation order
    assert torch.allclose(h2, hf_state, rtol=1e-5, atol=1e-6)
    # the oracle stores it round-to-nearest-even in bf16
    assert torch.equal(new_bf16, h2.to(torch.bfloat16))
    agree = (new_bf16 == hf_state.to(torch.bfloat16)).float().mean().item()
    assert agree > 0.999
    # y = C . h' + D x, times silu(z) when z is given
    assert torch.allclose(y, y_hf, rtol=1e-4, atol=1e-5)


def test_softplus_threshold_and_gate_are_the_ones_hf_uses():
    """softplus switches to the identity above 20 (both), and the gate is z * sigmoid(z)."""
    t = _inputs(5)
    for shift in (25.0, -40.0):  # large dt: identity branch; very negative: log(1 + e^x) ~ 0
        dt = t["dt"] + shift
        s = t["state"].clone()
        y_hf = hf.mamba2_selective_state_update(s, t["x"], dt, t["A"], t["B"], t["C"], D=t["D"],
                                                dt_bias=t["dt_bias"], dt_softplus=True, z=t["z"])
        _, y = omx.bf16_state_update(t["state"], t["x"], dt, t["A"], t["B"], t["C"], D=t["D"],
                                     z=t["z"], dt_bias=t["dt_bias"], dt_softplus=True)
        assert torch.allclose(y, y_hf, rtol=1e-4, atol=1e-5), shift
