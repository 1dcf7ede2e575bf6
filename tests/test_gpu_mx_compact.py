"""GPU tests of the compact MX state layout (micro-exponent bits; MX4 nibble mantissas): the
encoder writes exactly the oracle's compact form of its reference-layout output, the decoder and
the fused update give bit-identical results in both layouts (same arithmetic, every rounding
mode, both kernels), and the layout converter is lossless."""
import numpy as np
import pytest
import torch

from helpers import to_device
from hybrid_quant import mamba_state_8b_kernel as ms
from layer_quant_amd import _abi
from oracle import mx_state as omx

pytestmark = pytest.mark.gpu


def _state(shape, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(*shape, generator=g) * 0.5
    h = h * torch.exp(torch.randn(*shape[:-1], 1, generator=g))
    flat = h.view(-1, shape[-1])
    flat[0, :16] = 0.0
    flat[1, :16] *= 1e-20
    return h


def _tensors(shape, fb, layout, dev):
    b, h, p, n = shape
    if layout == "compact":
        q = torch.empty(b, h, p, n // 2 if fb == 4 else n, dtype=torch.uint8 if fb == 4 else torch.int8,
                        device=dev)
        m = torch.empty(b, h, p, n // 16, dtype=torch.uint8, device=dev)
    else:
        q = torch.empty(shape, dtype=torch.int8, device=dev)
        m = torch.empty(b, h, p, n // 2, dtype=torch.uint8, device=dev)
    return q, torch.empty(b, h, p, n // 16, dtype=torch.uint8, device=dev), m


def _as_np(t):
    return [x.cpu().numpy() for x in t]


@pytest.fixture(params=["rows", "general"])
def path(request, diag):
    """The row kernel (required: the library refuses a call that would take the general
    kernel), then the general kernel forced."""
    if request.param == "general":
        diag.set("LQ_MX_FORCE_GENERIC")
    else:
        diag.set("LQ_MX_REQUIRE_ROWS")
    return request.param


@pytest.mark.parametrize("fb", [4, 8])
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_encode_compact_is_oracle_compact(gpu, fb, mode):
    shape = (2, 4, 8, 128)
    h = _state(shape, 10 + fb)
    uni = torch.rand(shape, generator=torch.Generator().manual_seed(11))
    c = _tensors(shape, fb, "compact", gpu)
    _abi.mx_encode(h.to(gpu), *c, fb, mode, uniform=uni.to(gpu) if mode == 2 else None, seed=77,
                   rng_offset=4096)
    ref = omx.mx_encode(h.numpy(), fb, mode, uniform=uni.numpy() if mode == 2 else None, seed=77,
                        rng_offset=4096)
    want = omx.to_compact(*ref, fb)
    got = _as_np(c)
    for g, w, name in zip(got, want, ("q", "e", "micro")):
        assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), name
    deq = torch.empty(shape, device=gpu)
    _abi.mx_decode(*c, deq)
    assert np.array_equal(deq.cpu().numpy(), omx.mx_decode(*ref))


def _inputs(bsz, nh, p_, n, ng, seed):
    g = torch.Generator().manual_seed(seed)
    return dict(
        x=torch.randn(bsz, nh, p_, generator=g).to(torch.bfloat16),
        dt=torch.nn.functional.softplus(torch.randn(bsz, nh, 1, generator=g)).to(torch.bfloat16)
        .expand(bsz, nh, p_),
        A=(-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n),
        B=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        C=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        D=torch.randn(nh, generator=g)[:, None].expand(nh, p_),
        dt_bias=(torch.randn(nh, generator=g) * 0.1)[:, None].expand(nh, p_),
    )


@pytest.mark.parametrize("fb", [4, 8])
@pytest.mark.parametrize("mode", [1, 2, 3, 4])
@pytest.mark.parametrize("n", [64, 128])
def test_update_compact_equals_reference_layout(gpu, path, fb, mode, n):
    bsz, nh, p_, ng = 3, 16, 64, 4
    shape = (bsz, nh, p_, n)
    h0 = _state(shape, 20 + n)
    t = {k: to_device(v, gpu) for k, v in _inputs(bsz, nh, p_, n, ng, 21 + fb).items()}
    uni = torch.rand(shape, generator=torch.Generator().manual_seed(22)).to(gpu)
    states, ys = {}, {}
    for layout in ("reference", "compact"):
        st = _tensors(shape, fb, layout, gpu)
        _abi.mx_encode(h0.to(gpu), *st, fb, _abi.ROUND_NEAREST_EVEN)
        for step in range(3):
            y = torch.empty(bsz, nh, p_, device=gpu)
            _abi.mx_state_update(*st, t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"], t["D"],
                                 None, y, fb, True, mode, uniform=uni if mode == 2 else None,
                                 seed=5, rng_offset=step * bsz * nh * p_ * n)
        states[layout] = _as_np(st)
        ys[layout] = y.cpu()
    back = omx.from_compact(*states["compact"], fb)
    for g, w, name in zip(back, states["reference"], ("q", "e", "micro")):
        assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), name
    assert torch.equal(ys["compact"], ys["reference"])


@pytest.mark.parametrize("fb", [4, 8])
def test_module_api_compact_chain_and_conversion(gpu, fb):
    bsz, nh, p_, n, ng = 2, 8, 64, 128, 2
    h0 = _state((bsz, nh, p_, n), 30 + fb).to(gpu)
    ref = ms.allocate_state_kernel_cache(h0, format_bits=fb)
    cmp_ = ms.allocate_state_kernel_cache(h0, format_bits=fb, layout="compact")
    assert cmp_.layout == "compact" and cmp_.state_shape == (bsz, nh, p_, n)
    assert cmp_.micro_exp.shape[-1] == n // 16
    assert cmp_.q_state.shape[-1] == (n // 2 if fb == 4 else n)
    conv = ms.convert_state_cache_layout(ref, "compact")
    for a, b_ in ((conv.q_state, cmp_.q_state), (conv.shared_exp, cmp_.shared_exp),
                  (conv.micro_exp, cmp_.micro_exp)):
        assert torch.equal(a.view(torch.uint8), b_.view(torch.uint8))
    t = {k: to_device(v, gpu) for k, v in _inputs(bsz, nh, p_, n, ng, 31).items()}
    for _ in range(4):
        y1 = ms.mx_state_selective_update(ref, **t, dt_softplus=True)
        y2 = ms.mx_state_selective_update(cmp_, **t, dt_softplus=True)
        assert torch.equal(y1, y2)
    assert cmp_.step == ref.step == 4
    back = ms.convert_state_cache_layout(cmp_, "reference")
    assert back.step == 4 and back.layout == "reference"
    for a, b_ in ((back.q_state, ref.q_state), (back.shared_exp, ref.shared_exp),
                  (back.micro_exp, ref.micro_exp)):
        assert torch.equal(a, b_)
    assert torch.equal(ms.dequantize_state_cache(cmp_), ms.dequantize_state_cache(ref))


def test_full_size_b64_compact_mx4(gpu, diag):
    """Nemotron-H layer at batch 64 in the compact MX4 layout (row kernel), one counter-mode
    step: bit-identical to the reference layout."""
    diag.set("LQ_MX_REQUIRE_ROWS")
    bsz, nh, p_, n, ng = 64, 128, 64, 128, 8
    g = torch.Generator(device=gpu).manual_seed(8)
    h0 = torch.randn(bsz, nh, p_, n, device=gpu, generator=g) * 0.5
    t = {k: to_device(v, gpu) for k, v in _inputs(bsz, nh, p_, n, ng, 9).items()}
    out = {}
    for layout in ("reference", "compact"):
        c = ms.allocate_state_kernel_cache(h0, format_bits=4, layout=layout)
        y = ms.mx_state_selective_update(c, **t, dt_softplus=True)
        out[layout] = (ms.convert_state_cache_layout(c, "reference"), y)
    r, c = out["reference"][0], out["compact"][0]
    assert torch.equal(r.q_state, c.q_state)
    assert torch.equal(r.shared_exp, c.shared_exp)
    assert torch.equal(r.micro_exp, c.micro_exp)
    assert torch.equal(out["reference"][1], out["compact"][1])


def test_compact_layout_rejects_mx8_nibbles(gpu):
    shape = (1, 2, 4, 64)
    q, e, m = _tensors(shape, 4, "compact", gpu)
    with pytest.raises(_abi.LQError, match="MX4 only"):
        _abi.mx_encode(torch.zeros(shape, device=gpu), q, e, m, 8, 0)
