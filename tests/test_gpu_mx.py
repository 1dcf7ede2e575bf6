"""GPU parity of the MX8/MX4 state path through the C ABI: encoders and decoder bit-exact
against the oracle in every rounding mode; the fused update's y within 2e-3, its writeback
bit-exact when dt = 0 (h' = h) and within 2e-3 (normwise, with rare single-level boundary flips)
otherwise; multi-step chains with the counter generator."""
import numpy as np
import pytest
import torch

from helpers import assert_close_rel, assert_mx_writeback, to_device, update_term_magnitudes
from layer_quant_amd import _abi
from hybrid_quant import mamba_state_8b_kernel as ms
from oracle import mx_state as omx

pytestmark = pytest.mark.gpu


def _state(shape, seed, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    h = torch.randn(*shape, generator=gen) * 0.5
    h = h * torch.exp(torch.randn(*shape[:-1], 1, generator=gen))  # per-row magnitudes
    flat = h.view(-1, shape[-1])
    flat[0, :16] = 0.0                                                 # an all-zero block
    flat[1, :16] = 0.0
    flat[1, 3] = 126 * 2.0 ** -7                                       # amax/126 a power of two
    flat[2, 5] = float(np.float32(np.ldexp(1 + 2.0 ** -23, -3) * 126))  # inside the log2 band
    flat[3, :16] *= 1e-20                                              # tiny block
    return h.to(dtype)


def _mx_tensors(shape, device):
    b, h, p, n = shape
    return (torch.empty(shape, dtype=torch.int8, device=device),
            torch.empty(b, h, p, n // 16, dtype=torch.uint8, device=device),
            torch.empty(b, h, p, n // 2, dtype=torch.uint8, device=device))


def _assert_mx_equal(gpu_t, ref):
    q, e, m = (t.cpu().numpy() for t in gpu_t)
    rq, re_, rm = ref
    assert np.array_equal(e, re_), f"exponents differ at {np.argwhere(e != re_)[:5]}"
    assert np.array_equal(m, rm), f"micro bits differ at {np.argwhere(m != rm)[:5]}"
    assert np.array_equal(q, rq), f"mantissas differ at {np.argwhere(q != rq)[:5]}"


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_encode_bit_exact(gpu, fb, mode, dtype):
    shape = (3, 8, 16, 128)
    h = _state(shape, 10 + fb + mode, dtype)
    uni = torch.rand(shape, generator=torch.Generator().manual_seed(5)) if mode == 2 else None
    seed, off = 1234, 2 * 987654321
    out = _mx_tensors(shape, gpu)
    _abi.mx_encode(h.to(gpu), *out, fb, mode, None if uni is None else uni.to(gpu), seed, off)
    ref = omx.mx_encode(h.float().numpy(), fb, mode, uniform=uni, seed=seed, rng_offset=off)
    _assert_mx_equal(out, ref)


@pytest.mark.parametrize("n", [128, 64, 48, 16])
def test_encode_decode_state_widths(gpu, n):
    shape = (2, 4, 8, n)
    h = _state(shape, 20 + n)
    out = _mx_tensors(shape, gpu)
    _abi.mx_encode(h.to(gpu), *out, 8, 0)
    ref = omx.mx_encode(h.numpy(), 8, 0)
    _assert_mx_equal(out, ref)
    deq = torch.empty(shape, device=gpu)
    _abi.mx_decode(*out, deq)
    assert np.array_equal(deq.cpu().numpy(), omx.mx_decode(*ref))


def _inputs(bsz, nh, p_, n, ng, seed, device, dt_zero=False, head_dt=False):
    """Decode-step inputs. head_dt=True gives dt one value per (batch, head), expanded along
    head_dim as Nemotron-H passes it: with the head-constant A, D and dt_bias below, that is the
    layout the library's row kernel takes (the general kernel takes the rest)."""
    g = torch.Generator().manual_seed(seed)
    dt_shape = (bsz, nh, 1) if head_dt else (bsz, nh, p_)
    dt = torch.nn.functional.softplus(torch.randn(*dt_shape, generator=g)).to(torch.bfloat16)
    if dt_zero:
        dt = torch.zeros_like(dt)
    t = dict(
        x=torch.randn(bsz, nh, p_, generator=g).to(torch.bfloat16),
        dt=dt.expand(bsz, nh, p_),
        A=(-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n),
        B=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        C=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        D=torch.randn(nh, generator=g)[:, None].expand(nh, p_),
        dt_bias=(torch.randn(nh, generator=g) * 0.1)[:, None].expand(nh, p_),
    )
    return {k: to_device(v, device) for k, v in t.items()}


@pytest.fixture(params=["rows", "general"])
def path(request, diag):
    """Run a test on the row kernel's layout (the library refuses the call if it would take the
    general kernel), and once more with the general kernel forced."""
    if request.param == "general":
        diag.set("LQ_MX_FORCE_GENERIC")
    else:
        diag.set("LQ_MX_REQUIRE_ROWS")
    return request.param


def _cpu(t):
    return {k: v.cpu() for k, v in t.items()}


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_update_dt_zero_writeback_bit_exact(gpu, path, fb, mode):
    shape = (2, 16, 8, 128)
    h0 = _state(shape, 30 + fb)
    q, e, m = omx.mx_encode(h0.numpy(), fb, 0)
    t = _inputs(2, 16, 8, 128, 2, 31, gpu, dt_zero=True, head_dt=True)
    uni = torch.rand(shape, generator=torch.Generator().manual_seed(32))
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(2, 16, 8, device=gpu)
    _abi.mx_state_update(*st, t["x"], t["dt"], None, t["A"], t["B"], t["C"], t["D"], None, out,
                         fb, False, mode, uniform=uni.to(gpu) if mode == 2 else None, seed=99,
                         rng_offset=4096)
    c = _cpu(t)
    rq, re_, rm, ry, rh = omx.mx_update(q, e, m, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                        D=c["D"], format_bits=fb, round_mode=mode, uniform=uni,
                                        seed=99, rng_offset=4096)
    assert torch.equal(rh, torch.from_numpy(omx.mx_decode(q, e, m)))  # dt = 0: h' = h
    _assert_mx_equal(st, (rq, re_, rm))
    assert_close_rel(out.cpu(), ry, what="y")


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("softplus", [True, False])
@pytest.mark.parametrize("head_dt", [True, False])
def test_update_parity(gpu, diag, fb, softplus, head_dt):
    bsz, nh, p_, n, ng = 4, 32, 16, 128, 4
    if head_dt:  # the model's layout: the row kernel
        diag.set("LQ_MX_REQUIRE_ROWS")
    shape = (bsz, nh, p_, n)
    h0 = _state(shape, 40 + fb)
    q, e, m = omx.mx_encode(h0.numpy(), fb, 0)
    t = _inputs(bsz, nh, p_, n, ng, 41, gpu, head_dt=head_dt)
    z = torch.randn(bsz, nh, p_, generator=torch.Generator().manual_seed(42)).to(gpu)
    uni = torch.rand(shape, generator=torch.Generator().manual_seed(43))
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(bsz, nh, p_, device=gpu)
    _abi.mx_state_update(*st, t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"], t["D"], z,
                         out, fb, softplus, 2, uniform=uni.to(gpu))
    c = _cpu(t)
    rq, re_, rm, ry, rh = omx.mx_update(q, e, m, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                        D=c["D"], z=z.cpu(), dt_bias=c["dt_bias"],
                                        dt_softplus=softplus, format_bits=fb, round_mode=2,
                                        uniform=uni)
    assert_close_rel(out.cpu(), ry, what="y")
    mag = update_term_magnitudes(omx.mx_decode(q, e, m), c["x"], c["dt"], c["A"], c["B"],
                                 c["C"], dt_bias=c["dt_bias"], dt_softplus=softplus)
    assert_mx_writeback([a.cpu().numpy() for a in st], (rq, re_, rm), rh, mag, fb, 2,
                        uniform=uni, what="state")


def test_update_general_A_and_strides(gpu):
    """A varying along d_state (per-element exp), fp32 inputs, non-contiguous x."""
    bsz, nh, p_, n, ng = 2, 8, 8, 64, 2
    shape = (bsz, nh, p_, n)
    h0 = _state(shape, 50)
    q, e, m = omx.mx_encode(h0.numpy(), 8, 0)
    g = torch.Generator().manual_seed(51)
    x = torch.randn(bsz, p_, nh, generator=g).transpose(1, 2)  # strided view
    dt = torch.zeros(bsz, nh, p_)
    A = -torch.rand(nh, p_, n, generator=g)
    B = torch.randn(bsz, ng, n, generator=g)
    C = torch.randn(bsz, ng, n, generator=g)
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(bsz, nh, p_, device=gpu)
    _abi.mx_state_update(*st, x.to(gpu).transpose(1, 2).contiguous().transpose(1, 2), dt.to(gpu),
                         None, A.to(gpu), B.to(gpu), C.to(gpu), None, None, out, 8, False, 1)
    rq, re_, rm, ry, _ = omx.mx_update(q, e, m, x, dt, A, B, C, format_bits=8, round_mode=1)
    _assert_mx_equal(st, (rq, re_, rm))
    assert_close_rel(out.cpu(), ry, what="y")
    dt = torch.rand(bsz, nh, p_, generator=g)
    out2 = torch.empty(bsz, nh, p_, device=gpu)
    _abi.mx_state_update(*st, x.to(gpu), dt.to(gpu), None, A.to(gpu), B.to(gpu), C.to(gpu), None,
                         None, out2, 8, False, 1)
    rq2, re2, rm2, ry2, _ = omx.mx_update(rq, re_, rm, x, dt, A, B, C, format_bits=8,
                                          round_mode=1)
    assert_close_rel(out2.cpu(), ry2, what="y (A per element)")


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("n", [64, 96, 128, 256])
def test_update_counter_mode_nonzero_dt(gpu, path, diag, fb, n):
    """Counter-mode writeback after a real update on the row kernel's layout (d_state 64, 128,
    256, and 96 on the general kernel): y within 2e-3, the state equal to the oracle's except
    at encoder decision ties (one level at most); P = 40 leaves a partly filled last row
    group."""
    if n == 96:
        diag.clear("LQ_MX_REQUIRE_ROWS")
    bsz, nh, p_, ng = 2, 8, 40, 2
    shape = (bsz, nh, p_, n)
    h0 = _state(shape, 90 + fb + n)
    q, e, m = omx.mx_encode(h0.numpy(), fb, 0)
    t = _inputs(bsz, nh, p_, n, ng, 91, gpu, head_dt=True)
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(bsz, nh, p_, device=gpu)
    off = 16 * 12345
    _abi.mx_state_update(*st, t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"], t["D"], None,
                         out, fb, True, 3, seed=5, rng_offset=off)
    c = _cpu(t)
    rq, re_, rm, ry, rh = omx.mx_update(q, e, m, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                        D=c["D"], dt_bias=c["dt_bias"], dt_softplus=True,
                                        format_bits=fb, round_mode=3, seed=5, rng_offset=off)
    assert_close_rel(out.cpu(), ry, what="y")
    mag = update_term_magnitudes(omx.mx_decode(q, e, m), c["x"], c["dt"], c["A"], c["B"],
                                 c["C"], dt_bias=c["dt_bias"], dt_softplus=True)
    assert_mx_writeback([a.cpu().numpy() for a in st], (rq, re_, rm), rh, mag, fb, 3, seed=5,
                        rng_offset=off, what="state")


@pytest.mark.parametrize("off", [2**33 - 8192, 16 * 999 + 2])
def test_update_counter_offsets_general_kernel(gpu, off):
    """Offsets the row kernel declines (pair counters crossing 2^32 inside the launch; an offset
    not a multiple of 16) go to the general kernel: still bit-exact with dt = 0."""
    shape = (2, 8, 8, 128)
    h0 = _state(shape, 95)
    q, e, m = omx.mx_encode(h0.numpy(), 4, 0)
    t = _inputs(2, 8, 8, 128, 2, 96, gpu, dt_zero=True, head_dt=True)
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(2, 8, 8, device=gpu)
    _abi.mx_state_update(*st, t["x"], t["dt"], None, t["A"], t["B"], t["C"], None, None, out, 4,
                         False, 3, seed=6, rng_offset=off)
    c = _cpu(t)
    rq, re_, rm, _, _ = omx.mx_update(q, e, m, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                      format_bits=4, round_mode=3, seed=6, rng_offset=off)
    _assert_mx_equal(st, (rq, re_, rm))


@pytest.mark.parametrize("fb", [8, 4])
def test_counter_chain_module_api(gpu, fb):
    """allocate_state_kernel_cache + 5 chained updates with dt = 0 (pure re-encodes at rising
    counter offsets) stay bit-exact with the oracle chain."""
    shape = (2, 8, 4, 128)
    h0 = _state(shape, 60 + fb, torch.bfloat16)
    cache = ms.allocate_state_kernel_cache(h0.to(gpu), format_bits=fb)
    ref = omx.mx_encode(h0.float().numpy(), fb, 0)
    _assert_mx_equal((cache.q_state, cache.shared_exp, cache.micro_exp), ref)
    t = _inputs(2, 8, 4, 128, 2, 61, gpu, dt_zero=True, head_dt=True)
    c = _cpu(t)
    for step in range(5):
        y = ms.mx_state_selective_update(cache, t["x"], t["dt"], t["A"], t["B"], t["C"],
                                         D=t["D"], seed=77)
        rq, re_, rm, ry, _ = omx.mx_update(*ref, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                           D=c["D"], format_bits=fb,
                                           round_mode=omx.ROUND_SR_COUNTER, seed=77,
                                           rng_offset=step * int(np.prod(shape)))
        ref = (rq, re_, rm)
        _assert_mx_equal((cache.q_state, cache.shared_exp, cache.micro_exp), ref)
        assert y.dtype == torch.bfloat16
        assert_close_rel(y.float().cpu(), ry, rtol=8e-3, what=f"y step {step}")
    assert cache.step == 5
    deq = ms.dequantize_state_cache(cache)
    assert np.array_equal(deq.cpu().numpy(), omx.mx_decode(*ref))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("fb", [4])
def test_full_size_b64_dt_zero_bit_exact(gpu, fb):
    """Headline size (B=64, 128 heads x 64 x 128, the model's layout): counter-mode writeback
    bit-exact. (The numpy oracle needs about a minute here.)"""
    shape = (64, 128, 64, 128)
    gen = torch.Generator(device=gpu).manual_seed(70 + fb)
    h0 = torch.randn(shape, device=gpu, generator=gen) * 0.5
    st = _mx_tensors(shape, gpu)
    _abi.mx_encode(h0, *st, fb, 0)
    q0, e0, m0 = (a.cpu().numpy() for a in st)
    x = torch.randn(64, 128, 64, device=gpu, generator=gen).to(torch.bfloat16)
    dt = torch.zeros(64, 128, 1, device=gpu, dtype=torch.bfloat16).expand(64, 128, 64)
    A = (-torch.rand(128, device=gpu, generator=gen))[:, None, None].expand(128, 64, 128)
    B = torch.randn(64, 8, 128, device=gpu, generator=gen).to(torch.bfloat16)
    C = torch.randn(64, 8, 128, device=gpu, generator=gen).to(torch.bfloat16)
    out = torch.empty(64, 128, 64, device=gpu, dtype=torch.bfloat16)
    off = 3 * int(np.prod(shape))
    _abi.mx_state_update(*st, x, dt, None, A, B, C, None, None, out, fb, False, 3, seed=1234,
                         rng_offset=off)
    torch.cuda.synchronize()
    h = omx.mx_decode(q0, e0, m0)
    ref = omx.mx_encode(h, fb, omx.ROUND_SR_COUNTER, seed=1234, rng_offset=off)
    _assert_mx_equal(st, ref)


@pytest.mark.parametrize("fb", [4, 8])
def test_full_size_b64_uniform_update_sampled_groups(gpu, fb):
    """Headline size (B=64, 128 heads x 64 x 128, 8 groups, the model's layout) with a real update
    (softplus dt, decay, B x, y with D) and the supplied-uniform writeback: three (batch, group)
    slices of 16 heads against the oracle run on the same slices of the inputs."""
    bsz, nh, p_, n, ng = 64, 128, 64, 128, 8
    shape = (bsz, nh, p_, n)
    gen = torch.Generator(device=gpu).manual_seed(640 + fb)
    h0 = torch.randn(shape, device=gpu, generator=gen) * 0.5
    st = _mx_tensors(shape, gpu)
    _abi.mx_encode(h0, *st, fb, 0)
    del h0
    st0 = [a.clone() for a in st]
    x = torch.randn(bsz, nh, p_, device=gpu, generator=gen).to(torch.bfloat16)
    dt = torch.randn(bsz, nh, 1, device=gpu, generator=gen).to(torch.bfloat16).expand(bsz, nh, p_)
    A = (-torch.exp(torch.rand(nh, device=gpu, generator=gen) * 2))[:, None, None].expand(nh, p_, n)
    B = torch.randn(bsz, ng, n, device=gpu, generator=gen).to(torch.bfloat16)
    C = torch.randn(bsz, ng, n, device=gpu, generator=gen).to(torch.bfloat16)
    D = torch.randn(nh, device=gpu, generator=gen)[:, None].expand(nh, p_)
    dt_bias = (torch.randn(nh, device=gpu, generator=gen) * 0.1)[:, None].expand(nh, p_)
    uni = torch.rand(shape, device=gpu, generator=gen)
    out = torch.empty(bsz, nh, p_, device=gpu)
    _abi.mx_state_update(*st, x, dt, dt_bias, A, B, C, D, None, out, fb, True,
                         _abi.ROUND_SR_UNIFORM, uniform=uni)
    torch.cuda.synchronize()
    hpg = nh // ng
    for b, g in [(0, 0), (63, 7), (31, 3)]:
        bs, hs = slice(b, b + 1), slice(g * hpg, (g + 1) * hpg)
        q, e, m = (a[bs, hs].cpu().numpy() for a in st0)
        args = (x[bs, hs].cpu(), dt[bs, hs].cpu(), A[hs].cpu(), B[bs, g:g + 1].cpu(),
                C[bs, g:g + 1].cpu())
        rq, re_, rm, ry, rh = omx.mx_update(
            q, e, m, *args, D=D[hs].cpu(), dt_bias=dt_bias[hs].cpu(), dt_softplus=True,
            format_bits=fb, round_mode=2, uniform=uni[bs, hs].cpu())
        assert_close_rel(out[bs, hs].cpu(), ry, what=f"y b{b} g{g}")
        mag = update_term_magnitudes(omx.mx_decode(q, e, m), *args, dt_bias=dt_bias[hs].cpu(),
                                     dt_softplus=True)
        assert_mx_writeback([a[bs, hs].cpu().numpy() for a in st], (rq, re_, rm), rh, mag, fb,
                            2, uniform=uni[bs, hs].cpu(), what=f"state b{b} g{g}")


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("mode", [_abi.ROUND_SR_UNIFORM, _abi.ROUND_SR_COUNTER,
                                  _abi.ROUND_SR_PHILOX])
def test_config3_batch1_full_layer_every_group(gpu, diag, fb, mode):
    """BASELINE configs 3 (MX8) and 4 (MX4) at batch 1 on the full Nemotron-H layer (128 heads x
    64 x 128, 8 groups): h0 ~ N(0, 0.5) encoded by the initial encoder, x ~ N(0, 1),
    dt = softplus(N(0, 1)) per head (passed with dt_softplus off), A = -exp(U(0, 2)), B, C ~ N(0, 1)
    per group, D ~ N(0, 1); the seeded supplied-uniform writeback (the configurations' own
    rounding), the counter generator, or the reference's own tl.rand stream (Philox); the
    model's layout, so the row kernel (required). The
    whole state -- every group -- against the oracle: y within 2e-3, the writeback to the
    assert_mx_writeback bar."""
    diag.set("LQ_MX_REQUIRE_ROWS")
    bsz, nh, p_, n, ng = 1, 128, 64, 128, 8
    shape = (bsz, nh, p_, n)
    g = torch.Generator().manual_seed(300 + fb + mode)
    h0 = torch.randn(shape, generator=g) * 0.5
    t = dict(
        x=torch.randn(bsz, nh, p_, generator=g).to(torch.bfloat16),
        dt=torch.nn.functional.softplus(torch.randn(bsz, nh, 1, generator=g)).expand(bsz, nh, p_),
        A=(-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n),
        B=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        C=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        D=torch.randn(nh, generator=g)[:, None].expand(nh, p_),
    )
    uni = torch.rand(shape, generator=g) if mode == _abi.ROUND_SR_UNIFORM else None
    dev = {k: to_device(v, gpu) for k, v in t.items()}
    st = _mx_tensors(shape, gpu)
    _abi.mx_encode(h0.to(gpu), *st, fb, _abi.ROUND_NEAREST_EVEN)
    q0, e0, m0 = (a.cpu().numpy() for a in st)
    assert all(np.array_equal(a, b) for a, b in zip((q0, e0, m0), omx.mx_encode(h0.numpy(), fb)))
    out = torch.empty(bsz, nh, p_, device=gpu)
    seed, off = 1234, 7 * int(np.prod(shape))
    _abi.mx_state_update(*st, dev["x"], dev["dt"], None, dev["A"], dev["B"], dev["C"], dev["D"],
                         None, out, fb, False, mode, None if uni is None else uni.to(gpu),
                         seed=seed, rng_offset=off)
    torch.cuda.synchronize()
    args = (t["x"], t["dt"], t["A"], t["B"], t["C"])
    rq, re_, rm, ry, rh = omx.mx_update(q0, e0, m0, *args, D=t["D"], format_bits=fb,
                                        round_mode=mode, uniform=uni, seed=seed, rng_offset=off)
    assert_close_rel(out.cpu(), ry, what=f"y mx{fb} mode {mode}")
    mag = update_term_magnitudes(omx.mx_decode(q0, e0, m0), *args)
    assert_mx_writeback([a.cpu().numpy() for a in st], (rq, re_, rm), rh, mag, fb, mode,
                        uniform=uni, seed=seed, rng_offset=off, what=f"state mx{fb} mode {mode}")


@pytest.mark.parametrize("mode", [_abi.ROUND_SR_COUNTER, _abi.ROUND_SR_PHILOX])
@pytest.mark.parametrize("fb", [4, 8])
def test_counter_offsets_crossing_a_high_word_row_kernel(gpu, diag, fb, mode):
    """Offsets whose counters cross a 2^32 boundary of their high word inside one launch (the
    row kernel switches the per-block hash of the high word where the low word carries; the
    Philox counter's second word steps by one there): the dt = 0 writeback is bit-exact against
    the oracle, through the host offset and through a device step
    (lq_mx_state_update_device_step) giving the same offset."""
    diag.set("LQ_MX_REQUIRE_ROWS")
    shape = (2, 4, 16, 128)
    T = int(np.prod(shape))
    h0 = _state(shape, 500 + fb)
    t = _inputs(2, 4, 16, 128, 2, 501, gpu, dt_zero=True, head_dt=True)
    st0 = _mx_tensors(shape, gpu)
    _abi.mx_encode(h0.to(gpu), *st0, fb, 0)
    q0, e0, m0 = (a.cpu().numpy() for a in st0)
    base = (1 << 33) - T // 2 - 5 * T  # at step 5 the pair counters run from 2^32 - T/4 over 2^32
    step = torch.tensor([5], dtype=torch.int64, device=gpu)
    for how in ("host", "device"):
        st = [a.clone() for a in st0]
        out = torch.empty(2, 4, 16, device=gpu)
        if how == "host":
            _abi.mx_state_update(*st, t["x"], t["dt"], None, t["A"], t["B"], t["C"], None, None,
                                 out, fb, False, mode, seed=77, rng_offset=base + 5 * T)
        else:
            _abi.mx_state_update(*st, t["x"], t["dt"], None, t["A"], t["B"], t["C"], None, None,
                                 out, fb, False, mode, seed=77, rng_offset=base, step=step)
        torch.cuda.synchronize()
        ref = omx.mx_encode(omx.mx_decode(q0, e0, m0), fb, mode, seed=77,
                            rng_offset=base + 5 * T)
        _assert_mx_equal(st, ref)


@pytest.mark.parametrize("fb", [8, 4])
@pytest.mark.parametrize("n", [64, 128, 96])
def test_update_philox_mode_nonzero_dt(gpu, path, diag, fb, n):
    """The reference's own rounding stream (LQ_ROUND_SR_PHILOX: u = tl.rand(seed, offset) per
    element, the u < frac test) after a real update, on the row kernel's layout (d_state 64, 128;
    96 on the general kernel) and with the general kernel forced: y within 2e-3, the state equal
    to the oracle's except at encoder decision ties. The offsets run across 2^32 inside the
    launch, so the counter's second word changes between rows."""
    if n == 96:
        diag.clear("LQ_MX_REQUIRE_ROWS")
    bsz, nh, p_, ng = 2, 8, 40, 2
    shape = (bsz, nh, p_, n)
    h0 = _state(shape, 700 + fb + n)
    q, e, m = omx.mx_encode(h0.numpy(), fb, 0)
    t = _inputs(bsz, nh, p_, n, ng, 701, gpu, head_dt=True)
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(bsz, nh, p_, device=gpu)
    off = (1 << 32) - int(np.prod(shape)) // 3
    _abi.mx_state_update(*st, t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"], t["D"], None,
                         out, fb, True, _abi.ROUND_SR_PHILOX, seed=1234, rng_offset=off)
    c = _cpu(t)
    rq, re_, rm, ry, rh = omx.mx_update(q, e, m, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                        D=c["D"], dt_bias=c["dt_bias"], dt_softplus=True,
                                        format_bits=fb, round_mode=omx.ROUND_SR_PHILOX,
                                        seed=1234, rng_offset=off)
    assert_close_rel(out.cpu(), ry, what="y")
    mag = update_term_magnitudes(omx.mx_decode(q, e, m), c["x"], c["dt"], c["A"], c["B"],
                                 c["C"], dt_bias=c["dt_bias"], dt_softplus=True)
    assert_mx_writeback([a.cpu().numpy() for a in st], (rq, re_, rm), rh, mag, fb,
                        omx.ROUND_SR_PHILOX, seed=1234, rng_offset=off, what="state")


@pytest.mark.parametrize("fb", [8, 4])
def test_philox_chain_module_api(gpu, fb):
    """mx_state_selective_update(..., rng="philox"), 5 chained updates with dt = 0 (pure
    re-encodes at the reference's offsets step*B*H*P*N, seed 1234 as the reference's default):
    bit-exact with the oracle chain drawing tl.rand's stream."""
    shape = (2, 8, 4, 128)
    h0 = _state(shape, 720 + fb, torch.bfloat16)
    cache = ms.allocate_state_kernel_cache(h0.to(gpu), format_bits=fb)
    ref = omx.mx_encode(h0.float().numpy(), fb, 0)
    t = _inputs(2, 8, 4, 128, 2, 721, gpu, dt_zero=True, head_dt=True)
    c = _cpu(t)
    for step in range(5):
        ms.mx_state_selective_update(cache, t["x"], t["dt"], t["A"], t["B"], t["C"], D=t["D"],
                                     rng="philox")
        rq, re_, rm, _, _ = omx.mx_update(*ref, c["x"], c["dt"], c["A"], c["B"], c["C"],
                                          D=c["D"], format_bits=fb,
                                          round_mode=omx.ROUND_SR_PHILOX, seed=1234,
                                          rng_offset=step * int(np.prod(shape)))
        ref = (rq, re_, rm)
        _assert_mx_equal((cache.q_state, cache.shared_exp, cache.micro_exp), ref)
    assert cache.step == 5


@pytest.mark.timeout(300)
def test_full_size_b64_philox_dt_zero_sampled_slices(gpu, diag):
    """Headline size (B=64, 128 heads x 64 x 128, MX4, the model's layout, the row kernel) with
    the reference's stream at step 40 (offset 40*B*H*P*N, past 2^31, where the reference's int32
    offsets no longer compile): the dt = 0 writeback of three (batch, head) slices bit-exact
    against the oracle, each slice drawing offsets from (b*H + h)*P*N on."""
    diag.set("LQ_MX_REQUIRE_ROWS")
    bsz, nh, p_, n = 64, 128, 64, 128
    shape = (bsz, nh, p_, n)
    gen = torch.Generator(device=gpu).manual_seed(730)
    h0 = torch.randn(shape, device=gpu, generator=gen) * 0.5
    st = _mx_tensors(shape, gpu)
    _abi.mx_encode(h0, *st, 4, 0)
    del h0
    st0 = [a.clone() for a in st]
    x = torch.randn(bsz, nh, p_, device=gpu, generator=gen).to(torch.bfloat16)
    dt = torch.zeros(bsz, nh, 1, device=gpu, dtype=torch.bfloat16).expand(bsz, nh, p_)
    A = (-torch.rand(nh, device=gpu, generator=gen))[:, None, None].expand(nh, p_, n)
    B = torch.randn(bsz, 8, n, device=gpu, generator=gen).to(torch.bfloat16)
    C = torch.randn(bsz, 8, n, device=gpu, generator=gen).to(torch.bfloat16)
    out = torch.empty(bsz, nh, p_, device=gpu, dtype=torch.bfloat16)
    off = 40 * int(np.prod(shape))
    _abi.mx_state_update(*st, x, dt, None, A, B, C, None, None, out, 4, False,
                         _abi.ROUND_SR_PHILOX, seed=1234, rng_offset=off)
    torch.cuda.synchronize()
    for b, h in [(0, 0), (63, 127), (17, 90)]:
        q, e, m = (a[b, h].cpu().numpy() for a in st0)
        ref = omx.mx_encode(omx.mx_decode(q, e, m), 4, omx.ROUND_SR_PHILOX, seed=1234,
                            rng_offset=off + (b * nh + h) * p_ * n)
        _assert_mx_equal([a[b, h] for a in st], ref)
