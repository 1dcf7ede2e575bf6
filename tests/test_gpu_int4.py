"""GPU parity of the INT4 KV path through the C ABI: the pack is bit-exact against the oracle;
attention (MFMA fast path and generic path) is within 2e-3 of the float64 oracle."""
import pytest
import torch

from helpers import assert_close_rel, fast_attention_expected, require_env
from layer_quant_amd import _abi
from hybrid_quant import int4_8b_attention as ia
from oracle import int4_kv as oik

pytestmark = pytest.mark.gpu


def _activations(shape, seed, dtype=torch.bfloat16, outliers=True):
    """~N(0,1) with about 1% of head_dim channels scaled by 8 (shared across tokens)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen)
    if outliers:
        chan = torch.rand(shape[1], shape[-1], generator=gen) < 0.01
        x = torch.where(chan[None, :, None, :] if x.dim() == 4 else chan[None], x * 8, x)
    return x.to(dtype)


@pytest.mark.parametrize("g", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_pack_bit_exact(gpu, g, dtype):
    b, h, t, d, cap = 3, 8, 5, 128, 32
    x = _activations((b, h, t, d), 100 + g, dtype)
    pos = torch.tensor([0, 7, 8, 31, 12])
    packed = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8, device=gpu)
    scale = torch.full((b, h, cap, d // g), -1.0, device=gpu)
    _abi.int4_pack_kv(x.to(gpu), packed, scale, pos.to(gpu), g)
    torch.cuda.synchronize()
    ref_p = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8)
    ref_s = torch.full((b, h, cap, d // g), -1.0)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(packed.cpu(), ref_p)
    assert torch.equal(scale.cpu(), ref_s)


@pytest.mark.parametrize("g,d", [(48, 96), (6, 96), (256, 256)])
def test_pack_bit_exact_other_groups(gpu, g, d):
    """Groups whose g/2 is not a power of two up to 64 take the one-thread-per-group kernel."""
    b, h, t, cap = 2, 3, 4, 16
    x = _activations((b, h, t, d), 200 + g)
    pos = torch.tensor([3, 0, 15, 9])
    packed = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8, device=gpu)
    scale = torch.full((b, h, cap, d // g), -1.0, device=gpu)
    _abi.int4_pack_kv(x.to(gpu), packed, scale, pos.to(gpu), g)
    ref_p = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8)
    ref_s = torch.full((b, h, cap, d // g), -1.0)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(packed.cpu(), ref_p)
    assert torch.equal(scale.cpu(), ref_s)


@pytest.mark.parametrize("g,t,dtype", [(32, 1, torch.bfloat16), (64, 5, torch.float32),
                                       (128, 1, torch.float16), (48, 3, torch.bfloat16)])
def test_pack_pair_equals_two_single_packs(gpu, g, t, dtype):
    """lq_int4_pack_kv_pair writes exactly what two lq_int4_pack_kv calls write, including a V
    given as a transposed view (different strides from K); g = 48 takes the per-group kernel."""
    b, hkv, d, cap = 3, 8, 96 if g == 48 else 128, 12
    k = _activations((b, hkv, t, d), 40 + g, dtype).to(gpu)
    v = _activations((b, t, hkv, d), 50 + g, dtype).to(gpu).transpose(1, 2)
    pos = torch.tensor([2, 7, 0, 11, 5][:t], device=gpu)
    outs = []
    for pair in (True, False):
        kp = torch.full((b, hkv, cap, d // 2), 0x5A, dtype=torch.uint8, device=gpu)
        vp = torch.full_like(kp, 0xA5)
        ks = torch.full((b, hkv, cap, d // g), -1.0, device=gpu)
        vs = torch.full_like(ks, -2.0)
        if pair:
            _abi.int4_pack_kv_pair(k, v, kp, vp, ks, vs, pos, g)
        else:
            _abi.int4_pack_kv(k, kp, ks, pos, g)
            _abi.int4_pack_kv(v, vp, vs, pos, g)
        torch.cuda.synchronize()
        outs.append((kp.cpu(), vp.cpu(), ks.cpu(), vs.cpu()))
    for a_, b_ in zip(*outs):
        assert torch.equal(a_, b_)
    ref = oik.allocate_cache(b, hkv, cap, d, g)
    oik.pack_into(ref["k_packed"], ref["k_scale"], k.cpu(), pos.cpu(), g)
    oik.pack_into(ref["v_packed"], ref["v_scale"], v.cpu(), pos.cpu(), g)
    rows = pos.cpu()
    assert torch.equal(outs[0][0][:, :, rows], ref["k_packed"][:, :, rows])
    assert torch.equal(outs[0][1][:, :, rows], ref["v_packed"][:, :, rows])
    assert torch.equal(outs[0][2][:, :, rows], ref["k_scale"][:, :, rows])
    assert torch.equal(outs[0][3][:, :, rows], ref["v_scale"][:, :, rows])


def test_pack_edge_values(gpu):
    d, g = 128, 32
    x = torch.zeros(1, 1, 4, d)
    x[0, 0, 1, :8] = torch.tensor([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5])  # exact ties
    x[0, 0, 2] = torch.randn(d) * 1e-30                                          # tiny values
    x[0, 0, 3] = torch.randn(d) * 3e37                                           # huge values
    pos = torch.arange(4)
    packed = torch.zeros(1, 1, 4, d // 2, dtype=torch.uint8, device=gpu)
    scale = torch.zeros(1, 1, 4, d // g, device=gpu)
    _abi.int4_pack_kv(x.to(gpu), packed, scale, pos.to(gpu), g)
    ref_p = torch.zeros(1, 1, 4, d // 2, dtype=torch.uint8)
    ref_s = torch.zeros(1, 1, 4, d // g)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(packed.cpu(), ref_p) and torch.equal(scale.cpu(), ref_s)
    assert ref_s[0, 0, 0, 0].item() == torch.tensor(1e-8).item()


@pytest.mark.parametrize("g", [16, 32, 64, 128])
def test_pack_edge_values_prompt_sized(gpu, g):
    """The edge rows of test_pack_edge_values (a zero token, exact ties, 1e-30 and 3e37 values)
    inside a prompt of 64 tokens, so that the group-per-lane kernel (g 16 / 32 / 64) and the row
    kernel (g 128) quantise them: bit-exact against the oracle."""
    d, t = 128, 64
    gen = torch.Generator().manual_seed(g)
    x = torch.randn(2, 2, t, d, generator=gen)
    x[0, 0, 0] = 0
    x[0, 0, 1, :8] = torch.tensor([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5])
    x[0, 1, 2] = torch.randn(d, generator=gen) * 1e-30
    x[1, 0, 3] = torch.randn(d, generator=gen) * 3e37
    x[1, 1, 5, ::g] = 7.0 * 2.0 ** -130  # a subnormal group maximum
    pos = torch.arange(t)
    packed = torch.zeros(2, 2, t, d // 2, dtype=torch.uint8, device=gpu)
    scale = torch.zeros(2, 2, t, d // g, device=gpu)
    _abi.int4_pack_kv(x.to(gpu), packed, scale, pos.to(gpu), g)
    ref_p = torch.zeros(2, 2, t, d // 2, dtype=torch.uint8)
    ref_s = torch.zeros(2, 2, t, d // g)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(packed.cpu(), ref_p) and torch.equal(scale.cpu(), ref_s)


@pytest.mark.parametrize("g,d", [(8, 128), (16, 128), (32, 128), (64, 128), (128, 128),
                                 (256, 256), (32, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_pack_prompt_sized_bit_exact(gpu, g, d, dtype):
    """A prompt's worth of tokens per (batch, head) (96, shuffled positions, outlier channels,
    a token of zeros): the group-per-lane kernel (g 16 / 32 / 64) and the 8-values-per-lane row
    kernel (other g), both bit-exact against the oracle, K and V in one pair call; V given as the
    model's transposed view ([B, L, Hkv, D] -> [B, Hkv, L, D])."""
    b, h, t = 2, 3, 96
    k = _activations((b, h, t, d), 300 + g + d, dtype)
    v = _activations((b, t, h, d), 400 + g + d, dtype).transpose(1, 2)
    k[1, 2, 5] = 0
    pos = torch.randperm(t, generator=torch.Generator().manual_seed(g))
    cap = t + 4
    kp = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8, device=gpu)
    vp = torch.full_like(kp, 0xCD)
    ks = torch.full((b, h, cap, d // g), -1.0, device=gpu)
    vs = torch.full_like(ks, -2.0)
    _abi.int4_pack_kv_pair(k.to(gpu), v.to(gpu), kp, vp, ks, vs, pos.to(gpu), g)
    ref_kp = torch.full((b, h, cap, d // 2), 0xAB, dtype=torch.uint8)
    ref_vp = torch.full_like(ref_kp, 0xCD)
    ref_ks = torch.full((b, h, cap, d // g), -1.0)
    ref_vs = torch.full_like(ref_ks, -2.0)
    oik.pack_into(ref_kp, ref_ks, k, pos, g)
    oik.pack_into(ref_vp, ref_vs, v, pos, g)
    assert torch.equal(kp.cpu(), ref_kp) and torch.equal(vp.cpu(), ref_vp)
    assert torch.equal(ks.cpu(), ref_ks) and torch.equal(vs.cpu(), ref_vs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pack_near_ties_bit_exact(gpu, dtype):
    """Values whose quotient by the group scale lies within 2^-24 .. 2^-12 of a half-integer
    (both sides), under 256 different non-power-of-two scales: the row kernel's product with the
    reciprocal, and its IEEE-division fallback near half-integers, give the oracle's levels."""
    gen = torch.Generator().manual_seed(77)
    rows, d, g = 256, 128, 32
    s = (torch.rand(rows, d // g, 1, generator=gen) * 3 + 0.1)  # target scales
    k = torch.randint(-7, 7, (rows, d // g, g), generator=gen).float()
    dl = 2.0 ** -torch.randint(12, 25, (rows, d // g, g), generator=gen).float()
    sign = torch.where(torch.rand(rows, d // g, g, generator=gen) < 0.5, -1.0, 1.0)
    x = (k + 0.5 + sign * dl) * s
    x[:, :, 0] = 7.0 * s[:, :, 0]  # the group's absmax: scale = RN(7 s / 7)
    x = x.reshape(1, 1, rows, d).to(dtype)
    pos = torch.arange(rows)
    packed = torch.zeros(1, 1, rows, d // 2, dtype=torch.uint8, device=gpu)
    scale = torch.zeros(1, 1, rows, d // g, device=gpu)
    _abi.int4_pack_kv(x.to(gpu), packed, scale, pos.to(gpu), g)
    ref_p = torch.zeros(1, 1, rows, d // 2, dtype=torch.uint8)
    ref_s = torch.zeros(1, 1, rows, d // g)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(scale.cpu(), ref_s)
    assert torch.equal(packed.cpu(), ref_p)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_unaligned_rows_take_the_lane_kernel(gpu, dtype):
    """Token rows that are not 16-byte aligned (a view starting one element into wider rows)
    take the one-lane-per-byte kernel; both layouts give the oracle's bytes, and a prompt-sized
    pair call (batch 1, 8 KV heads, 4096 tokens, aligned) takes the row kernel."""
    d, g = 128, 32
    wide = _activations((2, 4, 6, d + 1), 90, dtype)
    x = wide[..., 1:]  # data pointer 2 bytes past a 16-byte boundary
    pos = torch.tensor([5, 1, 0, 3, 2, 4])
    packed = torch.zeros(2, 4, 6, d // 2, dtype=torch.uint8, device=gpu)
    scale = torch.zeros(2, 4, 6, d // g, device=gpu)
    _abi.int4_pack_kv(wide.to(gpu)[..., 1:], packed, scale, pos.to(gpu), g)
    ref_p = torch.zeros(2, 4, 6, d // 2, dtype=torch.uint8)
    ref_s = torch.zeros(2, 4, 6, d // g)
    oik.pack_into(ref_p, ref_s, x, pos, g)
    assert torch.equal(packed.cpu(), ref_p) and torch.equal(scale.cpu(), ref_s)
    t = 4096
    k = _activations((1, 8, t, d), 91, dtype)
    v = _activations((1, 8, t, d), 92, dtype)
    pos = torch.arange(t)
    kp = torch.zeros(1, 8, t, d // 2, dtype=torch.uint8, device=gpu)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(1, 8, t, d // g, device=gpu)
    vs = torch.zeros_like(ks)
    _abi.int4_pack_kv_pair(k.to(gpu), v.to(gpu), kp, vp, ks, vs, pos.to(gpu), g)
    ref = oik.allocate_cache(1, 8, t, d, g)
    oik.pack_kv_into_cache(ref, k, v, pos, g)
    assert torch.equal(kp.cpu(), ref["k_packed"]) and torch.equal(vp.cpu(), ref["v_packed"])
    assert torch.equal(ks.cpu(), ref["k_scale"]) and torch.equal(vs.cpu(), ref["v_scale"])


def _packed_cache(b, hkv, s, d, g, seed, cap=None):
    cap = cap or s
    cache = oik.allocate_cache(b, hkv, cap, d, g)
    k = _activations((b, hkv, s, d), seed, torch.bfloat16)
    v = _activations((b, hkv, s, d), seed + 1, torch.bfloat16)
    oik.pack_kv_into_cache(cache, k, v, torch.arange(s), g)
    return cache


def _run_attention(gpu, cache, q, s, nrep, g, mask=None, out_dtype=torch.float32):
    """One call; a call whose shape and dtype pass the MFMA gate must take the MFMA kernel."""
    dev = {k: v.to(gpu) for k, v in cache.items() if torch.is_tensor(v)}
    out = torch.empty(q.shape[0], q.shape[1], q.shape[-1], dtype=out_dtype, device=gpu)
    with require_env("LQ_ATTN_REQUIRE_FAST", fast_attention_expected(q.dtype, q.shape[-1], g, nrep)):
        _abi.int4_decode_attention(q.to(gpu), dev["k_packed"], dev["v_packed"], dev["k_scale"],
                                   dev["v_scale"], None if mask is None else mask.to(gpu), out,
                                   s, nrep, g)
    torch.cuda.synchronize()
    return out.cpu()


ATTN_CASES = [
    # b, hkv, nrep, s, g
    (1, 8, 4, 1024, 32),   # the CPU reference config shape
    (2, 8, 4, 1, 32),
    (3, 2, 4, 37, 32),
    (2, 4, 4, 1000, 64),
    (2, 2, 4, 333, 128),
    (2, 4, 2, 200, 32),
    (1, 2, 1, 513, 32),
    (2, 2, 8, 129, 64),
    (1, 1, 16, 77, 128),
    (2, 8, 4, 4133, 32),
]


@pytest.mark.parametrize("b,hkv,nrep,s,g", ATTN_CASES)
def test_attention_parity_fast_and_generic(gpu, b, hkv, nrep, s, g):
    d = 128
    cache = _packed_cache(b, hkv, s, d, g, 200 + s, cap=s + 3)
    q = _activations((b, hkv * nrep, 1, d), 300 + s, torch.bfloat16)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g)
    fast = _run_attention(gpu, cache, q, s, nrep, g)            # bf16 q: MFMA path
    generic = _run_attention(gpu, cache, q.float(), s, nrep, g)  # fp32 q: generic path
    assert_close_rel(fast, ref, what="fast")
    assert_close_rel(generic, ref, what="generic")


@pytest.mark.parametrize("b,hkv,nrep,s,g,d", [(2, 2, 4, 300, 16, 128), (1, 4, 2, 150, 32, 64),
                                              (2, 1, 3, 70, 64, 256)])
def test_attention_generic_shapes(gpu, b, hkv, nrep, s, g, d):
    cache = _packed_cache(b, hkv, s, d, g, 400 + d)
    q = _activations((b, hkv * nrep, 1, d), 500 + d, torch.bfloat16)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g)
    assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g), ref)


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
def test_attention_masks(gpu, qdtype):
    b, hkv, nrep, s, g, d = 3, 2, 4, 700, 32, 128
    cache = _packed_cache(b, hkv, s, d, g, 600)
    q = _activations((b, hkv * nrep, 1, d), 601).to(qdtype)
    keep = torch.ones(b, s + 5, dtype=torch.bool)
    keep[0, :100] = False          # left padding longer than a key tile
    keep[1, 5:9] = False
    keep[2, -300:-200] = False
    mask = oik.decode_attention_mask(keep, b, s)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g, mask=mask)
    assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g, mask=mask), ref, what="keep")
    bias = torch.randn(b, 1, 4, s) * 2
    fmask = oik.decode_attention_mask(bias, b, s)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g, mask=fmask)
    assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g, mask=fmask), ref, what="bias")
    short = torch.zeros(b, 1, 1, 450)  # keys at or beyond the mask length are excluded
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g, mask=short)
    assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g, mask=short), ref, what="short")


def test_attention_bf16_output(gpu):
    b, hkv, nrep, s, g, d = 2, 8, 4, 2048, 32, 128
    cache = _packed_cache(b, hkv, s, d, g, 700)
    q = _activations((b, hkv * nrep, 1, d), 701)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g)
    out = _run_attention(gpu, cache, q, s, nrep, g, out_dtype=torch.bfloat16)
    assert_close_rel(out.float(), ref, rtol=8e-3, what="bf16 out")


@pytest.mark.parametrize("s,g", [(999, 32), (1057, 64), (805, 128)])
def test_attention_long_wave_ranges_ragged_tail(gpu, s, g):
    """B * Hkv = 512 (one resident generation of 2048 waves, one split): each (batch, KV head)
    workgroup deals its 32, 34 or 26 tiles of 32 keys to its 4 waves in turn, 7-9 per wave through
    the 3-buffer LDS ring; the ragged last tile (S % 32 = 7, 1, 5) is the wave's tile 7, 8 or 6,
    i.e. ring position 1, 2 or 0."""
    b, hkv, nrep, d = 64, 8, 4, 128
    cache = _packed_cache(b, hkv, s, d, g, 1200 + s, cap=s + 5)
    q = _activations((b, hkv * nrep, 1, d), 1300 + s, torch.bfloat16)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g)
    assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g), ref, what="fast")


def _long_range_masks(b, s):
    """Masks for B=64 at S ~ 800-1060, where each wave of the MFMA path takes every fourth 32-key
    tile of its (batch, KV head): a keep-mask whose left padding covers the first 9-10 tiles,
    i.e. two or more of every wave's tiles (rows 0-7: 300-307 keys), padding inside one tile and
    a gap across a tile edge in other rows; a 4-D additive bias; and a short bias mask that ends
    inside a tile (700 keys), so that later tiles of every wave are fully masked."""
    gen = torch.Generator().manual_seed(s)
    keep = torch.ones(b, s, dtype=torch.bool)
    for r in range(8):
        keep[r, :300 + r] = False
    keep[8:16, :17] = False
    keep[16:24, 500:540] = False
    keep[24, s - 1] = False
    return {
        "keep": oik.decode_attention_mask(keep, b, s),
        "bias": oik.decode_attention_mask(torch.randn(b, 1, 1, s, generator=gen) * 3, b, s),
        "short": torch.randn(b, 1, 1, 700, generator=gen),
    }


@pytest.mark.parametrize("s,g", [(999, 32), (1057, 64), (805, 128)])
def test_attention_long_wave_ranges_masked(gpu, s, g):
    """The masked MFMA instance (7 LDS-direct loads per tile) through the whole 3-buffer ring and
    the ragged last tile of each ring position, with masks that end or open inside a wave."""
    b, hkv, nrep, d = 64, 8, 4, 128
    cache = _packed_cache(b, hkv, s, d, g, 1400 + s, cap=s + 5)
    q = _activations((b, hkv * nrep, 1, d), 1450 + s, torch.bfloat16)
    for name, mask in _long_range_masks(b, s).items():
        ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                                   cache["v_scale"], s, nrep, g, mask=mask)
        assert_close_rel(_run_attention(gpu, cache, q, s, nrep, g, mask=mask), ref, what=name)


@pytest.mark.parametrize("b,hkv,nrep,s,g,masked", [(64, 8, 4, 4096, 32, False),
                                                   (8, 8, 4, 4133, 32, False),
                                                   (16, 8, 4, 2999, 64, False),
                                                   (2, 2, 16, 777, 128, False),
                                                   (64, 8, 4, 1057, 64, True),
                                                   (8, 8, 4, 4133, 32, True)])
def test_attention_repeats_bit_identical(gpu, diag, b, hkv, nrep, s, g, masked):
    """The MFMA path's tile loads land in LDS behind explicit waits: repeated calls on the same
    inputs must give bit-identical outputs (a missing or short wait would read a tile early).
    The masked instance counts 7 loads per tile in its waits."""
    diag.set("LQ_ATTN_REQUIRE_FAST")
    d = 128
    gen = torch.Generator(device=gpu).manual_seed(b * 7 + s)
    kp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    ks = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) + 0.01
    vs = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) + 0.01
    q = torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen).to(torch.bfloat16)
    mask = None
    if masked:
        mask = (torch.randn(b, 1, 1, s, device=gpu, generator=gen) * 2).contiguous()
        mask[:, :, :, :300] = float("-inf")
    ref = torch.empty(b, hkv * nrep, d, device=gpu)
    _abi.int4_decode_attention(q, kp, vp, ks, vs, mask, ref, s, nrep, g)
    out = torch.empty_like(ref)
    for _ in range(20):
        out.fill_(float("nan"))
        _abi.int4_decode_attention(q, kp, vp, ks, vs, mask, out, s, nrep, g)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    assert torch.isfinite(ref).all()


def test_attention_concurrent_streams(gpu, diag):
    """Split-K calls in flight on two streams at once use separate workspaces (one per stream):
    each stream's results equal the same calls made one at a time on the default stream."""
    diag.set("LQ_ATTN_REQUIRE_FAST")
    b, hkv, nrep, d, g = 2, 8, 4, 128, 32
    cases = []
    for i, s in enumerate((3000, 1777)):
        cache = _packed_cache(b, hkv, s, d, g, 1500 + i)
        dev = {k: v.to(gpu) for k, v in cache.items() if torch.is_tensor(v)}
        q = _activations((b, hkv * nrep, 1, d), 1600 + i).to(gpu)
        cases.append((dev, q, s))
    ref = []
    for dev, q, s in cases:
        out = torch.empty(b, hkv * nrep, d, device=gpu)
        _abi.int4_decode_attention(q, dev["k_packed"], dev["v_packed"], dev["k_scale"],
                                   dev["v_scale"], None, out, s, nrep, g)
        ref.append(out)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty_like(r) for _ in range(8)] for r in ref]
    for it in range(8):
        for (dev, q, s), st, o in zip(cases, streams, outs):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                _abi.int4_decode_attention(q, dev["k_packed"], dev["v_packed"], dev["k_scale"],
                                           dev["v_scale"], None, o[it], s, nrep, g)
    torch.cuda.synchronize()
    for r, o in zip(ref, outs):
        for x in o:
            assert torch.equal(x, r)


@pytest.mark.parametrize("b,s", [(64, 16384), (8, 4096)])
def test_attention_full_size_sampled_heads(gpu, diag, b, s):
    """BASELINE sizes: random packed cache built on the GPU, oracle on sampled (b, kv head)."""
    diag.set("LQ_ATTN_REQUIRE_FAST")
    hkv, nrep, d, g = 8, 4, 128, 32
    gen = torch.Generator(device=gpu).manual_seed(b + s)
    kp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    ks = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) * 0.5 + 0.05
    vs = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) * 0.5 + 0.05
    q = (torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen)).to(torch.bfloat16)
    out = torch.empty(b, hkv * nrep, d, device=gpu)
    _abi.int4_decode_attention(q, kp, vp, ks, vs, None, out, s, nrep, g)
    torch.cuda.synchronize()
    for bi, kv in [(0, 0), (b - 1, hkv - 1), (b // 2, 3)]:
        sl = slice(bi, bi + 1)
        ref = oik.decode_attention(q[sl, kv * nrep:(kv + 1) * nrep].cpu(),
                                   kp[sl, kv:kv + 1].cpu(), vp[sl, kv:kv + 1].cpu(),
                                   ks[sl, kv:kv + 1].cpu(), vs[sl, kv:kv + 1].cpu(), s, nrep, g)
        assert_close_rel(out[sl, kv * nrep:(kv + 1) * nrep].cpu(), ref, what=f"b{bi} kv{kv}")


def test_module_api_pack_then_attend(gpu):
    """_ensure_layer_cache -> _pack_kv_into_cache -> _decode_attention, token by token."""
    b, hkv, nrep, d, g, steps = 2, 8, 4, 128, 64, 40
    holder = type("Cache", (), {})()
    k_all = _activations((b, hkv, steps, d), 800)
    v_all = _activations((b, hkv, steps, d), 801)
    ref_cache = oik.allocate_cache(b, hkv, 64, d, g)
    for t in range(steps):
        cache = ia._ensure_layer_cache(holder, 0, b, hkv, t + 1, d, g, gpu)
        pos = torch.tensor([t], device=gpu)
        ia._pack_kv_into_cache(cache, k_all[:, :, t:t + 1].to(gpu), v_all[:, :, t:t + 1].to(gpu),
                               pos, g)
        oik.pack_kv_into_cache(ref_cache, k_all[:, :, t:t + 1], v_all[:, :, t:t + 1],
                               torch.tensor([t]), g)
    assert cache.length == steps and cache.k_packed.shape[2] == 64
    assert torch.equal(cache.k_packed[:, :, :steps].cpu(), ref_cache["k_packed"][:, :, :steps])
    assert torch.equal(cache.v_scale[:, :, :steps].cpu(), ref_cache["v_scale"][:, :, :steps])
    q = _activations((b, hkv * nrep, 1, d), 802)
    out = ia._decode_attention(q.to(gpu), cache, steps, nrep, g)
    assert out.dtype == torch.bfloat16 and out.shape == (b, hkv * nrep, d)
    ref = oik.decode_attention(q, ref_cache["k_packed"], ref_cache["v_packed"],
                               ref_cache["k_scale"], ref_cache["v_scale"], steps, nrep, g)
    assert_close_rel(out.float().cpu(), ref, rtol=8e-3)


def test_folded_split_merge_matches_merge_kernel_and_leaves_counters_zero(gpu, diag):
    """With LQ_ATTN_FOLD_MERGE, multi-split MFMA calls merge their partials in the kernel (the
    last workgroup of each (batch, KV head) to arrive): over shapes with 2-64 splits, masked and
    not, groups 32/64/128, 1-16 query heads per KV head (1 head: 128 splits' partials per thread in
    the merge), all through one reused workspace, the
    output equals the default two-launch form's (the same partials, merged by attn_merge_kernel,
    whose sums run in another order: within 1e-5 of the output's mean magnitude) and the
    oracle's, and after every call the workspace's arrival counters are all zero again."""
    diag.set("LQ_ATTN_REQUIRE_FAST")
    gen = torch.Generator(device=gpu).manual_seed(77)
    d = 128
    counter_words = (64 << 10) // 4
    ws = torch.zeros(4 << 20, dtype=torch.uint8, device=gpu)
    lib = _abi.lib()
    cases = [(1, 8, 4, 16384, 32, False), (8, 8, 4, 2072, 64, False), (2, 8, 4, 5000, 32, True),
             (1, 1, 16, 9000, 128, False), (3, 2, 8, 3001, 64, True), (1, 8, 2, 700, 32, False),
             (1, 8, 1, 16384, 32, False), (2, 4, 1, 4100, 64, True)]
    for b, hkv, nrep, s, g, masked in cases:
        need = lib.lq_int4_decode_attention_workspace(b, hkv * nrep, hkv, d, s, g)
        assert need > 64 << 10, (b, s, need)  # several splits
        kp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
        vp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
        ks = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) + 0.01
        vs = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) + 0.01
        q = torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen).to(torch.bfloat16)
        mask = None
        if masked:
            mask = torch.randn(b, 1, 1, s, device=gpu, generator=gen)
            mask[..., s // 3: s // 2] = float("-inf")
        outs = []
        for merge_kernel in (False, True):
            with _abi.diagnostic("LQ_ATTN_FOLD_MERGE", on=not merge_kernel):
                out = torch.full((b, hkv * nrep, d), float("nan"), device=gpu)
                rc = lib.lq_int4_decode_attention(
                    _abi.desc(q), _abi.desc(kp), _abi.desc(vp), _abi.desc(ks), _abi.desc(vs),
                    _abi.desc(mask), _abi.desc(out), s, nrep, g, ws.data_ptr(), ws.numel(),
                    torch.cuda.current_stream().cuda_stream)
                _abi.check(rc, "lq_int4_decode_attention")
                torch.cuda.synchronize()
                assert not ws[: counter_words * 4].view(torch.int32).any(), (b, s, merge_kernel)
                outs.append(out)
        assert torch.isfinite(outs[0]).all()
        scale = outs[1].abs().mean().item()
        torch.testing.assert_close(outs[0], outs[1], rtol=1e-5, atol=1e-5 * scale)
        ref = oik.decode_attention(q.cpu(), kp.cpu(), vp.cpu(), ks.cpu(), vs.cpu(), s, nrep, g,
                                   mask=None if mask is None else mask.cpu())
        assert_close_rel(outs[0], ref, what=f"folded merge b{b} s{s} g{g}")
