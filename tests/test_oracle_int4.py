"""Pins the CPU oracle of the INT4 KV path (oracle/int4_kv.py) with checks that do not restate
its formulas: exact representable groups, invariants, ties, an independent numpy path, a
per-element bit-layout loop, and torch's scaled_dot_product_attention as the attention
reference."""
import math

import numpy as np
import pytest
import torch

from oracle import int4_kv as ik


def test_exactly_representable_groups_recover_levels():
    gen = torch.Generator().manual_seed(1)
    for s in (0.25, 2.0 ** -10, 8.0):
        k = torch.randint(-7, 8, (64, 32), generator=gen)
        k[:, 0] = 7  # absmax = 7 s, so scale = s exactly
        x = k.float() * s
        q, scale = ik.quantize_groups(x, 32)
        assert torch.equal(scale, torch.full((64, 1), s))
        assert torch.equal(q.long(), k)


def test_invariants_on_random_data():
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(4, 8, 16, 128, generator=gen) * torch.rand(4, 8, 16, 1, generator=gen) * 10
    q, scale = ik.quantize_groups(x, 32)
    assert q.min() >= -7 and q.max() <= 7  # -8 is unreachable with scale = absmax / 7
    amax = x.reshape(4, 8, 16, 4, 32).abs().amax(-1)
    assert torch.equal(scale, torch.clamp(amax / 7.0, min=1e-8))
    err = (q.float() - x / scale.repeat_interleave(32, -1)).abs()
    assert err.max() <= 0.5 + 1e-6


def test_zero_group_and_ties_round_half_even():
    x = torch.zeros(1, 32)
    q, scale = ik.quantize_groups(x, 32)
    assert scale.item() == np.float32(1e-8)
    assert torch.equal(q, torch.zeros_like(q))
    assert torch.equal(ik.pack_nibbles(q), torch.zeros(1, 16, dtype=torch.uint8))
    # absmax 7 -> scale exactly 1: x/scale is exactly k + 0.5
    x = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] + [0.0] * 24])
    q, scale = ik.quantize_groups(x, 32)
    assert scale.item() == 1.0
    assert q[0, :8].tolist() == [7, 0, 2, 2, 0, -2, -2, 4]


def test_numpy_path_matches_torch_path():
    gen = torch.Generator().manual_seed(3)
    for g in (16, 32, 64, 128):
        x = (torch.randn(3, 2, 5, 128, generator=gen) * 3).to(torch.bfloat16)
        q, scale = ik.quantize_groups(x, g)
        packed = ik.pack_nibbles(q)
        np_packed, np_scale = ik.numpy_pack_reference(x.float().numpy(), g)
        assert np.array_equal(packed.numpy(), np_packed)
        assert np.array_equal(scale.numpy(), np_scale)


def test_nibble_layout_against_element_loop():
    gen = torch.Generator().manual_seed(4)
    q = torch.randint(-8, 8, (3, 40), generator=gen).to(torch.int8)
    packed = ik.pack_nibbles(q)
    for r in range(3):
        for p in range(20):
            lo = int(q[r, 2 * p]) & 15
            hi = int(q[r, 2 * p + 1]) & 15
            assert int(packed[r, p]) == lo | (hi << 4)
    all_vals = torch.arange(-8, 8, dtype=torch.int8).repeat(2)
    assert torch.equal(ik.unpack_nibbles(ik.pack_nibbles(all_vals)), all_vals)


def test_pack_into_cache_rows_and_length():
    gen = torch.Generator().manual_seed(5)
    cache = ik.allocate_cache(2, 2, 16, 128, 32)
    k = torch.randn(2, 2, 3, 128, generator=gen)
    v = torch.randn(2, 2, 3, 128, generator=gen)
    pos = torch.tensor([4, 9, 2])
    ik.pack_kv_into_cache(cache, k, v, pos, 32)
    assert cache["length"] == 10
    qk, sk = ik.quantize_groups(k, 32)
    assert torch.equal(cache["k_packed"][:, :, 9], ik.pack_nibbles(qk)[:, :, 1])
    assert torch.equal(cache["k_scale"][:, :, 2], sk[:, :, 2])
    untouched = [i for i in range(16) if i not in (2, 4, 9)]
    assert cache["v_packed"][:, :, untouched].abs().sum() == 0


def _cache(b, hkv, s, d, g, seed):
    gen = torch.Generator().manual_seed(seed)
    cache = ik.allocate_cache(b, hkv, s, d, g)
    k = torch.randn(b, hkv, s, d, generator=gen)
    v = torch.randn(b, hkv, s, d, generator=gen)
    ik.pack_kv_into_cache(cache, k, v, torch.arange(s), g)
    return cache


@pytest.mark.parametrize("nrep,g", [(4, 32), (2, 64), (1, 16)])
def test_attention_matches_sdpa(nrep, g):
    b, hkv, s, d = 2, 2, 37, 128
    c = _cache(b, hkv, s, d, g, 6)
    q = torch.randn(b, hkv * nrep, d, generator=torch.Generator().manual_seed(7))
    out = ik.decode_attention(q, c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"], s,
                              nrep, g)
    kd = ik.dequantize(c["k_packed"], c["k_scale"], g).double().repeat_interleave(nrep, 1)
    vd = ik.dequantize(c["v_packed"], c["v_scale"], g).double().repeat_interleave(nrep, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double()[:, :, None], kd, vd)[:, :, 0]
    assert torch.allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_attention_special_cases():
    b, hkv, nrep, d, g = 1, 2, 4, 128, 32
    c = _cache(b, hkv, 9, d, g, 8)
    args = (c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"])
    q = torch.randn(b, hkv * nrep, d)
    v0 = ik.dequantize(c["v_packed"][:, :, 0], c["v_scale"][:, :, 0], g).double()
    out1 = ik.decode_attention(q, *args, 1, nrep, g)  # one key: out = V_0 of the KV head
    assert torch.allclose(out1, v0.repeat_interleave(nrep, 1), rtol=0, atol=1e-12)
    out0 = ik.decode_attention(torch.zeros_like(q), *args, 9, nrep, g)  # uniform weights
    vmean = ik.dequantize(c["v_packed"][:, :, :9], c["v_scale"][:, :, :9], g).double().mean(2)
    assert torch.allclose(out0, vmean.repeat_interleave(nrep, 1), atol=1e-12)
    # GQA: query head h reads KV head h // nrep
    qs = q.clone()
    qs[:, 1] = qs[:, 0]
    out = ik.decode_attention(qs, *args, 9, nrep, g)
    assert torch.equal(out[:, 0], out[:, 1])
    c2 = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in c.items()}
    c2["v_scale"][:, 1] *= 2
    out2 = ik.decode_attention(q, c2["k_packed"], c2["v_packed"], c2["k_scale"], c2["v_scale"],
                               9, nrep, g)
    base = ik.decode_attention(q, *args, 9, nrep, g)
    assert torch.equal(out2[:, :nrep], base[:, :nrep])
    assert torch.allclose(out2[:, nrep:], 2 * base[:, nrep:])


def test_attention_mask_excludes_and_shifts():
    b, hkv, nrep, d, g, s = 2, 1, 4, 128, 32, 20
    c = _cache(b, hkv, s, d, g, 9)
    args = (c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"])
    q = torch.randn(b, hkv * nrep, d)
    keep = torch.ones(b, s, dtype=torch.bool)
    keep[0, :5] = False
    keep[1, 7] = False
    mask = ik.decode_attention_mask(keep, b, s)
    out = ik.decode_attention(q, *args, s, nrep, g, mask=mask)
    for bi in range(b):
        idx = keep[bi].nonzero()[:, 0]
        sub = ik.decode_attention(q[bi:bi + 1], *(t[bi:bi + 1, :, idx] for t in args), len(idx),
                                  nrep, g)
        assert torch.allclose(out[bi:bi + 1], sub, atol=1e-12)
    # additive bias: a constant shift of every key changes nothing
    shifted = ik.decode_attention(q, *args, s, nrep, g, mask=mask + 3.0)
    assert torch.allclose(out, shifted, atol=1e-12)
    # keys beyond the mask length are excluded
    short = ik.decode_attention(q, *args, s, nrep, g, mask=torch.zeros(b, 1, 1, 12))
    assert torch.allclose(short, ik.decode_attention(q, *args, 12, nrep, g), atol=1e-12)


def test_decode_attention_mask_branches():
    keep = torch.tensor([[1, 1, 0, 1, 1], [0, 1, 1, 1, 1]])
    m2 = ik.decode_attention_mask(keep, 2, 3)
    assert m2.shape == (2, 1, 1, 3)
    assert m2[0, 0, 0].tolist() == [-math.inf, 0.0, 0.0]
    m4b = torch.ones(2, 1, 3, 6, dtype=torch.bool)
    m4b[1, 0, -1, 2] = False
    m4 = ik.decode_attention_mask(m4b, 2, 4)
    assert m4.shape == (2, 1, 1, 4) and m4[1, 0, 0, 2] == -math.inf and m4[0].max() == 0
    m4f = torch.randn(2, 1, 3, 6)
    assert torch.equal(ik.decode_attention_mask(m4f, 2, 4), m4f[:, :, -1:, :4])
    assert ik.decode_attention_mask(None, 2, 4) is None
    with pytest.raises(ValueError, match="2D or 4D"):
        ik.decode_attention_mask(torch.ones(2, 3, 4), 2, 4)


def test_algorithmic_bytes_headline_figure():
    # B=64, ctx 16384, group 32, bf16 q and out: the figure quoted for the headline config
    assert ik.algorithmic_bytes(64, 32, 8, 128, 16384, 32) == 1_343_225_856


def test_package_byte_counts_match_the_oracle():
    from layer_quant_amd import traffic

    for args in [(64, 32, 8, 128, 16384, 32), (1, 32, 8, 128, 1024, 32), (8, 32, 8, 128, 4096, 64)]:
        assert traffic.attention_bytes(*args) == ik.algorithmic_bytes(*args)
    assert traffic.pack_bytes(64, 8, 1, 128, 32) == ik.pack_algorithmic_bytes(64, 8, 1, 128, 32)
    assert traffic.prefill_flops(1, 32, 16384, 128) == ik.prefill_flops(1, 32, 16384, 128)


@pytest.mark.parametrize("nrep,g,L", [(4, 32, 23), (2, 64, 40), (1, 16, 7)])
def test_prefill_matches_causal_sdpa(nrep, g, L):
    b, hkv, d = 2, 2, 128
    c = _cache(b, hkv, L + 5, d, g, 30)  # capacity above L: rows past L must not be read
    q = torch.randn(b, hkv * nrep, L, d, generator=torch.Generator().manual_seed(31))
    out = ik.prefill_attention(q, c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"], nrep, g)
    kd = ik.dequantize(c["k_packed"][:, :, :L], c["k_scale"][:, :, :L], g).double()
    vd = ik.dequantize(c["v_packed"][:, :, :L], c["v_scale"][:, :, :L], g).double()
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double(), kd.repeat_interleave(nrep, 1), vd.repeat_interleave(nrep, 1), is_causal=True)
    assert out.shape == (b, hkv * nrep, L, d)
    assert torch.allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_prefill_row_is_decode_over_its_prefix():
    b, hkv, nrep, d, g, L = 1, 2, 4, 128, 32, 19
    c = _cache(b, hkv, L, d, g, 32)
    args = (c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"])
    q = torch.randn(b, hkv * nrep, L, d, generator=torch.Generator().manual_seed(33))
    out = ik.prefill_attention(q, *args, nrep, g)
    for t in (0, 1, 7, L - 1):
        dec = ik.decode_attention(q[:, :, t], *args, t + 1, nrep, g)
        assert torch.allclose(out[:, :, t], dec, rtol=1e-12, atol=1e-13), t


def test_prefill_element_loop_and_special_cases():
    b, hkv, nrep, d, g, L = 1, 1, 2, 8, 4, 5
    c = _cache(b, hkv, L, d, g, 34)
    args = (c["k_packed"], c["v_packed"], c["k_scale"], c["v_scale"])
    q = torch.randn(b, hkv * nrep, L, d, generator=torch.Generator().manual_seed(35))
    out = ik.prefill_attention(q, *args, nrep, g)
    kd = ik.dequantize(c["k_packed"], c["k_scale"], g).double()
    vd = ik.dequantize(c["v_packed"], c["v_scale"], g).double()
    for h in range(hkv * nrep):
        for t in range(L):
            w = [math.exp(sum(q[0, h, t, i].item() * kd[0, h // nrep, n, i].item()
                              for i in range(d)) / math.sqrt(d)) for n in range(t + 1)]
            for i in range(d):
                want = sum(w[n] * vd[0, h // nrep, n, i].item() for n in range(t + 1)) / sum(w)
                assert abs(out[0, h, t, i].item() - want) <= 1e-12 * (1 + abs(want))
    one = ik.prefill_attention(q[:, :, :1], *args, nrep, g)  # q_len 1: V row 0
    assert torch.allclose(one[:, :, 0], vd[:, :, 0].repeat_interleave(nrep, 1), atol=1e-12)
    zero = ik.prefill_attention(torch.zeros_like(q), *args, nrep, g)  # uniform: running mean
    run = vd.cumsum(2) / torch.arange(1, L + 1, dtype=torch.float64)[:, None]
    assert torch.allclose(zero, run.repeat_interleave(nrep, 1), atol=1e-12)


def test_prefill_flops_closed_form():
    assert ik.prefill_flops(1, 32, 16384, 128) == 4 * 128 * 32 * (16384 * 16385 // 2)
    assert ik.prefill_flops(2, 1, 1, 64) == 2 * 4 * 64
