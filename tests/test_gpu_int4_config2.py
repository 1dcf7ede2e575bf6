"""GPU parity of the INT4 decode attention at the BASELINE config-2 grid and on inputs built to
stress its arithmetic.

Config 2: 32 query / 8 KV heads, head_dim 128, group 32, batch {1, 8, 64} x ctx {1024, 4096,
16384}; Q/K/V bf16 ~N(0,1) with about 1% of the channels (per KV head, shared by K, V and the
query heads of that KV head) scaled by 8. The whole context is packed on the GPU in one
lq_int4_pack_kv_pair call; on sampled (batch, KV head) pairs the packed bytes and scales must
equal the oracle's pack bit for bit, and the attention output must be within 2e-3 of the float64
oracle (reference hybrid_quant/int4_8b_attention.py:32-111 and :254-402).

The precision tests target the two places where the MFMA kernel's arithmetic differs from a
plain fp32 dot product: nibbles enter the bf16 MFMAs as 136 + n (the offset is removed with
-136 * sum(q) for scores and -136 * sum(P') for values, so fp32 accumulation rounds at the
magnitude of the offset), and P' = p * vscale enters as a bf16 hi + lo pair.
"""
import pytest
import torch

from helpers import assert_close_rel
from layer_quant_amd import _abi
from oracle import int4_kv as oik

pytestmark = pytest.mark.gpu

HKV, NREP, D = 8, 4, 128


@pytest.fixture(autouse=True)
def _mfma_kernel_required(diag):
    """Every call here (bf16 queries, 4 query heads per KV head, group 32/64/128) must take the
    MFMA kernel: the library refuses it otherwise."""
    diag.set("LQ_ATTN_REQUIRE_FAST")


def _outlier_channels(gen, device, hkv=HKV, d=D, frac=0.01):
    """[hkv, d] multipliers: 8 on about `frac` of the channels, at least one per KV head."""
    chan = torch.rand(hkv, d, device=device, generator=gen) < frac
    pick = torch.randint(0, d, (hkv,), device=device, generator=gen)
    chan[torch.arange(hkv, device=device), pick] = True
    return torch.where(chan, 8.0, 1.0)


def _config2_inputs(gpu, b, s, seed):
    gen = torch.Generator(device=gpu).manual_seed(seed)
    mult = _outlier_channels(gen, gpu)
    k = (torch.randn(b, HKV, s, D, device=gpu, generator=gen) * mult[None, :, None]).to(torch.bfloat16)
    v = (torch.randn(b, HKV, s, D, device=gpu, generator=gen) * mult[None, :, None]).to(torch.bfloat16)
    q = torch.randn(b, HKV, NREP, D, device=gpu, generator=gen) * mult[None, :, None]
    return q.to(torch.bfloat16).reshape(b, HKV * NREP, 1, D), k, v


def _pack_on_gpu(gpu, k, v, g):
    b, hkv, s, d = k.shape
    kp = torch.empty(b, hkv, s, d // 2, dtype=torch.uint8, device=gpu)
    vp = torch.empty_like(kp)
    ks = torch.empty(b, hkv, s, d // g, device=gpu)
    vs = torch.empty_like(ks)
    _abi.int4_pack_kv_pair(k, v, kp, vp, ks, vs, torch.arange(s, device=gpu), g)
    return kp, vp, ks, vs


def _sample_pairs(b):
    if b == 1:
        return [(0, kv) for kv in range(HKV)]
    return sorted({(0, 0), (b - 1, HKV - 1), (b // 2, 3), (b // 3, 6)})


def _check_pairs(q, k, v, packed, out, s, g, pairs, what):
    kp, vp, ks, vs = packed
    for bi, kv in pairs:
        ref_kp, ref_ks = oik.numpy_pack_reference(k[bi, kv].float().cpu().numpy(), g)
        ref_vp, ref_vs = oik.numpy_pack_reference(v[bi, kv].float().cpu().numpy(), g)
        got = [t[bi, kv].cpu().numpy() for t in (kp, ks, vp, vs)]
        for name, a, r in zip(("k bytes", "k scales", "v bytes", "v scales"), got,
                              (ref_kp, ref_ks, ref_vp, ref_vs)):
            assert (a == r).all(), f"{what} b{bi} kv{kv}: {name} differ from the oracle pack"
        heads = slice(kv * NREP, (kv + 1) * NREP)
        sl = slice(bi, bi + 1)
        ref = oik.decode_attention(q[sl, heads].cpu(), kp[sl, kv:kv + 1].cpu(),
                                   vp[sl, kv:kv + 1].cpu(), ks[sl, kv:kv + 1].cpu(),
                                   vs[sl, kv:kv + 1].cpu(), s, NREP, g)
        assert_close_rel(out[sl, heads].cpu(), ref, what=f"{what} b{bi} kv{kv}")


@pytest.mark.parametrize("s", [1024, 4096, 16384])
@pytest.mark.parametrize("b", [1, 8, 64])
def test_config2_grid(gpu, b, s):
    """Every cell of config 2: pack the context on the GPU, attend, check sampled pairs (at batch
    1 and ctx 16384 the plan splits each (batch, KV head) 64 ways and merges the partials)."""
    g = 32
    q, k, v = _config2_inputs(gpu, b, s, seed=1000 * b + s)
    packed = _pack_on_gpu(gpu, k, v, g)
    out = torch.empty(b, HKV * NREP, D, device=gpu)
    _abi.int4_decode_attention(q, *packed, None, out, s, NREP, g)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check_pairs(q, k, v, packed, out, s, g, _sample_pairs(b), f"B{b} S{s}")


@pytest.mark.parametrize("g", [64, 128])
def test_config2_full_size_other_groups(gpu, g):
    """The headline size with the reference driver's default group (64) and with 128."""
    b, s = 64, 16384
    q, k, v = _config2_inputs(gpu, b, s, seed=77 + g)
    packed = _pack_on_gpu(gpu, k, v, g)
    out = torch.empty(b, HKV * NREP, D, device=gpu)
    _abi.int4_decode_attention(q, *packed, None, out, s, NREP, g)
    torch.cuda.synchronize()
    _check_pairs(q, k, v, packed, out, s, g, _sample_pairs(b), f"g{g}")


def _random_cache(gpu, gen, b, s, g, kscale, vscale):
    kp = torch.randint(0, 256, (b, HKV, s, D // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vp = torch.randint(0, 256, (b, HKV, s, D // 2), dtype=torch.uint8, device=gpu, generator=gen)
    return kp, vp, kscale, vscale


def _run_and_check(gpu, q, cache, s, g, pairs, what):
    kp, vp, ks, vs = cache
    out = torch.empty(q.shape[0], q.shape[1], D, device=gpu)
    _abi.int4_decode_attention(q, kp, vp, ks, vs, None, out, s, NREP, g)
    torch.cuda.synchronize()
    for bi, kv in pairs:
        heads = slice(kv * NREP, (kv + 1) * NREP)
        sl = slice(bi, bi + 1)
        ref = oik.decode_attention(q[sl, heads].cpu(), kp[sl, kv:kv + 1].cpu(),
                                   vp[sl, kv:kv + 1].cpu(), ks[sl, kv:kv + 1].cpu(),
                                   vs[sl, kv:kv + 1].cpu(), s, NREP, g)
        assert_close_rel(out[sl, heads].cpu(), ref, what=f"{what} b{bi} kv{kv}")


def _outlier_queries(gpu, gen, b, scale, positive):
    """Queries whose 32-dim groups have a large sum: |N(0,1)| (or N(0,1)) with about 1% of the
    channels times `scale`; positive=True makes every component positive, so -136 * sum(q) is as
    large as the query's magnitude allows."""
    q = torch.randn(b, HKV, NREP, D, device=gpu, generator=gen)
    if positive:
        q = q.abs()
    mult = _outlier_channels(gen, gpu) / 8.0 * scale
    mult = torch.where(mult > 1.0, mult, torch.ones_like(mult))
    return (q * mult[None, :, None]).to(torch.bfloat16).reshape(b, HKV * NREP, 1, D)


@pytest.mark.parametrize("b", [2, 64])
@pytest.mark.parametrize("qscale", [8.0, 32.0])
def test_precision_flat_softmax_wide_value_scales(gpu, b, qscale):
    """A flat softmax over 16384 keys (tiny key scales, so every weight is about equal) with value
    scales spread log-uniformly over 2^10 and outlier query channels: the output is a small
    weighted mean of zero-mean values, the case in which the value offset's cancellation
    (sum P'(136 + n) - 136 sum P', accumulated over 4096 keys per wave at batch 64) is largest
    relative to the result."""
    s, g = 16384, 32
    gen = torch.Generator(device=gpu).manual_seed(int(31 * b + qscale))
    ks = torch.rand(b, HKV, s, D // g, device=gpu, generator=gen) * 1e-4 + 1e-5
    vs = 0.01 * torch.exp2(torch.rand(b, HKV, s, D // g, device=gpu, generator=gen) * 10.0)
    cache = _random_cache(gpu, gen, b, s, g, ks, vs)
    q = _outlier_queries(gpu, gen, b, qscale, positive=False)
    _run_and_check(gpu, q, cache, s, g, _sample_pairs(b)[:4], f"flat q*{qscale}")


@pytest.mark.parametrize("b", [2, 64])
@pytest.mark.parametrize("score_std", [4.0, 16.0])
def test_precision_peaked_softmax_same_sign_queries(gpu, b, score_std):
    """Same-sign queries with x32 outlier channels (the largest -136 * sum(q) per group for their
    norm) and key scales set so that the scores spread with a standard deviation of `score_std`
    log2 units over 16384 keys: a handful of keys carry the softmax, so errors in their scores
    reach the output directly. Value scales span 2^10."""
    s, g = 16384, 32
    gen = torch.Generator(device=gpu).manual_seed(int(17 * b + score_std))
    q = _outlier_queries(gpu, gen, b, 32.0, positive=True)
    # raw score std = |q| * std(nibble) * kscale; std(nibble) = sqrt(85/4) over -8..7
    qnorm = q.float().norm(dim=-1).mean().item()
    kscale = score_std / (qnorm * (85.0 / 4.0) ** 0.5 * 1.4426950408889634 / D ** 0.5)
    ks = kscale * (0.75 + 0.5 * torch.rand(b, HKV, s, D // g, device=gpu, generator=gen))
    vs = 0.01 * torch.exp2(torch.rand(b, HKV, s, D // g, device=gpu, generator=gen) * 10.0)
    cache = _random_cache(gpu, gen, b, s, g, ks, vs)
    _run_and_check(gpu, q, cache, s, g, _sample_pairs(b)[:4], f"peaked std{score_std}")


def test_precision_single_key_dominates(gpu):
    """One key per (batch, KV head) scores 40 log2 units above the rest (p of the others below
    2^-40): the output must be that key's value row, exactly as the oracle's."""
    b, s, g = 4, 16384, 32
    gen = torch.Generator(device=gpu).manual_seed(5)
    q = _outlier_queries(gpu, gen, b, 8.0, positive=True)
    kp = torch.zeros(b, HKV, s, D // 2, dtype=torch.uint8, device=gpu)
    hot = torch.randint(0, s, (b, HKV), device=gpu, generator=gen)
    # all nibbles of the hot key are +7 (0x77), every other key is 0
    kp[torch.arange(b)[:, None], torch.arange(HKV)[None], hot] = 0x77
    ks = torch.full((b, HKV, s, D // g), 1.0, device=gpu)
    qsum = q.float().view(b, HKV, NREP, D).sum(-1).amin(-1)  # [b, HKV]
    ks_hot = 40.0 / (7.0 * qsum * 1.4426950408889634 / D ** 0.5)
    ks[torch.arange(b)[:, None], torch.arange(HKV)[None], hot] = ks_hot[..., None]
    vp = torch.randint(0, 256, (b, HKV, s, D // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vs = torch.rand(b, HKV, s, D // g, device=gpu, generator=gen) + 0.1
    _run_and_check(gpu, q, (kp, vp, ks, vs), s, g, _sample_pairs(b)[:4], "one hot key")
