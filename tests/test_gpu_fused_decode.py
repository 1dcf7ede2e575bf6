"""GPU parity of lq_int4_decode_attention_pack, the decode branch of the reference's patched
attention forward as one call (reference hybrid_quant/int4_8b_attention.py:678-690:
_pack_kv_into_cache of the new token, then _decode_attention).

The bar is bit-identity with the two separate calls it replaces, lq_int4_pack_kv_pair into row
seq_len - 1 followed by lq_int4_decode_attention, on the same inputs: every byte of both packed
caches and both scale caches, and every output value. On the MFMA path the attention kernel packs
the token itself (the wave that attends to key seq_len - 1); elsewhere the two kernels run in
turn. The packed row is also checked against the oracle's pack (ia.py:56-111) and the output,
on some cases, against the float64 oracle attention (:254-402).

Seeded cases draw the group (32/64/128), query heads per KV head, KV heads, batch (including 64,
one workgroup per (batch, KV head), and small batches that split the keys across workgroups),
the context (so that key seq_len - 1 falls in every position of a tile, of the 3-deep tile ring
and of the 4 waves' dealing), the token's dtype and layout (a transposed view), the mask kind and
the output dtype; fp32 queries take the generic path."""
import random

import pytest
import torch

from helpers import assert_close_rel, fast_attention_expected, require_env
from layer_quant_amd import _abi
from oracle import int4_kv as oik

pytestmark = pytest.mark.gpu

D = 128
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _draw(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        g = rng.choice([32, 64, 128])
        nrep = rng.choice([r for r in (1, 2, 4, 8, 16) if r * (D // g) <= 16])
        hkv = rng.choice([h for h in (1, 2, 8) if h * nrep <= 32])
        b = rng.choice([1, 2, 3, 64]) if hkv == 8 else rng.randint(1, 4)
        s = rng.choice([1, 2, 31, 32, 33, 95, 96, 97, 128, 129]) if rng.random() < 0.4 \
            else rng.randint(130, 5000 if b < 64 else 1200)
        out.append(dict(i=i, g=g, nrep=nrep, hkv=hkv, b=b, s=s,
                        kdt=rng.choice(["bf16", "bf16", "f16", "f32"]),
                        strided=rng.random() < 0.3,
                        mask=rng.choice([None, None, "keep", "bias", "short"]),
                        qdt=rng.choice(["bf16", "bf16", "bf16", "f32"]),
                        odt=rng.choice(["f32", "bf16"]),
                        oracle=rng.random() < 0.25))
    return out


CASES = _draw(72, 4242)


def _token(c, gen, gpu):
    """The new token's K or V [B, Hkv, 1, D] (optionally a transposed [B, 1, Hkv, D] view)."""
    shape = (c["b"], 1, c["hkv"], D) if c["strided"] else (c["b"], c["hkv"], 1, D)
    x = (torch.randn(*shape, generator=gen) * 2).to(DTYPES[c["kdt"]]).to(gpu)
    return x.transpose(1, 2) if c["strided"] else x


def _mask(kind, b, s, gen):
    if kind is None:
        return None
    if kind == "keep":
        keep = torch.rand(b, s + 2, generator=gen) > 0.3
        keep[:, -1] = True
        return oik.decode_attention_mask(keep, b, s)
    if kind == "bias":
        return oik.decode_attention_mask(torch.randn(b, 1, 2, s, generator=gen) * 3, b, s)
    return torch.zeros(b, 1, 1, int(torch.randint(1, s + 1, (1,), generator=gen)))


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_fused_pack_attention_equals_two_calls(gpu, diag, c):
    print(f"[fused case {c['i']}] {c}", flush=True)
    b, hkv, nrep, s, g = c["b"], c["hkv"], c["nrep"], c["s"], c["g"]
    gen = torch.Generator().manual_seed(7000 + c["i"])
    cap = s + int(torch.randint(0, 9, (1,), generator=gen))
    dgen = torch.Generator(device=gpu).manual_seed(7000 + c["i"])
    kp = torch.randint(0, 256, (b, hkv, cap, D // 2), dtype=torch.uint8, device=gpu,
                       generator=dgen)
    vp = torch.randint(0, 256, (b, hkv, cap, D // 2), dtype=torch.uint8, device=gpu,
                       generator=dgen)
    ks = torch.rand(b, hkv, cap, D // g, device=gpu, generator=dgen) * 0.5 + 0.05
    vs = torch.rand(b, hkv, cap, D // g, device=gpu, generator=dgen) * 0.5 + 0.05
    q = torch.randn(b, hkv * nrep, 1, D, generator=gen).to(DTYPES[c["qdt"]]).to(gpu)
    k_new, v_new = _token(c, gen, gpu), _token(c, gen, gpu)
    mask = _mask(c["mask"], b, s, gen)
    mask = None if mask is None else mask.to(gpu)
    if fast_attention_expected(q.dtype, D, g, nrep):  # then the fused MFMA kernel is required
        diag.set("LQ_ATTN_REQUIRE_FAST")
    sep = [t.clone() for t in (kp, vp, ks, vs)]
    fus = [t.clone() for t in (kp, vp, ks, vs)]
    out_sep = torch.full((b, hkv * nrep, D), float("nan"), dtype=DTYPES[c["odt"]], device=gpu)
    out_fus = torch.full_like(out_sep, float("nan"))
    _abi.int4_pack_kv_pair(k_new, v_new, *sep, torch.tensor([s - 1], device=gpu), g)
    _abi.int4_decode_attention(q, *sep, mask, out_sep, s, nrep, g)
    _abi.int4_decode_attention_pack(q, k_new, v_new, *fus, mask, out_fus, s, nrep, g)
    torch.cuda.synchronize()
    for a, f, name in zip(sep, fus, ("k_packed", "v_packed", "k_scale", "v_scale")):
        assert torch.equal(a, f), f"case {c['i']}: {name} differs"
    assert torch.equal(out_sep, out_fus), f"case {c['i']}: outputs differ"
    # the packed row against the oracle's pack of the token
    for x, pk, sc in ((k_new, fus[0], fus[2]), (v_new, fus[1], fus[3])):
        rp = torch.zeros(b, hkv, 1, D // 2, dtype=torch.uint8)
        rs = torch.zeros(b, hkv, 1, D // g)
        oik.pack_into(rp, rs, x.cpu(), torch.tensor([0]), g)
        assert torch.equal(pk[:, :, s - 1:s].cpu(), rp)
        assert torch.equal(sc[:, :, s - 1:s].cpu(), rs)
    if c["oracle"]:
        ref = oik.decode_attention(q.cpu(), fus[0].cpu(), fus[1].cpu(), fus[2].cpu(),
                                   fus[3].cpu(), s, nrep, g,
                                   mask=None if mask is None else mask.cpu())
        assert_close_rel(out_fus.float().cpu(), ref, rtol=2e-3 if c["odt"] == "f32" else 8e-3,
                         what=f"fused case {c['i']}")


@pytest.mark.parametrize("b,s,g", [(64, 16384, 32), (8, 4133, 64), (1, 1057, 128)])
def test_fused_repeats_bit_identical(gpu, b, s, g):
    """Repeated fused calls on the same inputs (each rewriting the same row) give bit-identical
    caches and outputs: the pack and the tile ring's waits leave nothing to chance."""
    hkv, nrep = 8, 4
    dgen = torch.Generator(device=gpu).manual_seed(b + s + g)
    kp = torch.randint(0, 256, (b, hkv, s, D // 2), dtype=torch.uint8, device=gpu, generator=dgen)
    vp = torch.randint(0, 256, (b, hkv, s, D // 2), dtype=torch.uint8, device=gpu, generator=dgen)
    ks = torch.rand(b, hkv, s, D // g, device=gpu, generator=dgen) + 0.01
    vs = torch.rand(b, hkv, s, D // g, device=gpu, generator=dgen) + 0.01
    q = torch.randn(b, hkv * nrep, 1, D, device=gpu, generator=dgen).to(torch.bfloat16)
    kn = torch.randn(b, hkv, 1, D, device=gpu, generator=dgen).to(torch.bfloat16)
    vn = torch.randn(b, hkv, 1, D, device=gpu, generator=dgen).to(torch.bfloat16)
    ref = torch.empty(b, hkv * nrep, D, device=gpu)
    with require_env("LQ_ATTN_REQUIRE_FAST"):
        _abi.int4_decode_attention_pack(q, kn, vn, kp, vp, ks, vs, None, ref, s, nrep, g)
        torch.cuda.synchronize()
        first = [t.clone() for t in (kp, vp, ks, vs)]
        out = torch.empty_like(ref)
        for _ in range(10):
            out.fill_(float("nan"))
            _abi.int4_decode_attention_pack(q, kn, vn, kp, vp, ks, vs, None, out, s, nrep, g)
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    assert all(torch.equal(a, f) for a, f in zip(first, (kp, vp, ks, vs)))
    assert torch.isfinite(ref).all()


def test_fused_branch_bad_mask_leaves_token_packed(gpu):
    """A mask of unsupported rank raises ValueError after the token is packed and cache.length
    moved, as in the reference, whose decode branch packs (ia.py:678) before its mask check
    raises (:532)."""
    from hybrid_quant import int4_8b_attention as ia

    b, hkv, nrep, g, s = 2, 8, 4, 32, 40
    gen = torch.Generator().manual_seed(5)
    holder = type("Cache", (), {})()
    cache = ia._ensure_layer_cache(holder, 0, b, hkv, s, D, g, gpu)
    cache.k_packed.zero_(), cache.v_packed.zero_(), cache.k_scale.zero_(), cache.v_scale.zero_()
    cache.length = s - 1
    q = torch.randn(b, hkv * nrep, 1, D, generator=gen).to(torch.bfloat16).to(gpu)
    kn = torch.randn(b, hkv, 1, D, generator=gen).to(torch.bfloat16).to(gpu)
    vn = torch.randn(b, hkv, 1, D, generator=gen).to(torch.bfloat16).to(gpu)
    bad_mask = torch.ones(b, 1, s, device=gpu)
    with pytest.raises(ValueError, match="2D or 4D"):
        ia._pack_and_decode_attention(q, kn, vn, cache, s, nrep, g, attention_mask=bad_mask)
    assert cache.length == s
    for x, pk, sc in ((kn, cache.k_packed, cache.k_scale), (vn, cache.v_packed, cache.v_scale)):
        rp = torch.zeros(b, hkv, 1, D // 2, dtype=torch.uint8)
        rs = torch.zeros(b, hkv, 1, D // g)
        oik.pack_into(rp, rs, x.cpu(), torch.tensor([0]), g)
        assert torch.equal(pk[:, :, s - 1:s].cpu(), rp)
        assert torch.equal(sc[:, :, s - 1:s].cpu(), rs)
        assert not pk[:, :, : s - 1].any()
