"""Seeded random sweep of decode-attention calls through the C ABI against the float64 oracle.

Each case draws batch, KV heads, query heads per KV head, context length, group size, mask kind
and query dtype, so the sweep reaches combinations the fixed cases do not: contexts ragged
against the 32-key tile and the 3-deep tile ring at every position, every column packing
nrep x (128 / g) <= 16 of the MFMA path, masks on calls that split the context across
workgroups, and the generic path (fp32 queries) on the same shapes. The reference semantics are
hybrid_quant/int4_8b_attention.py:254-402 (kernel) and :569-591 (mask)."""
import random

import pytest
import torch

from helpers import assert_close_rel, fast_attention_expected
from layer_quant_amd import _abi
from oracle import int4_kv as oik

pytestmark = pytest.mark.gpu

D = 128


def _draw_cases(n, seed):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        g = rng.choice([32, 64, 128])
        nrep = rng.choice([r for r in (1, 2, 4, 8, 16) if r * (D // g) <= 16])
        hkv = rng.choice([h for h in (1, 2, 4, 8) if h * nrep <= 32])
        b = rng.randint(1, 4)
        # a third short (within a few tiles), the rest up to a few thousand keys
        s = rng.randint(1, 100) if rng.random() < 0.33 else rng.randint(100, 3000)
        mask = rng.choice([None, "keep", "bias", "short"])
        qdt = rng.choice(["bf16", "f32"])
        cases.append((i, b, hkv, nrep, s, g, mask, qdt))
    return cases


CASES = _draw_cases(100, 20241202)


def _activations(shape, gen, outliers=True):
    x = torch.randn(*shape, generator=gen)
    if outliers:  # about 1 % of channels x8, shared across tokens (the config-2 data)
        chan = torch.rand(shape[1], shape[-1], generator=gen) < 0.01
        x = torch.where(chan[None, :, None, :], x * 8, x)
    return x


def _mask(kind, b, s, gen):
    if kind is None:
        return None
    if kind == "keep":  # 2-D keep-mask, longer than the context; the current token always kept
        keep = torch.rand(b, s + 3, generator=gen) > 0.3
        keep[:, -1] = True
        if b > 1:
            keep[0, : max(0, s - 1)] = False  # one row sees only its last key
        return oik.decode_attention_mask(keep, b, s)
    if kind == "bias":  # 4-D additive mask, last query row taken
        return oik.decode_attention_mask(torch.randn(b, 1, 3, s + 2, generator=gen) * 3, b, s)
    # a mask shorter than the context: keys at or past its length are excluded
    length = int(torch.randint(1, s + 1, (1,), generator=gen))
    return torch.zeros(b, 1, 1, length)


@pytest.mark.parametrize("i,b,hkv,nrep,s,g,mask_kind,qdt", CASES,
                         ids=[f"case{c[0]}" for c in CASES])
def test_attention_random_shapes(gpu, diag, i, b, hkv, nrep, s, g, mask_kind, qdt):
    print(f"[case {i}] b={b} hkv={hkv} nrep={nrep} s={s} g={g} mask={mask_kind} q={qdt}",
          flush=True)
    gen = torch.Generator().manual_seed(1000 + i)
    cap = s + int(torch.randint(0, 40, (1,), generator=gen))
    cache = oik.allocate_cache(b, hkv, cap, D, g)
    k = _activations((b, hkv, s, D), gen).to(torch.bfloat16)
    v = _activations((b, hkv, s, D), gen).to(torch.bfloat16)
    oik.pack_kv_into_cache(cache, k, v, torch.arange(s), g)
    q = _activations((b, hkv * nrep, 1, D), gen).to(torch.bfloat16)
    if qdt == "f32":
        q = q.float()
    if fast_attention_expected(q.dtype, D, g, nrep):  # then the MFMA kernel is required
        diag.set("LQ_ATTN_REQUIRE_FAST")
    mask = _mask(mask_kind, b, s, gen)
    ref = oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                               cache["v_scale"], s, nrep, g, mask=mask)
    dev = {n: t.to(gpu) for n, t in cache.items() if torch.is_tensor(t)}
    out = torch.empty(b, hkv * nrep, D, device=gpu)
    _abi.int4_decode_attention(q.to(gpu), dev["k_packed"], dev["v_packed"], dev["k_scale"],
                               dev["v_scale"], None if mask is None else mask.to(gpu), out, s,
                               nrep, g)
    torch.cuda.synchronize()
    assert_close_rel(out.cpu(), ref, what=f"case {i}")
