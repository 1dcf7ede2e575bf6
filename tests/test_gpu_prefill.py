"""GPU parity of the causal INT4 prefill attention through the C ABI (MFMA path for bf16 queries,
generic path for fp32 queries) against the float64 oracle: within 2e-3 for fp32 outputs, 8e-3 for
bf16 outputs (the output rounding itself is 2^-9 relative)."""
import pytest
import torch

from helpers import assert_close_rel, prefill_mfma_expected, require_env
from layer_quant_amd import _abi
from hybrid_quant import int4_8b_attention as ia
from oracle import int4_kv as oik

pytestmark = pytest.mark.gpu


def _activations(shape, seed, dtype=torch.bfloat16):
    """~N(0,1) with about 1% of head_dim channels scaled by 8 (shared across tokens)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen)
    chan = torch.rand(shape[1], shape[-1], generator=gen) < 0.01
    return torch.where(chan[None, :, None, :], x * 8, x).to(dtype)


def _packed_cache(b, hkv, s, d, g, seed, cap):
    cache = oik.allocate_cache(b, hkv, cap, d, g)
    k = _activations((b, hkv, s, d), seed)
    v = _activations((b, hkv, s, d), seed + 1)
    oik.pack_kv_into_cache(cache, k, v, torch.arange(s), g)
    return cache


def _run(gpu, cache, q, nrep, g, out_dtype=torch.float32):
    dev = {k: v.to(gpu) for k, v in cache.items() if torch.is_tensor(v)}
    out = torch.empty(*q.shape, dtype=out_dtype, device=gpu)
    # a call that passes the MFMA gate must take the MFMA kernel
    with require_env("LQ_PREFILL_REQUIRE_MFMA", prefill_mfma_expected(q.dtype, q.shape[-1], g)):
        _abi.int4_prefill_attention(q.to(gpu), dev["k_packed"], dev["v_packed"], dev["k_scale"],
                                    dev["v_scale"], out, nrep, g)
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(cache, q, nrep, g):
    return oik.prefill_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                                 cache["v_scale"], nrep, g)


PREFILL_CASES = [
    # b, hkv, nrep, L, g
    (1, 2, 4, 1, 32),
    (2, 2, 4, 37, 32),
    (1, 8, 4, 256, 32),
    (2, 2, 4, 100, 64),
    (1, 2, 4, 65, 128),
    (2, 2, 2, 70, 32),
    (1, 2, 1, 97, 32),
    (1, 1, 8, 50, 64),
    (1, 2, 4, 545, 32),   # 18 key tiles: two folds of the V offset
]


@pytest.mark.parametrize("b,hkv,nrep,L,g", PREFILL_CASES)
def test_prefill_parity_mfma_and_generic(gpu, b, hkv, nrep, L, g):
    d = 128
    cache = _packed_cache(b, hkv, L, d, g, 900 + L, cap=L + 7)
    q = _activations((b, hkv * nrep, L, d), 950 + L)
    ref = _oracle(cache, q, nrep, g)
    assert_close_rel(_run(gpu, cache, q, nrep, g), ref, what="mfma")
    assert_close_rel(_run(gpu, cache, q.float(), nrep, g), ref, what="generic")


@pytest.mark.parametrize("span", [10, 13])
@pytest.mark.parametrize("b,hkv,nrep,L,g", [(1, 2, 4, 200, 32), (2, 2, 4, 100, 64)])
def test_prefill_wide_value_scale_span(gpu, b, hkv, nrep, L, g, span):
    """Each key's values scaled by 2^-u, u uniform in [0, span): a group's V scales span up to
    2^span across a workgroup's keys, so P' = p * vscale / vmax reaches down to 2^-span times p,
    which the MFMA kernel's fp16 hi + lo split must still carry to the 2e-3 bar (the stated limit
    of the split is a span of 2^14)."""
    d = 128
    gen = torch.Generator().manual_seed(1000 + span + L)
    cache = oik.allocate_cache(b, hkv, L + 7, d, g)
    k = _activations((b, hkv, L, d), 1100 + L)
    v = _activations((b, hkv, L, d), 1101 + L).float()
    v = (v * torch.exp2(-torch.rand(b, hkv, L, 1, generator=gen) * span)).to(torch.bfloat16)
    oik.pack_kv_into_cache(cache, k, v, torch.arange(L), g)
    vs = cache["v_scale"][:, :, :L]
    assert (vs.amax() / vs.amin()).item() > 2.0 ** (span - 2)
    q = _activations((b, hkv * nrep, L, d), 1150 + L)
    ref = _oracle(cache, q, nrep, g)
    assert_close_rel(_run(gpu, cache, q, nrep, g), ref, what="mfma")
    assert_close_rel(_run(gpu, cache, q.float(), nrep, g), ref, what="generic")


@pytest.mark.parametrize("b,hkv,nrep,L,g,d", [(1, 2, 4, 90, 16, 128), (2, 1, 2, 40, 32, 64),
                                              (1, 1, 3, 33, 64, 256)])
def test_prefill_generic_shapes(gpu, b, hkv, nrep, L, g, d):
    cache = _packed_cache(b, hkv, L, d, g, 960 + d, cap=L)
    q = _activations((b, hkv * nrep, L, d), 970 + d)
    assert_close_rel(_run(gpu, cache, q, nrep, g), _oracle(cache, q, nrep, g))


def test_prefill_strided_query_and_module_api(gpu, diag):
    """The model's query_states is a transposed view [B, L, Hq, D] -> [B, Hq, L, D], taken by the
    MFMA kernel; _prefill_attention returns q's dtype like the reference (ia.py:600)."""
    diag.set("LQ_PREFILL_REQUIRE_MFMA")
    b, hkv, nrep, L, d, g = 2, 2, 4, 77, 128, 32
    cache = _packed_cache(b, hkv, L, d, g, 980, cap=128)
    q_bl = _activations((b, L, hkv * nrep, d), 981).transpose(1, 2)
    layer = ia.Int4KVLayerCache(*(cache[k].to(gpu) for k in
                                  ("k_packed", "v_packed", "k_scale", "v_scale")), length=L)
    out = ia._prefill_attention(q_bl.to(gpu), layer, nrep, g)
    assert out.dtype == torch.bfloat16 and out.shape == (b, hkv * nrep, L, d)
    assert_close_rel(out.float().cpu(), _oracle(cache, q_bl.contiguous(), nrep, g), rtol=8e-3)


def test_prefill_full_size_sampled_rows(gpu, diag):
    """Nemotron-H attention layer at L = 16384 (32 q heads, 8 KV heads, group 32): sampled
    (head, position) rows against the oracle's decode over the row's prefix, and the last row
    against the HIP decode kernel over the whole cache (both calls on their MFMA kernels)."""
    diag.set("LQ_PREFILL_REQUIRE_MFMA")
    diag.set("LQ_ATTN_REQUIRE_FAST")
    b, hkv, nrep, L, d, g = 1, 8, 4, 16384, 128, 32
    gen = torch.Generator(device=gpu).manual_seed(16384)
    kp = torch.randint(0, 256, (b, hkv, L, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vp = torch.randint(0, 256, (b, hkv, L, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    ks = torch.rand(b, hkv, L, d // g, device=gpu, generator=gen) * 0.5 + 0.05
    vs = torch.rand(b, hkv, L, d // g, device=gpu, generator=gen) * 0.5 + 0.05
    q = torch.randn(b, hkv * nrep, L, d, device=gpu, generator=gen).to(torch.bfloat16)
    out = torch.empty(b, hkv * nrep, L, d, device=gpu)
    _abi.int4_prefill_attention(q, kp, vp, ks, vs, out, nrep, g)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    kpc, vpc, ksc, vsc = kp.cpu(), vp.cpu(), ks.cpu(), vs.cpu()
    for h, t in [(0, 0), (1, 1), (5, 31), (13, 32), (31, 4095), (22, 9000), (7, L - 1)]:
        kv = h // nrep
        sl = slice(kv, kv + 1)
        ref = oik.decode_attention(q[:, h:h + 1, t].cpu(), kpc[:, sl], vpc[:, sl], ksc[:, sl],
                                   vsc[:, sl], t + 1, 1, g)
        assert_close_rel(out[:, h:h + 1, t].cpu(), ref, what=f"head {h} pos {t}")
    dec = torch.empty(b, hkv * nrep, d, device=gpu)
    _abi.int4_decode_attention(q[:, :, L - 1:L], kp, vp, ks, vs, None, dec, L, nrep, g)
    torch.cuda.synchronize()
    assert_close_rel(out[:, :, L - 1].cpu(), dec.cpu().double(), rtol=4e-3, what="vs decode")
