"""Seeded random sweeps of the INT4 pack, the causal INT4 prefill attention and the unquantized
selective-state update through the C ABI against the CPU oracle, each case drawing its shape,
dtypes and optional inputs (the fixed cases of the other test files pin the named edge cases).

* pack (hybrid_quant/int4_8b_attention.py:32-111, 477-515): bytes and scales bit-exact, single
  and K+V-pair entry points, head_dim 64/96/128/256, every even group dividing it, bf16/fp16/fp32
  inputs, random distinct positions in a larger cache; prompt-sized packs (16-600 tokens per
  (batch, head), g 8-256, V as a transposed view in some) for the group-per-lane and row kernels.
* prefill (:114-251, 594-625): within 2e-3 of the float64 oracle (8e-3 for bf16 outputs), MFMA
  path (bf16 queries) and generic path (fp32), prompts of 1-300 tokens, group 32/64/128, 1-8
  query heads per KV head.
* unquantized update (mamba-ssm selective_state_update, the reference's fallback at
  mamba_state_8b_kernel.py:738-747): y within the output's rounding of the oracle's, the state
  equal to the oracle's fp32 update rounded to the state dtype for >= 99.9 % of the elements and
  within one ulp elsewhere (one fp32 rounding differs; fp32 states within 1e-5), on both
  kernels' layouts."""
import random

import pytest
import torch

from helpers import assert_close_rel, prefill_mfma_expected, to_device
from hybrid_quant import mamba_state_8b_kernel as ms
from layer_quant_amd import _abi
from oracle import int4_kv as oik
from oracle import mx_state as omx

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _activations(shape, gen):
    x = torch.randn(*shape, generator=gen)
    chan = torch.rand(shape[1], shape[-1], generator=gen) < 0.01
    return torch.where(chan[None, :, None, :], x * 8, x)


# ---------------------------------------------------------------------------------------- pack

def _pack_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        d = rng.choice([64, 96, 128, 256])
        g = rng.choice([gg for gg in range(2, d + 1, 2) if d % gg == 0])
        out.append((i, rng.randint(1, 3), rng.choice([1, 2, 8]), rng.randint(1, 6), d, g,
                    rng.choice(["bf16", "f16", "f32"]), rng.random() < 0.5))
    return out


PACK_CASES = _pack_cases(48, 77)


@pytest.mark.parametrize("i,b,h,t,d,g,dt,pair", PACK_CASES, ids=[f"case{c[0]}" for c in PACK_CASES])
def test_pack_random(gpu, i, b, h, t, d, g, dt, pair):
    print(f"[pack case {i}] b={b} h={h} t={t} d={d} g={g} {dt} pair={pair}", flush=True)
    gen = torch.Generator().manual_seed(300 + i)
    cap = t + int(torch.randint(0, 20, (1,), generator=gen))
    pos = torch.randperm(cap, generator=gen)[:t]
    k = _activations((b, h, t, d), gen).to(DTYPES[dt])
    v = _activations((b, h, t, d), gen).to(DTYPES[dt])
    kp = torch.full((b, h, cap, d // 2), 0x3C, dtype=torch.uint8, device=gpu)
    vp = torch.full_like(kp, 0xC3)
    ks = torch.full((b, h, cap, d // g), -1.0, device=gpu)
    vs = torch.full_like(ks, -2.0)
    if pair:
        _abi.int4_pack_kv_pair(k.to(gpu), v.to(gpu), kp, vp, ks, vs, pos.to(gpu), g)
    else:
        _abi.int4_pack_kv(k.to(gpu), kp, ks, pos.to(gpu), g)
        _abi.int4_pack_kv(v.to(gpu), vp, vs, pos.to(gpu), g)
    torch.cuda.synchronize()
    for x, p_dev, s_dev, fill, sfill in ((k, kp, ks, 0x3C, -1.0), (v, vp, vs, 0xC3, -2.0)):
        ref_p = torch.full((b, h, cap, d // 2), fill, dtype=torch.uint8)
        ref_s = torch.full((b, h, cap, d // g), sfill)
        oik.pack_into(ref_p, ref_s, x, pos, g)
        assert torch.equal(p_dev.cpu(), ref_p)
        assert torch.equal(s_dev.cpu(), ref_s)


def _prompt_pack_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        d = rng.choice([64, 128, 256])
        g = rng.choice([gg for gg in (8, 16, 24, 32, 48, 64, 128, 256) if d % gg == 0])
        b, h = rng.randint(1, 2), rng.choice([1, 2, 8])
        out.append((i, b, h, rng.randint(max(16, 2048 // d), 600 if b * h <= 2 else 160), d, g,
                    rng.choice(["bf16", "f16", "f32"]), rng.random() < 0.6, rng.random() < 0.5,
                    rng.random() < 0.5))
    return out


PROMPT_PACK_CASES = _prompt_pack_cases(24, 2026)


@pytest.mark.parametrize("i,b,h,t,d,g,dt,pair,vt,shuffled", PROMPT_PACK_CASES,
                         ids=[f"case{c[0]}" for c in PROMPT_PACK_CASES])
def test_pack_random_prompt(gpu, i, b, h, t, d, g, dt, pair, vt, shuffled):
    """Prompt-sized packs (many tokens per (batch, head), so the group-per-lane and the row
    kernels take them where their layouts allow): bit-exact against the oracle, with V as the
    model's transposed view in some cases and the positions shuffled or offset."""
    print(f"[prompt pack case {i}] b={b} h={h} t={t} d={d} g={g} {dt} pair={pair} vt={vt}",
          flush=True)
    gen = torch.Generator().manual_seed(700 + i)
    cap = t + int(torch.randint(0, 20, (1,), generator=gen))
    pos = torch.randperm(cap, generator=gen)[:t] if shuffled else torch.arange(t) + (cap - t)
    k = _activations((b, h, t, d), gen).to(DTYPES[dt])
    if vt:
        v = _activations((b, t, h, d), gen).to(DTYPES[dt]).transpose(1, 2)
    else:
        v = _activations((b, h, t, d), gen).to(DTYPES[dt])
    k[0, 0, t // 2] = 0
    kp = torch.full((b, h, cap, d // 2), 0x3C, dtype=torch.uint8, device=gpu)
    vp = torch.full_like(kp, 0xC3)
    ks = torch.full((b, h, cap, d // g), -1.0, device=gpu)
    vs = torch.full_like(ks, -2.0)
    if pair:
        _abi.int4_pack_kv_pair(k.to(gpu), v.to(gpu), kp, vp, ks, vs, pos.to(gpu), g)
    else:
        _abi.int4_pack_kv(k.to(gpu), kp, ks, pos.to(gpu), g)
        _abi.int4_pack_kv(v.to(gpu), vp, vs, pos.to(gpu), g)
    torch.cuda.synchronize()
    for x, p_dev, s_dev, fill, sfill in ((k, kp, ks, 0x3C, -1.0), (v, vp, vs, 0xC3, -2.0)):
        ref_p = torch.full((b, h, cap, d // 2), fill, dtype=torch.uint8)
        ref_s = torch.full((b, h, cap, d // g), sfill)
        oik.pack_into(ref_p, ref_s, x.contiguous(), pos, g)
        assert torch.equal(p_dev.cpu(), ref_p)
        assert torch.equal(s_dev.cpu(), ref_s)


# ------------------------------------------------------------------------------------- prefill

def _prefill_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        g = rng.choice([32, 64, 128])
        nrep = rng.choice([r for r in (1, 2, 4, 8) if r * (128 // g) <= 16])
        out.append((i, rng.randint(1, 2), rng.choice([1, 2]), nrep,
                    rng.randint(1, 40) if rng.random() < 0.4 else rng.randint(40, 300), g,
                    rng.choice(["bf16", "f32"]), rng.choice(["f32", "f32", "bf16"])))
    return out


PREFILL_CASES = _prefill_cases(32, 88)


@pytest.mark.parametrize("i,b,hkv,nrep,L,g,qdt,odt", PREFILL_CASES,
                         ids=[f"case{c[0]}" for c in PREFILL_CASES])
def test_prefill_random(gpu, diag, i, b, hkv, nrep, L, g, qdt, odt):
    print(f"[prefill case {i}] b={b} hkv={hkv} nrep={nrep} L={L} g={g} q={qdt} out={odt}",
          flush=True)
    d = 128
    gen = torch.Generator().manual_seed(400 + i)
    cap = L + int(torch.randint(0, 33, (1,), generator=gen))
    cache = oik.allocate_cache(b, hkv, cap, d, g)
    k = _activations((b, hkv, L, d), gen).to(torch.bfloat16)
    v = _activations((b, hkv, L, d), gen).to(torch.bfloat16)
    oik.pack_kv_into_cache(cache, k, v, torch.arange(L), g)
    q = _activations((b, hkv * nrep, L, d), gen).to(torch.bfloat16)
    if qdt == "f32":
        q = q.float()
    if prefill_mfma_expected(q.dtype, d, g):  # then the MFMA kernel is required
        diag.set("LQ_PREFILL_REQUIRE_MFMA")
    ref = oik.prefill_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                                cache["v_scale"], nrep, g)
    dev = {n_: t.to(gpu) for n_, t in cache.items() if torch.is_tensor(t)}
    out = torch.empty(*q.shape, dtype=DTYPES[odt], device=gpu)
    _abi.int4_prefill_attention(q.to(gpu), dev["k_packed"], dev["v_packed"], dev["k_scale"],
                                dev["v_scale"], out, nrep, g)
    torch.cuda.synchronize()
    # fp32 out within 2e-3; bf16 out adds its own rounding (2^-9 relative)
    assert_close_rel(out.float().cpu(), ref, rtol=2e-3 if odt == "f32" else 8e-3,
                     what=f"prefill case {i}")


# --------------------------------------------------------------------------- unquantized update

ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -23}
BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def _ssm_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        out.append((i, dict(
            sdt=rng.choice(["bf16", "f16", "f32"]), n=rng.choice([64, 128, 256, 96]),
            p=rng.choice([8, 32, 64, 50]), bsz=rng.randint(1, 3), ng=rng.choice([1, 2, 4]),
            ratio=rng.choice([1, 2, 4]), head_const=rng.random() < 0.7, z=rng.random() < 0.3,
            dtb=rng.random() < 0.7, has_d=rng.random() < 0.7, softplus=rng.random() < 0.7,
            xdt=rng.choice(["bf16", "f32"]))))
    return out


SSM_CASES = _ssm_cases(48, 99)


@pytest.mark.parametrize("i,c", SSM_CASES, ids=[f"case{c[0]}" for c in SSM_CASES])
def test_unquantized_update_random(gpu, diag, i, c):
    rows = c["head_const"] and c["n"] != 96  # the row kernel's layout: required to take it
    if rows:
        diag.set("LQ_SSM_REQUIRE_ROWS")
    print(f"[ssm case {i}] {'rows' if rows else 'general'} {c}", flush=True)
    g = torch.Generator().manual_seed(600 + i)
    bsz, ng, n, p_ = c["bsz"], c["ng"], c["n"], c["p"]
    nh = ng * c["ratio"]
    sdt, xdt = DTYPES[c["sdt"]], DTYPES[c["xdt"]]
    # without the kernel's softplus, dt arrives already positive
    pos = (lambda v: v) if c["softplus"] else torch.nn.functional.softplus
    if c["head_const"]:  # the model's layout (stride-0 along head_dim): the row kernel
        dt = pos(torch.randn(bsz, nh, 1, generator=g)).to(xdt).expand(bsz, nh, p_)
        A = (-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n)
        D = torch.randn(nh, generator=g)[:, None].expand(nh, p_)
        dt_bias = (torch.randn(nh, generator=g) * 0.1)[:, None].expand(nh, p_)
    else:  # per-element dt, A, D, dt_bias: the general kernel
        dt = pos(torch.randn(bsz, nh, p_, generator=g)).to(xdt)
        A = -torch.rand(nh, p_, n, generator=g)
        D = torch.randn(nh, p_, generator=g)
        dt_bias = torch.randn(nh, p_, generator=g) * 0.1
    t = dict(x=torch.randn(bsz, nh, p_, generator=g).to(xdt), dt=dt, A=A,
             D=D if c["has_d"] else None, dt_bias=dt_bias if c["dtb"] else None,
             B=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
             C=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
             z=torch.randn(bsz, nh, p_, generator=g).to(xdt) if c["z"] else None)
    h0 = (torch.randn(bsz, nh, p_, n, generator=g) * 0.5).to(sdt)
    state = h0.to(gpu)
    dev = {k: to_device(v, gpu) for k, v in t.items()}
    out = ms.selective_state_update(state, dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"],
                                    D=dev["D"], z=dev["z"], dt_bias=dev["dt_bias"],
                                    dt_softplus=c["softplus"])
    torch.cuda.synchronize()
    _, ref_y = omx.bf16_state_update(h0.float(), t["x"], t["dt"], t["A"], t["B"], t["C"],
                                     t["D"], t["z"], t["dt_bias"], c["softplus"])
    rtol = 8e-3 if out.dtype == torch.bfloat16 else 2e-3
    assert_close_rel(out.float().cpu(), ref_y.to(out.dtype).float(), rtol=rtol,
                     what=f"y case {i}")
    ref_h = omx.update_math(h0.float(), t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["z"],
                            t["dt_bias"], c["softplus"])[0]
    if sdt == torch.float32:  # the kernel's fma rounds once where the oracle rounds twice
        assert_close_rel(state.cpu(), ref_h, rtol=1e-5, what=f"fp32 state case {i}")
        return
    ref_h = ref_h.to(sdt)
    gi = state.cpu().contiguous().view(BITS[sdt])
    ri = ref_h.contiguous().view(BITS[sdt])
    same = (gi == ri).double().mean().item()
    assert same >= 0.999, f"case {i}: only {same:.5f} of state values identical"
    gd, rd = state.cpu().double(), ref_h.double()
    bound = ULP[sdt] * rd.abs() + 1e-5 * rd.abs().mean()
    worst = ((gd - rd).abs() / bound).max().item()
    assert worst <= 1.0, f"case {i}: state differs by {worst:.3g} x the one-ulp bound"
