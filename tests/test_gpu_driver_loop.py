"""The reference driver's decode loop on the GPU, through the patched stand-in model.

Follows run_decode_ppl (reference run_nemotron_8b_decode_degradation.py:95-133) and main()'s
patching (:253-275): patch_attention_cache_in_blocks, patch_nemotron_h_attention_int4_kv
(group 64, the driver's --kv-group-size default), patch_nemotron_h_mamba_decode_state_kernel;
a prefill of the context, register_mamba_state_kernel_caches for a mixed {mx8, mx4} plan, then
decode steps with the driver's model call and loss.

The remote module is emulated as imported without mamba-ssm (selective_state_update = None), so
layers left out of the plan take this library's HIP bf16-state update. Every decode step is
checked against the oracle:
  * each attention layer's INT4 cache equals the oracle's pack of the layer's K/V projections,
    rows [0, length) bit for bit (reference int4_8b_attention.py:477-515), and its output equals
    the float64 oracle attention over that cache (:518-566) within the bf16-output bar;
  * each registered Mamba layer's MX state after the step equals the oracle's update of the
    state before the step (mamba_state_8b_kernel.py:97-222, 289-544) except at encoder decision
    ties (helpers.assert_mx_writeback: the oracle's h' within 2^-20 of |h*dA| + |dt*B*x| of a
    block-exponent, micro-exponent or rounding threshold; one level at most there), and y is
    within the bf16-output bar, with the driver's counter-based stochastic rounding (or half-up
    with --deterministic);
  * each unregistered layer's bf16 state equals the oracle's fp32 update rounded to bf16 on
    >= 99.9% of its elements (elsewhere within one bf16 ulp plus the hardware exp/log error
    on h*dA + dt*B*x) -- the HIP fallback, not a torch one.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fake_nemotron as fk
from helpers import assert_close_rel, assert_mx_writeback, update_term_magnitudes
from hybrid_quant import int4_8b_attention as ia
from hybrid_quant import mamba_state_8b_kernel as ms
from hybrid_quant import nemotron_8b_decode_eval as de
from oracle import int4_kv as oik
from oracle import mx_state as omx

pytestmark = pytest.mark.gpu

KV_GROUP = 64
PLAN = {0: "mx8", 2: "mx4", 4: "mx4"}  # layer 6 stays unregistered


def _assert_bf16_state_close(got: torch.Tensor, before: torch.Tensor, x, dt, A, B, C, D,
                             dt_bias, dt_softplus):
    """The stored bf16 state against the oracle's fp32 update h' = h*dA + dt*B*x: identical to
    RNE(h') on >= 99.9% of elements, and everywhere within one bf16 ulp of h' plus 2^-20 of
    |h*dA| + |dt*B*x|. The slack is the error of the hardware exp/log the kernel uses for dA and
    softplus (about 1e-6 relative, as the reference's Triton tl.exp/tl.log); it decides the
    result only where the two terms cancel (one element in about 4e5 in this test's data)."""
    h2, _ = omx.update_math(before.float(), x, dt, A, B, C, D, None, dt_bias, dt_softplus)
    mag, _ = omx.update_math(before.float().abs(), x.float().abs(), dt, A, B.float().abs(), C,
                             D, None, dt_bias, dt_softplus)
    ref = h2.to(torch.bfloat16)
    same = (got == ref).float().mean().item()
    assert same > 0.999, f"only {same:.5f} of bf16 state elements identical"
    g = got.double()
    ulp = torch.ldexp(torch.ones_like(g), torch.frexp(h2.double().abs().clamp_min(2.0 ** -126))[1]
                      - 8)
    bound = ulp + 2.0 ** -20 * mag.double()
    err = (g - h2.double()).abs()
    worst = torch.argmax(err / bound)
    idx = np.unravel_index(worst.item(), tuple(g.shape))
    assert torch.all(err <= bound), (
        f"a bf16 state element is off by more than one ulp plus the exp/log slack: at "
        f"{idx} got {g.flatten()[worst].item():.9g} oracle h' {h2.flatten()[worst].item():.9g} "
        f"bound {bound.flatten()[worst].item():.3g} |h*dA|+|dt*B*x| {mag.flatten()[worst].item():.3g} "
        f"h {before.flatten()[worst].item():.9g} x {x[idx[:3]].item():.6g} "
        f"dt {dt[idx[:3]].item():.6g} dt_bias {dt_bias[idx[1:3]].item():.6g} "
        f"A {A[idx[1:]].item():.6g}; {(err > bound).sum().item()} of {err.numel()} elements")


class _Recorder:
    """Wraps the rebound module-level selective_state_update: snapshots each call's inputs and
    the state (MX tensors or bf16 state) before and after, and the output."""

    def __init__(self, inner):
        self.inner = inner
        self.calls = []

    def __call__(self, ssm_state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                 dt_softplus=False):
        registry = getattr(fk, "_mamba_decode_state_kernel_caches", {})
        mx = registry.get(id(ssm_state))
        snap = (lambda: tuple(t.cpu().numpy().copy() for t in
                              (mx.q_state, mx.shared_exp, mx.micro_exp))) if mx is not None \
            else (lambda: ssm_state.detach().cpu().clone())
        entry = dict(mx=mx, step=None if mx is None else mx.step, before=snap(),
                     args=[t.detach().cpu().clone() for t in (x, dt, A, B, C)],
                     D=None if D is None else D.detach().cpu().clone(),
                     dt_bias=None if dt_bias is None else dt_bias.detach().cpu().clone(),
                     dt_softplus=dt_softplus, shape=tuple(ssm_state.shape))
        y = self.inner(ssm_state, x, dt, A, B, C, D=D, z=z, dt_bias=dt_bias,
                       dt_softplus=dt_softplus)
        entry["after"] = snap()
        entry["y"] = y.detach().float().cpu()
        self.calls.append(entry)
        return y


def _attention_taps(model):
    """Forward hooks that capture each attention layer's q/k/v projections and o_proj input."""
    taps = {}
    for idx, layer in enumerate(model.backbone.layers):
        if layer.block_type != "attention":
            continue
        rec = taps.setdefault(idx, {})
        m = layer.mixer
        for name in ("q_proj", "k_proj", "v_proj"):
            getattr(m, name).register_forward_hook(
                lambda mod, inp, out, rec=rec, name=name: rec.__setitem__(name, out.detach()))
        m.o_proj.register_forward_pre_hook(
            lambda mod, inp, rec=rec: rec.__setitem__("attn", inp[0].detach()))
    return taps


def _heads(t, n, d):
    b, L, _ = t.shape
    return t.view(b, L, n, d).transpose(1, 2).contiguous().cpu()


@pytest.mark.parametrize("stochastic", [True, False])
def test_driver_decode_loop(gpu, diag, stochastic):
    # every decode-step call of the patched model must take the library's fast kernels: the MFMA
    # attention, the MX row kernel and, for the unregistered layers, the unquantized row kernel
    for name in ("LQ_ATTN_REQUIRE_FAST", "LQ_MX_REQUIRE_ROWS", "LQ_SSM_REQUIRE_ROWS"):
        diag.set(name)
    fk.reset_module()
    torch.manual_seed(0)
    cfg = fk.make_config(hybrid_override_pattern="M*M-M*M", num_attention_heads=8,
                         num_key_value_heads=2, head_dim=128, mamba_num_heads=16,
                         mamba_head_dim=64, ssm_state_size=128, n_groups=2, vocab_size=128)
    model = fk.FakeNemotronHForCausalLM(cfg).to(torch.bfloat16).to(gpu).eval()
    batch, context, steps, seed = 3, 60, 9, 1234
    ids = torch.randint(0, cfg.vocab_size, (batch, context + steps + 1), device=gpu)
    try:
        fk.selective_state_update = None  # remote module without mamba-ssm
        de.patch_attention_cache_in_blocks(model)
        ia.patch_nemotron_h_attention_int4_kv(model, group_size=KV_GROUP)
        ms.patch_nemotron_h_mamba_decode_state_kernel(model, group_size=16,
                                                      stochastic=stochastic, seed=seed)
        assert fk._mx_state_kernel_original is ms.selective_state_update
        recorder = _Recorder(fk.selective_state_update)
        fk.selective_state_update = recorder
        taps = _attention_taps(model)
        attn_layers = sorted(taps)
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        nrep = hq // hkv
        oracle_caches = {i: oik.allocate_cache(batch, hkv, context + steps, d, KV_GROUP)
                         for i in attn_layers}
        cache = de.make_hybrid_cache(model, batch_size=batch)

        def check_attention(positions, decode):
            for i in attn_layers:
                rec = taps[i]
                oc = oracle_caches[i]
                oik.pack_kv_into_cache(oc, _heads(rec["k_proj"], hkv, d),
                                       _heads(rec["v_proj"], hkv, d), positions, KV_GROUP)
                lc = cache._int4_kv_layer_caches[i]
                n = lc.length
                assert n == oc["length"]
                for name in ("k_packed", "v_packed", "k_scale", "v_scale"):
                    assert torch.equal(getattr(lc, name)[:, :, :n].cpu(), oc[name][:, :, :n]), \
                        f"layer {i} {name} differs from the oracle pack"
                if decode:
                    q = _heads(rec["q_proj"], hq, d)
                    ref = oik.decode_attention(q, oc["k_packed"], oc["v_packed"],
                                               oc["k_scale"], oc["v_scale"], n, nrep, KV_GROUP)
                    got = rec["attn"].float().view(batch, hq, d).cpu()
                    assert_close_rel(got, ref, rtol=8e-3, what=f"attention layer {i}")

        with torch.inference_mode():
            prefill_pos = torch.arange(context, device=gpu, dtype=torch.long)
            model(input_ids=ids[:, :context], cache_params=cache, cache_position=prefill_pos,
                  use_cache=True, return_dict=True)
            check_attention(torch.arange(context), decode=False)
            ms.register_mamba_state_kernel_caches(model, cache, PLAN)
            registry = fk._mamba_decode_state_kernel_caches
            assert len(registry) == len(PLAN)
            for idx, mode in PLAN.items():
                mx = registry[id(cache.ssm_states[idx])]
                assert mx.format_bits == (8 if mode == "mx8" else 4) and mx.step == 0
                ref = omx.mx_encode(cache.ssm_states[idx].float().cpu().numpy(),
                                    mx.format_bits, omx.ROUND_NEAREST_EVEN)
                for a, r in zip((mx.q_state, mx.shared_exp, mx.micro_exp), ref):
                    assert np.array_equal(a.cpu().numpy(), r), f"initial encode of layer {idx}"

            total_nll, total_tokens = 0.0, 0
            for step in range(steps):
                recorder.calls.clear()
                pos = context + step
                cache_pos = torch.tensor([pos], device=gpu, dtype=torch.long)
                outputs = model(input_ids=ids[:, pos:pos + 1], cache_params=cache,
                                cache_position=cache_pos, use_cache=True, return_dict=True)
                loss = F.cross_entropy(outputs.logits[:, -1, :].float(), ids[:, pos + 1],
                                       reduction="sum")
                total_nll += float(loss.item())
                total_tokens += batch
                check_attention(torch.tensor([pos]), decode=True)
                assert len(recorder.calls) == 4  # one per Mamba layer
                n_mx = 0
                for call in recorder.calls:
                    x, dt, A, B, C = call["args"]
                    if call["mx"] is not None:
                        n_mx += 1
                        mx = call["mx"]
                        b_, h_, p_, n_ = call["shape"]
                        assert mx.step == call["step"] + 1
                        mode = omx.ROUND_SR_COUNTER if stochastic else omx.ROUND_HALF_UP
                        off = call["step"] * b_ * h_ * p_ * n_
                        rq, re_, rm, y_ref, rh = omx.mx_update(
                            *call["before"], x, dt, A, B, C, D=call["D"], z=None,
                            dt_bias=call["dt_bias"], dt_softplus=call["dt_softplus"],
                            format_bits=mx.format_bits, round_mode=mode, seed=seed,
                            rng_offset=off)
                        mag = update_term_magnitudes(omx.mx_decode(*call["before"]), x, dt, A,
                                                     B, C, dt_bias=call["dt_bias"],
                                                     dt_softplus=call["dt_softplus"])
                        assert_mx_writeback(call["after"], (rq, re_, rm), rh, mag,
                                            mx.format_bits, mode, seed=seed, rng_offset=off,
                                            what=f"step {step} mx{mx.format_bits}")
                        assert_close_rel(call["y"], y_ref, rtol=8e-3, what="MX y")
                    else:
                        _, y_ref = omx.bf16_state_update(
                            call["before"], x, dt, A, B, C, D=call["D"], z=None,
                            dt_bias=call["dt_bias"], dt_softplus=call["dt_softplus"])
                        _assert_bf16_state_close(call["after"], call["before"], x, dt, A, B, C,
                                                 call["D"], call["dt_bias"], call["dt_softplus"])
                        assert_close_rel(call["y"], y_ref, rtol=8e-3, what="bf16-state y")
                assert n_mx == len(PLAN)
            assert np.isfinite(total_nll) and total_tokens == batch * steps
            # the INT4 caches grew past their prefill capacity (64 rows) during decode
            assert all(cache._int4_kv_layer_caches[i].k_packed.shape[2] == 128
                       for i in attn_layers)
    finally:
        fk.reset_module()
