"""Host-side logic of the API-compatible modules, on the CPU with a stand-in Nemotron-H module:
patching, cache bookkeeping, masks, argument validation and fall-through paths."""
import math

import pytest
import torch

import fake_nemotron as fk
import hybrid_quant
from hybrid_quant import int4_8b_attention as ia
from hybrid_quant import mamba_state_8b_kernel as ms
from hybrid_quant import nemotron_8b_decode_eval as de
from oracle import int4_kv as oik


@pytest.fixture()
def model():
    fk.reset_module()
    torch.manual_seed(0)
    m = fk.FakeNemotronHForCausalLM(fk.make_config())
    yield m
    fk.reset_module()


def test_alias_modules_are_the_package_modules():
    import layer_quant_amd.int4_8b_attention as a
    import layer_quant_amd.mamba_state_8b_kernel as b

    assert ia is a and ms is b
    assert hybrid_quant.int4_8b_attention is a


def test_attention_patch_attributes_and_cpu_fallback(model):
    ids = torch.randint(0, 64, (2, 5))
    ref = model(ids)
    ia.patch_nemotron_h_attention_int4_kv(model, group_size=32)
    attn = [l.mixer for l in model.backbone.layers if l.block_type == "attention"]
    assert attn and all(a._int4_kv_patched and a._int4_kv_group_size == 32 for a in attn)
    assert all(a._int4_kv_repeat_kv is fk.repeat_kv for a in attn)
    first = attn[0].forward
    ia.patch_nemotron_h_attention_int4_kv(model, group_size=64)  # idempotent
    assert attn[0].forward is first and attn[0]._int4_kv_group_size == 32
    # CPU hidden states take the original forward
    assert torch.allclose(model(ids), ref)


def test_block_patch_routes_cache_to_attention(model):
    de.patch_attention_cache_in_blocks(model)
    assert all(b._decode_eval_block_patched for b in model.backbone.layers)
    cache = de.make_hybrid_cache(model, 2)
    assert isinstance(cache.ssm_states, de.DeviceList) and cache.conv_kernel_size == 4
    model(torch.randint(0, 64, (2, 3)), cache_params=cache)
    attn_layers = [i for i, l in enumerate(model.backbone.layers) if l.block_type == "attention"]
    assert sorted(cache.key_cache) == attn_layers


def test_layer_groups_and_adjacency():
    cfg = fk.make_config(hybrid_override_pattern="M-M*-MM*M-")
    mamba, attn, mlp = de.layer_groups(cfg)
    assert mamba == [0, 2, 5, 6, 8] and attn == [3, 7] and mlp == [1, 4, 9]
    assert de.adjacent_mamba_layers(mamba, attn) == {2, 5, 6, 8}


def test_positions():
    assert ia._positions(None, 3, torch.device("cpu")).tolist() == [0, 1, 2]
    assert ia._positions(torch.tensor([7]), 1, torch.device("cpu")).tolist() == [7]
    assert ia._positions(torch.tensor([4, 5]), 2, torch.device("cpu")).dtype == torch.long
    with pytest.raises(ValueError, match="cache_position has 2 entries for q_len=3"):
        ia._positions(torch.tensor([4, 5]), 3, torch.device("cpu"))


def test_layer_cache_capacity_and_growth():
    holder = type("Cache", (), {})()
    dev = torch.device("cpu")
    c = ia._ensure_layer_cache(holder, 3, 2, 4, 5, 128, 32, dev)
    assert c.k_packed.shape == (2, 4, 16, 64) and c.k_scale.shape == (2, 4, 16, 4)
    assert ia._ensure_layer_cache(holder, 3, 2, 4, 16, 128, 32, dev) is c
    c.k_packed.fill_(7)
    c.v_scale.fill_(0.5)
    c.length = 16
    g = ia._ensure_layer_cache(holder, 3, 2, 4, 17, 128, 32, dev)
    assert g is not c and g.k_packed.shape[2] == 32 and g.length == 16
    assert torch.all(g.k_packed[:, :, :16] == 7) and torch.all(g.v_scale[:, :, :16] == 0.5)
    assert holder._int4_kv_layer_caches[3] is g
    big = ia._ensure_layer_cache(holder, 5, 1, 1, 1000, 128, 64, dev)
    assert big.k_packed.shape[2] == 1024 and big.k_scale.shape[3] == 2
    with pytest.raises(ValueError, match="does not match batch/kv_heads"):
        ia._ensure_layer_cache(holder, 3, 3, 4, 5, 128, 32, dev)


def test_decode_attention_validates_before_launch():
    cache = ia._allocate_layer_cache(1, 2, 16, 128, 4, torch.device("cpu"))
    with pytest.raises(ValueError, match="expects q_len=1, got 2"):
        ia._decode_attention(torch.zeros(1, 8, 2, 128), cache, 4, 4, 32)


def test_mask_matches_oracle():
    keep = torch.tensor([[1, 0, 1, 1, 1, 1], [1, 1, 1, 0, 1, 1]])
    for s in (3, 6):
        assert torch.equal(ia._decode_attention_mask(keep, 2, s, torch.device("cpu")),
                           oik.decode_attention_mask(keep, 2, s))
    m4 = torch.randn(2, 1, 4, 9)
    assert torch.equal(ia._decode_attention_mask(m4, 2, 7, torch.device("cpu")),
                       oik.decode_attention_mask(m4, 2, 7))
    m4b = torch.rand(2, 1, 4, 9) > 0.3
    assert torch.equal(ia._decode_attention_mask(m4b, 2, 7, torch.device("cpu")),
                       oik.decode_attention_mask(m4b, 2, 7))
    assert ia._decode_attention_mask(None, 2, 7, torch.device("cpu")) is None
    with pytest.raises(ValueError, match="got 3D"):
        ia._decode_attention_mask(torch.ones(2, 1, 7), 2, 7, torch.device("cpu"))


def test_int4_quant_dequant_matches_oracle():
    x = torch.randn(3, 5, 128, dtype=torch.bfloat16) * 4
    for g in (32, 64):
        q, s = oik.quantize_groups(x, g)
        ref = (q.float() * s.repeat_interleave(g, -1)).to(torch.bfloat16)
        assert torch.equal(ia.int4_quant_dequant(x, g), ref)
    with pytest.raises(ValueError, match="must be divisible by group_size=48"):
        ia.int4_quant_dequant(x, 48)


def test_mx_argument_validation():
    with pytest.raises(ValueError, match="MX8 uses a fixed 16-value block, got group_size=32"):
        ms.allocate_state_kernel_cache(torch.zeros(1, 2, 2, 32), group_size=32, format_bits=8)
    with pytest.raises(ValueError, match="got format_bits=6"):
        ms.allocate_state_kernel_cache(torch.zeros(1, 2, 2, 32), format_bits=6)
    with pytest.raises(ValueError, match="divisible by 16, got 40"):
        ms._quantize_initial_state_mx(torch.zeros(1, 40), format_bits=8, block_size=16,
                                      pair_size=2, mantissa_max=63.0)
    cache = ms.MambaStateKernelCache(torch.zeros(2, 4, 8, 32, dtype=torch.int8),
                                     torch.zeros(2, 4, 8, 2, dtype=torch.uint8),
                                     torch.zeros(2, 4, 8, 16, dtype=torch.uint8))
    A = torch.zeros(4, 8, 32)
    B = torch.zeros(2, 2, 32)
    with pytest.raises(ValueError, match=r"Expected x shape \(2, 4, 8\)"):
        ms.mx_state_selective_update(cache, torch.zeros(2, 4, 7), torch.zeros(2, 4, 7), A, B, B)
    with pytest.raises(ValueError, match="Expected B and C"):
        ms.mx_state_selective_update(cache, torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), A,
                                     torch.zeros(2, 64), B)
    cache.format_bits = 6
    with pytest.raises(ValueError, match="format_bits=6"):
        ms.mx_state_selective_update(cache, torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), A, B, B)
    with pytest.raises(ValueError, match="q_state"):
        ms.mx_state_selective_update(ms.MambaStateKernelCache(torch.zeros(2, 3), None, None),
                                     torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), A, B, B)
    with pytest.raises(ValueError, match="rng must be 'counter' or 'philox'"):
        ms.mx_state_selective_update(cache, torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), A, B, B,
                                     rng="pcg")


def test_dt_bias_is_read_with_D_strides():
    dtb = torch.arange(8.0)
    D_exp = torch.randn(8)[:, None].expand(8, 4)
    view = ms._dt_bias_as_read(dtb[:, None].expand(8, 4), D_exp, 8, 4)
    assert torch.equal(view, dtb[:, None].expand(8, 4))
    # D absent: the reference reads dt_bias[0, 0] for every row
    view0 = ms._dt_bias_as_read(dtb[:, None].expand(8, 4), None, 8, 4)
    assert torch.equal(view0, torch.zeros(8, 4))
    # D contiguous while dt_bias is an expanded [H] vector: the reads would leave its storage
    with pytest.raises(ValueError, match="storage"):
        ms._dt_bias_as_read(dtb[:, None].expand(8, 4), torch.randn(8, 4), 8, 4)
    assert ms._dt_bias_as_read(None, D_exp, 8, 4) is None


def test_mamba_patch_falls_through_for_unregistered_states(model):
    ms.patch_nemotron_h_mamba_decode_state_kernel(model, stochastic=False, seed=7)
    assert fk._mx_state_kernel_patched and fk._mx_state_kernel_seed == 7
    assert fk._mx_state_kernel_stochastic is False
    assert fk.selective_state_update is not fk._mx_state_kernel_original
    assert model._mx_state_kernel_group_size == 16
    state = torch.zeros(1, 2, 2, 16)
    x = torch.ones(1, 2, 2)
    dt = torch.ones(1, 2, 2)
    A = -torch.ones(2, 2, 16)
    B = torch.ones(1, 1, 16)
    y = fk.selective_state_update(state, x, dt, A, B, B)
    ref_state = torch.zeros(1, 2, 2, 16)
    yr = fk._mx_state_kernel_original(ref_state, x, dt, A, B, B)
    assert torch.equal(y, yr) and torch.equal(state, ref_state)
    # patching again keeps the first original and updates the knobs
    ms.patch_nemotron_h_mamba_decode_state_kernel(model, stochastic=True, seed=9)
    assert fk._mx_state_kernel_seed == 9 and fk._mx_state_kernel_original is not None


def test_register_rejects_unknown_mode(model):
    cache = de.make_hybrid_cache(model, 1)
    with pytest.raises(ValueError, match="mode='mx6'"):
        ms.register_mamba_state_kernel_caches(model, cache, {0: "mx6"})


def test_mx_constants():
    assert (ms.MX8_BLOCK_SIZE, ms.MX8_PAIR_SIZE, ms.MX8_MANTISSA_MAX) == (16, 2, 63.0)
    assert (ms.MX4_BLOCK_SIZE, ms.MX4_PAIR_SIZE, ms.MX4_MANTISSA_MAX) == (16, 2, 7.0)
    assert math.isclose(ms.MX4_MANTISSA_MAX, 7)


def test_mx8_mx4_aliases_forward_every_argument(monkeypatch):
    """mx8_/mx4_state_selective_update (ms.py:724-729) call mx_state_selective_update with the
    caller's positional and keyword arguments unchanged."""
    seen = []
    monkeypatch.setattr(ms, "mx_state_selective_update",
                        lambda *a, **k: seen.append((a, k)) or "y")
    assert ms.mx8_state_selective_update(1, 2, D=3, stochastic=False) == "y"
    assert ms.mx4_state_selective_update("c", seed=9) == "y"
    assert seen == [((1, 2), {"D": 3, "stochastic": False}), (("c",), {"seed": 9})]


def test_load_wikitext_texts_filters_blank_lines(monkeypatch, tmp_path):
    """The driver's text source keeps the non-whitespace lines of the split and passes a local
    directory as a path, anything else as a dataset name (reference data.py:14-20)."""
    import sys
    import types

    from hybrid_quant import data

    calls = []

    def load_dataset(source, config, split):
        calls.append((source, config, split))
        return {"text": ["a", "", "  \n", " b ", "\n"]}

    monkeypatch.setitem(sys.modules, "datasets", types.SimpleNamespace(load_dataset=load_dataset))
    assert data.load_wikitext_texts("wikitext") == ["a", " b "]
    assert data.load_wikitext_texts(str(tmp_path), split="validation") == ["a", " b "]
    assert calls == [("wikitext", "wikitext-103-raw-v1", "test"),
                     (str(tmp_path), "wikitext-103-raw-v1", "validation")]


def test_token_segments_window_boundaries():
    """token_segments (reference data.py:23-32): windows of up to context_length + 1 tokens
    starting every context_length tokens, sharing one token with the next window, over the
    first min(n - 1, max_eval_tokens) predicted tokens of the texts joined by blank lines."""
    from types import SimpleNamespace


    from hybrid_quant import data

    seen = []

    def tokenizer(text, add_special_tokens, return_tensors):
        seen.append((text, add_special_tokens, return_tensors))
        return SimpleNamespace(input_ids=torch.arange(len(text)).unsqueeze(0))

    def windows(n, ctx, cap):
        seen.clear()
        out = [w.tolist() for w in data.token_segments(tokenizer, ["x" * (n - 2), ""], ctx, cap)]
        assert seen == [("x" * (n - 2) + "\n\n", False, "pt")]
        return out

    r = list(range(11))
    # 11 tokens, 10 predicted: starts 0, 4, 8; the last window is short
    assert windows(11, 4, 100) == [r[0:5], r[4:9], r[8:11]]
    # max_eval_tokens caps the predicted tokens at 6: the last window ends at token 6
    assert windows(11, 4, 6) == [r[0:5], r[4:7]]
    # an exact multiple: 8 predicted tokens in two full windows
    assert windows(9, 4, 100) == [r[0:5], r[4:9]]
    # one token per window (context 1): every window is an (input, target) pair
    assert windows(4, 1, 100) == [[0, 1], [1, 2], [2, 3]]
    # two tokens: one window; nothing to predict with fewer
    assert windows(2, 4, 100) == [[0, 1]]
    assert windows(2, 4, 0) == []
    with pytest.raises(ValueError):
        next(data.token_segments(tokenizer, ["abc"], 0, 10))
    # every predicted token is the target of exactly one window
    targets = [t for w in windows(50, 7, 40) for t in w[1:]]
    assert targets == list(range(1, 41))
