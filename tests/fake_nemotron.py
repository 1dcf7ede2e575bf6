"""A small stand-in for the remote Nemotron-H modeling module (test double).

It has just the surface that the reference's patch / register functions touch:
model.backbone.layers[i].{block_type, mixer, norm, residual_in_fp32}; attention mixers with
q/k/v/o projections, num_heads, head_dim, num_key_value_heads, num_key_value_groups,
hidden_size, layer_idx, attention_dropout; Mamba mixers with num_heads, head_dim,
ssm_state_size whose decode step (one token with a cache) calls the module-level
`selective_state_update` (looked up at call time, so rebinding it takes effect) on the cache's
own [B, H, P, N] state tensor, as the remote module does, so an id()-keyed registry finds it;
module-level `repeat_kv` and `HybridMambaAttentionDynamicCache`. A remote module imported
without mamba-ssm has `selective_state_update = None`; tests emulate that by setting it to
None before patching. Weights are random; nothing here is the real model.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    b, h, s, d = hidden_states.shape
    if n_rep == 1:
        return hidden_states
    return hidden_states[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False):
    """Plain fp32 recurrent update of a float state, in place; returns y in x's dtype."""
    nheads = state.shape[1]
    ratio = nheads // B.shape[1]
    dtf = dt.float() + (dt_bias.float() if dt_bias is not None else 0.0)
    if dt_softplus:
        dtf = F.softplus(dtf)
    Bh = B.float().repeat_interleave(ratio, 1)[:, :, None, :]
    Ch = C.float().repeat_interleave(ratio, 1)[:, :, None, :]
    new = state.float() * torch.exp(A.float() * dtf[..., None]) + Bh * (dtf * x.float())[..., None]
    state.copy_(new.to(state.dtype))
    y = (new * Ch).sum(-1)
    if D is not None:
        y = y + x.float() * D.float()
    if z is not None:
        y = y * F.silu(z.float())
    return y.to(x.dtype)


def make_config(**overrides):
    cfg = dict(hybrid_override_pattern="M*M-M*", hidden_size=256, num_attention_heads=8,
               num_key_value_heads=2, head_dim=32 * 4, mamba_num_heads=8, mamba_head_dim=16,
               ssm_state_size=32, n_groups=2, conv_kernel=4, vocab_size=64)
    cfg.update(overrides)
    cfg["hidden_size"] = cfg["num_attention_heads"] * cfg["head_dim"]
    return SimpleNamespace(**cfg)


class HybridMambaAttentionDynamicCache:
    def __init__(self, config, batch_size, dtype, device=None):
        self.ssm_states, self.conv_states = [], []
        self.key_cache, self.value_cache = {}, {}
        for kind in config.hybrid_override_pattern:
            if kind == "M":
                self.ssm_states.append(torch.zeros(
                    batch_size, config.mamba_num_heads, config.mamba_head_dim,
                    config.ssm_state_size, dtype=dtype, device=device))
            else:
                self.ssm_states.append(torch.zeros(0, device=device))
            self.conv_states.append(torch.zeros(0, device=device))


class FakeAttention(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = self.num_heads // self.num_key_value_heads
        self.head_dim = config.head_dim
        self.hidden_size = config.hidden_size
        self.attention_dropout = 0.0
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=False)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
                output_attentions=False, use_cache=False, cache_position=None):
        bsz, q_len, _ = hidden_states.shape

        def heads(proj, n):
            return proj(hidden_states).view(bsz, q_len, n, self.head_dim).transpose(1, 2)

        q = heads(self.q_proj, self.num_heads)
        k = heads(self.k_proj, self.num_key_value_heads)
        v = heads(self.v_proj, self.num_key_value_heads)
        if past_key_value is not None:
            if self.layer_idx in past_key_value.key_cache:
                k = torch.cat([past_key_value.key_cache[self.layer_idx], k], dim=2)
                v = torch.cat([past_key_value.value_cache[self.layer_idx], v], dim=2)
            past_key_value.key_cache[self.layer_idx] = k
            past_key_value.value_cache[self.layer_idx] = v
        k = repeat_kv(k, self.num_key_value_groups)
        v = repeat_kv(v, self.num_key_value_groups)
        out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                             is_causal=q_len > 1).to(q.dtype)
        out = out.transpose(1, 2).reshape(bsz, q_len, self.hidden_size)
        return self.o_proj(out), None, past_key_value


class FakeMamba(nn.Module):
    """Decode-only Mamba2 mixer: projections, then the module-level selective_state_update."""

    def __init__(self, config, layer_idx):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = config.mamba_num_heads
        self.head_dim = config.mamba_head_dim
        self.ssm_state_size = config.ssm_state_size
        self.n_groups = config.n_groups
        inner = self.num_heads * self.head_dim
        self.in_proj = nn.Linear(config.hidden_size,
                                 inner + 2 * self.n_groups * self.ssm_state_size + self.num_heads,
                                 bias=False)
        self.out_proj = nn.Linear(inner, config.hidden_size, bias=False)
        self.A_log = nn.Parameter(torch.rand(self.num_heads) * 2)
        self.D = nn.Parameter(torch.randn(self.num_heads))
        self.dt_bias = nn.Parameter(torch.randn(self.num_heads) * 0.1)

    def _step_args(self, proj):
        bsz = proj.shape[0]
        inner = self.num_heads * self.head_dim
        gn = self.n_groups * self.ssm_state_size
        x, B, C, dt = torch.split(proj, [inner, gn, gn, self.num_heads], dim=-1)
        return (x.reshape(bsz, self.num_heads, self.head_dim),
                dt[:, :, None].expand(-1, -1, self.head_dim),
                (-torch.exp(self.A_log.float()))[:, None, None].expand(-1, self.head_dim,
                                                                      self.ssm_state_size),
                B.reshape(bsz, self.n_groups, self.ssm_state_size),
                C.reshape(bsz, self.n_groups, self.ssm_state_size),
                self.D[:, None].expand(-1, self.head_dim),
                self.dt_bias[:, None].expand(-1, self.head_dim))

    def forward(self, hidden_states, cache_params=None, cache_position=None, attention_mask=None):
        bsz, seq_len, _ = hidden_states.shape
        inner = self.num_heads * self.head_dim
        proj = self.in_proj(hidden_states)
        if cache_params is not None and seq_len == 1:
            # decode: the (possibly rebound) module-level update on the cache's own state object
            x, dt, A, B, C, D, dt_bias = self._step_args(proj[:, 0])
            ssm_update = globals()["selective_state_update"]
            y = ssm_update(cache_params.ssm_states[self.layer_idx], x, dt, A, B, C, D, z=None,
                           dt_bias=dt_bias, dt_softplus=True)
            return self.out_proj(y.reshape(bsz, 1, inner))
        # prefill (the remote module's chunked scan): the same recurrence token by token in
        # fp32, leaving the final state in the cache
        state = torch.zeros(bsz, self.num_heads, self.head_dim, self.ssm_state_size,
                            device=hidden_states.device)
        ys = []
        for t in range(seq_len):
            x, dt, A, B, C, D, dt_bias = self._step_args(proj[:, t])
            ys.append(_torch_selective_state_update(state, x, dt, A, B, C, D, dt_bias=dt_bias,
                                                    dt_softplus=True))
        if cache_params is not None:
            cache_params.ssm_states[self.layer_idx].copy_(state)
        y = torch.stack(ys, dim=1)
        return self.out_proj(y.reshape(bsz, seq_len, inner))


class FakeMLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.fc = nn.Linear(config.hidden_size, config.hidden_size, bias=False)

    def forward(self, hidden_states):
        return self.fc(hidden_states)


class Block(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        kind = config.hybrid_override_pattern[layer_idx]
        self.block_type = {"M": "mamba", "*": "attention", "-": "mlp"}[kind]
        self.residual_in_fp32 = True
        self.norm = nn.LayerNorm(config.hidden_size)
        if kind == "M":
            self.mixer = FakeMamba(config, layer_idx)
        elif kind == "*":
            self.mixer = FakeAttention(config, layer_idx)
        else:
            self.mixer = FakeMLP(config)

    def forward(self, hidden_states, cache_params=None, cache_position=None, attention_mask=None):
        residual = hidden_states
        hidden_states = self.norm(hidden_states.to(dtype=self.norm.weight.dtype))
        if self.block_type == "mamba":
            hidden_states = self.mixer(hidden_states, cache_params=cache_params)
        elif self.block_type == "attention":
            hidden_states = self.mixer(hidden_states)[0]
        else:
            hidden_states = self.mixer(hidden_states)
        return residual.float() + hidden_states


class Backbone(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.embeddings = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [Block(config, i) for i in range(len(config.hybrid_override_pattern))])


class FakeNemotronHForCausalLM(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.backbone = Backbone(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)

    @property
    def device(self):
        return self.lm_head.weight.device

    def forward(self, input_ids, cache_params=None, cache_position=None, attention_mask=None,
                use_cache=False, return_dict=False):
        h = self.backbone.embeddings(input_ids)
        for layer in self.backbone.layers:
            h = layer(h, cache_params=cache_params, cache_position=cache_position,
                      attention_mask=attention_mask).to(self.lm_head.weight.dtype)
        logits = self.lm_head(h)
        return SimpleNamespace(logits=logits) if return_dict else logits


_torch_selective_state_update = selective_state_update


def reset_module():
    """Undo every attribute the patch functions set on this module (and a None
    selective_state_update set by a test)."""
    g = globals()
    g["selective_state_update"] = _torch_selective_state_update
    for name in ("_mx_state_kernel_original", "_mx_state_kernel_patched",
                 "_mx_state_kernel_stochastic", "_mx_state_kernel_seed",
                 "_mamba_decode_state_kernel_caches"):
        g.pop(name, None)
