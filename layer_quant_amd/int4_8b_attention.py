"""INT4 KV cache and fused q_len=1 decode attention for Nemotron-H attention layers.

API-compatible with the reference module hybrid_quant/int4_8b_attention.py (cited as ia.py:line):
the same public names, argument meaning and error messages, with the two Triton kernels replaced
by HIP kernels for gfx950 behind the C ABI (include/layer_quant.h):

    _pack_int4_kv_kernel            -> lq_int4_pack_kv            (ia.py:32-111)
    _int4_decode_attention_kernel   -> lq_int4_decode_attention   (ia.py:254-402)
    _int4_prefill_attention_kernel  -> lq_int4_prefill_attention  (ia.py:114-251)

The reference never calls its prefill kernel (the patched forward runs SDPA on unquantized K/V
for q_len > 1, ia.py:693-714, and so does this module); _prefill_attention keeps its
signature (ia.py:594-625) for callers that attend over the packed cache instead.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from types import MethodType

import torch

from . import _abi


@dataclass
class Int4KVLayerCache:
    """Packed per-layer cache (ia.py:12-18): nibbles [B, Hkv, cap, D/2] uint8, fp32 group
    scales [B, Hkv, cap, D/g], and the number of valid rows."""

    k_packed: torch.Tensor
    v_packed: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    length: int = 0


def int4_quant_dequant(x: torch.Tensor, group_size: int = 64) -> torch.Tensor:
    """Fake-quantize x along its last dim with the cache's INT4 group format (ia.py:21-29).

    Plain torch on any device: absmax scale max(absmax/7, 1e-8), round half to even, clamp to
    [-8, 7], multiply back, return in x's dtype.
    """
    d = x.shape[-1]
    if d % group_size != 0:
        raise ValueError(f"head_dim={d} must be divisible by group_size={group_size}")
    groups = x.float().reshape(*x.shape[:-1], d // group_size, group_size)
    scale = (groups.abs().amax(dim=-1, keepdim=True) / 7.0).clamp_min(1.0e-8)
    levels = (groups / scale).round().clamp(-8.0, 7.0)
    return (levels * scale).reshape(x.shape).to(x.dtype)


def _cache_dict(past_key_value) -> dict[int, Int4KVLayerCache]:
    """Per-layer caches stored on the HF cache object as `_int4_kv_layer_caches` (ia.py:405-410)."""
    caches = getattr(past_key_value, "_int4_kv_layer_caches", None)
    if caches is None:
        caches = {}
        past_key_value._int4_kv_layer_caches = caches
    return caches


def _positions(cache_position, q_len: int, device: torch.device) -> torch.Tensor:
    """Cache rows of the new tokens (ia.py:413-420)."""
    if cache_position is None:
        return torch.arange(q_len, device=device, dtype=torch.long)
    n = cache_position.numel()
    if n == q_len or (n == 1 and q_len == 1):
        return cache_position.to(device=device, dtype=torch.long)
    raise ValueError(f"cache_position has {n} entries for q_len={q_len}")


def _allocate_layer_cache(batch: int, kv_heads: int, capacity: int, head_dim: int, groups: int,
                          device: torch.device) -> Int4KVLayerCache:
    """Uninitialized cache tensors of the given capacity (ia.py:423-436)."""
    packed_shape = (batch, kv_heads, capacity, head_dim // 2)
    scale_shape = (batch, kv_heads, capacity, groups)
    return Int4KVLayerCache(
        k_packed=torch.empty(packed_shape, device=device, dtype=torch.uint8),
        v_packed=torch.empty(packed_shape, device=device, dtype=torch.uint8),
        k_scale=torch.empty(scale_shape, device=device, dtype=torch.float32),
        v_scale=torch.empty(scale_shape, device=device, dtype=torch.float32),
    )


def _ensure_layer_cache(past_key_value, layer_idx: int, batch: int, kv_heads: int,
                        required_len: int, head_dim: int, group_size: int,
                        device: torch.device) -> Int4KVLayerCache:
    """Return a layer cache with at least `required_len` rows (ia.py:439-474).

    A new cache gets capacity max(16, next power of two); a full one grows to the next power of
    two of required_len and keeps its rows and length. A cache created for another (batch,
    kv_heads) raises ValueError.
    """
    groups = head_dim // group_size
    caches = _cache_dict(past_key_value)
    current = caches.get(layer_idx)
    if current is None:
        capacity = max(16, 1 << math.ceil(math.log2(max(required_len, 1))))
        current = _allocate_layer_cache(batch, kv_heads, capacity, head_dim, groups, device)
        caches[layer_idx] = current
        return current
    if tuple(current.k_packed.shape[:2]) != (batch, kv_heads):
        raise ValueError(
            f"Layer {layer_idx} INT4 cache shape {tuple(current.k_packed.shape[:2])} "
            f"does not match batch/kv_heads {(batch, kv_heads)}")
    old_cap = current.k_packed.shape[2]
    if required_len <= old_cap:
        return current
    grown = _allocate_layer_cache(batch, kv_heads, 1 << math.ceil(math.log2(required_len)),
                                  head_dim, groups, device)
    for name in ("k_packed", "v_packed", "k_scale", "v_scale"):
        getattr(grown, name)[:, :, :old_cap].copy_(getattr(current, name))
    grown.length = current.length
    caches[layer_idx] = grown
    return grown


def _pack_kv_into_cache(cache: Int4KVLayerCache, key_states: torch.Tensor,
                        value_states: torch.Tensor, positions: torch.Tensor,
                        group_size: int) -> None:
    """INT4-pack K and V [B, Hkv, q_len, D] into rows `positions` (ia.py:477-515); one launch
    for both (the reference launches _pack_int4_kv_kernel once for K and once for V)."""
    _abi.int4_pack_kv_pair(key_states, value_states, cache.k_packed, cache.v_packed,
                           cache.k_scale, cache.v_scale, positions, group_size)
    cache.length = max(cache.length, int(positions.max().item()) + 1)


def _decode_attention_mask(attention_mask: torch.Tensor | None, batch: int, seq_len: int,
                           device: torch.device) -> torch.Tensor | None:
    """Additive fp32 key bias [B, 1, 1, S] for the decode kernel (ia.py:569-591).

    A 4-D mask contributes its last query row over the first seq_len keys (bool -> 0 / -inf,
    else cast to fp32); a 2-D keep-mask contributes its last seq_len columns.
    """
    if attention_mask is None:
        return None
    if attention_mask.dim() == 4:
        rows = attention_mask[:, :, -1:, :seq_len].to(device=device)
        if rows.dtype != torch.bool:
            return rows.to(dtype=torch.float32).contiguous()
        bias = torch.zeros(rows.shape, device=device, dtype=torch.float32)
        return bias.masked_fill(rows.logical_not(), -float("inf")).contiguous()
    if attention_mask.dim() == 2:
        cols = attention_mask[:, -seq_len:].to(device=device)
        keep = cols if cols.dtype == torch.bool else cols != 0
        bias = torch.zeros((batch, 1, 1, seq_len), device=device, dtype=torch.float32)
        return bias.masked_fill(keep.logical_not()[:, None, None, :], -float("inf"))
    raise ValueError(
        f"INT4 decode attention only supports 2D or 4D attention_mask, got {attention_mask.dim()}D")


def _decode_attention(query_states: torch.Tensor, cache: Int4KVLayerCache, seq_len: int,
                      num_key_value_groups: int, group_size: int,
                      attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of q [B, Hq, 1, D] over cache rows [0, seq_len) -> [B, Hq, D] in q's dtype
    (ia.py:518-566)."""
    batch, n_heads, q_len, head_dim = query_states.shape
    if q_len != 1:
        raise ValueError(f"Fused INT4 decode attention expects q_len=1, got {q_len}")
    out = torch.empty((batch, n_heads, head_dim), device=query_states.device,
                      dtype=query_states.dtype)
    mask = _decode_attention_mask(attention_mask, batch, seq_len, query_states.device)
    _abi.int4_decode_attention(query_states, cache.k_packed, cache.v_packed, cache.k_scale,
                               cache.v_scale, mask, out, seq_len, num_key_value_groups,
                               group_size)
    return out


def _pack_and_decode_attention(query_states: torch.Tensor, key_states: torch.Tensor,
                               value_states: torch.Tensor, cache: Int4KVLayerCache,
                               seq_len: int, num_key_value_groups: int, group_size: int,
                               attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """_pack_kv_into_cache of the step's one token into row seq_len - 1, then _decode_attention
    over rows [0, seq_len): the reference's decode branch (ia.py:678-690) as one library call,
    which on the MFMA path is one kernel launch. Same cache bytes, length and output."""
    batch, n_heads, q_len, head_dim = query_states.shape
    if q_len != 1 or key_states.shape[2] != 1:
        raise ValueError(f"Fused INT4 decode attention expects q_len=1, got {q_len}")
    out = torch.empty((batch, n_heads, head_dim), device=query_states.device,
                      dtype=query_states.dtype)
    try:
        mask = _decode_attention_mask(attention_mask, batch, seq_len, query_states.device)
    except ValueError:
        # the reference packs the token and moves cache.length before its mask check raises
        # (ia.py:678 packs, :532 raises): leave the cache in that state on this error path too
        _pack_kv_into_cache(cache, key_states, value_states,
                            torch.tensor([seq_len - 1], device=key_states.device), group_size)
        raise
    _abi.int4_decode_attention_pack(query_states, key_states, value_states, cache.k_packed,
                                    cache.v_packed, cache.k_scale, cache.v_scale, mask, out,
                                    seq_len, num_key_value_groups, group_size)
    cache.length = max(cache.length, seq_len)
    return out


def _prefill_attention(query_states: torch.Tensor, cache: Int4KVLayerCache,
                       num_key_value_groups: int, group_size: int) -> torch.Tensor:
    """Causal attention of q [B, Hq, L, D] over cache rows [0, L): position t attends to rows
    0 .. t -> [B, Hq, L, D] in q's dtype (ia.py:594-625)."""
    batch, n_heads, q_len, head_dim = query_states.shape
    out = torch.empty((batch, n_heads, q_len, head_dim), device=query_states.device,
                      dtype=query_states.dtype)
    _abi.int4_prefill_attention(query_states, cache.k_packed, cache.v_packed, cache.k_scale,
                                cache.v_scale, out, num_key_value_groups, group_size)
    return out


def _forward_fused_int4_kv(self, hidden_states, attention_mask=None, position_ids=None,
                           past_key_value=None, output_attentions=False, use_cache=False,
                           cache_position=None):
    """Patched attention forward (ia.py:628-714): pack this step's K/V into the INT4 cache;
    decode (q_len == 1) attends over the cache, prefill runs SDPA on the unquantized K/V."""
    if output_attentions or hidden_states.device.type != "cuda" or past_key_value is None:
        return self._int4_kv_original_forward(
            hidden_states=hidden_states, attention_mask=attention_mask,
            position_ids=position_ids, past_key_value=past_key_value,
            output_attentions=output_attentions, use_cache=use_cache,
            cache_position=cache_position)

    bsz, q_len, _ = hidden_states.size()

    def heads(proj, n):
        return proj(hidden_states).view(bsz, q_len, n, self.head_dim).transpose(1, 2).contiguous()

    query_states = heads(self.q_proj, self.num_heads)
    key_states = heads(self.k_proj, self.num_key_value_heads)
    value_states = heads(self.v_proj, self.num_key_value_heads)

    group_size = self._int4_kv_group_size
    if self.head_dim % group_size != 0:
        raise ValueError(f"head_dim={self.head_dim} must be divisible by group_size={group_size}")
    if group_size % 2 != 0:
        raise ValueError(f"group_size={group_size} must be even for INT4 packing")

    positions = _positions(cache_position, q_len, hidden_states.device)
    required_len = int(positions.max().item()) + 1
    layer_cache = _ensure_layer_cache(past_key_value, self.layer_idx, bsz,
                                      self.num_key_value_heads, required_len, self.head_dim,
                                      group_size, hidden_states.device)
    if q_len == 1:
        # the token's row is required_len - 1 (positions holds that one value)
        attn = _pack_and_decode_attention(query_states, key_states, value_states, layer_cache,
                                          required_len, self.num_key_value_groups, group_size,
                                          attention_mask=attention_mask)
        attn = attn.reshape(bsz, q_len, self.hidden_size)
        return self.o_proj(attn), None, past_key_value

    _pack_kv_into_cache(layer_cache, key_states, value_states, positions, group_size)

    key_full = self._int4_kv_repeat_kv(key_states, self.num_key_value_groups)
    value_full = self._int4_kv_repeat_kv(value_states, self.num_key_value_groups)
    causal_mask = None
    if attention_mask is not None:
        causal_mask = attention_mask[:, :, :, : key_full.shape[-2]]
        query_states = query_states.contiguous()
        key_full = key_full.contiguous()
        value_full = value_full.contiguous()
    attn = torch.nn.functional.scaled_dot_product_attention(
        query_states, key_full, value_full, attn_mask=causal_mask,
        dropout_p=self.attention_dropout if self.training else 0.0,
        is_causal=causal_mask is None and q_len > 1)
    attn = attn.transpose(1, 2).contiguous().view(bsz, q_len, self.hidden_size)
    return self.o_proj(attn), None, past_key_value


def patch_nemotron_h_attention_int4_kv(model, group_size: int = 64):
    """Route every attention block's forward through the INT4 cache (ia.py:717-731).

    Idempotent per layer; records the original forward, the group size and the remote module's
    repeat_kv on each patched mixer.
    """
    remote = __import__(model.__class__.__module__, fromlist=["repeat_kv"])
    repeat_kv = remote.repeat_kv
    for layer in model.backbone.layers:
        if getattr(layer, "block_type", None) != "attention":
            continue
        attn = getattr(layer, "mixer", None)
        if attn is None or getattr(attn, "_int4_kv_patched", False):
            continue
        attn._int4_kv_original_forward = attn.forward
        attn._int4_kv_group_size = group_size
        attn._int4_kv_repeat_kv = repeat_kv
        attn.forward = MethodType(_forward_fused_int4_kv, attn)
        attn._int4_kv_patched = True
