"""CPU restatement of the reference's INT4 KV-cache path -- TEST INFRASTRUCTURE ONLY.

Reference: hybrid_quant/int4_8b_attention.py (cited as ia.py:line below).

Pinning (tests/test_oracle_int4.py):
  quantize_groups     brute force on exactly representable groups (x = k*s recovers k), the
                      invariants |q| <= 7 and |x - q*s| <= s/2, all-zero groups (scale 1e-8),
                      exact ties (round half to even), and an independent float64 recomputation
  pack_nibbles        bit layout checked against a per-element loop; unpack(pack(q)) == q for
                      all 16 nibble values
  pack_kv_into_cache  rows land at `positions`, other rows untouched, length bookkeeping
  decode_attention    torch scaled_dot_product_attention on the dequantized cache (library
                      routine); seq_len=1 -> V row 0; q=0 -> mean of V; masked keys excluded;
                      GQA head mapping kvh = qh // n_rep
  decode_attention_mask  each branch of ia.py:569-591 against hand-built masks
  prefill_attention   torch scaled_dot_product_attention(is_causal=True) on the dequantized cache
                      (library routine); row t equals decode_attention over t + 1 keys (the causal
                      length q_pos + 1 of ia.py:170); a per-element loop on tiny inputs; q_len=1 ->
                      V row 0; q=0 -> running mean of V
"""
from __future__ import annotations

import math

import numpy as np
import torch

INT4_MIN = -8
INT4_MAX = 7
SCALE_FLOOR = 1.0e-8  # ia.py:27 and ia.py:76


def quantize_groups(x: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Signed INT4 group quantization along the last dim.

    Follows the pack kernel ia.py:75-85 (absmax -> scale = max(absmax / 7, 1e-8) ->
    round-half-even(x / scale) -> clamp [-8, 7]), which equals the closed form
    int4_quant_dequant at ia.py:26-28. All arithmetic is fp32, as in the kernel.
    Returns (q int8 [..., D], scale f32 [..., D/g]).
    """
    d = x.shape[-1]
    if d % group_size != 0:
        raise ValueError(f"head_dim={d} must be divisible by group_size={group_size}")
    xf = x.float().reshape(*x.shape[:-1], d // group_size, group_size)
    amax = xf.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp(amax / 7.0, min=SCALE_FLOOR)
    q = torch.clamp(torch.round(xf / scale), INT4_MIN, INT4_MAX)
    return q.reshape(x.shape).to(torch.int8), scale.squeeze(-1)


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """Two's-complement nibbles, two per byte: even d -> low nibble, odd d -> high (ia.py:86-97)."""
    qi = q.to(torch.int32) & 15
    low = qi[..., 0::2]
    high = qi[..., 1::2]
    return ((high << 4) | low).to(torch.uint8)


def unpack_nibbles(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_nibbles; a nibble n >= 8 means n - 16 (ia.py:336-337)."""
    b = packed.to(torch.int32)
    low = b & 15
    high = (b >> 4) & 15
    out = torch.stack([low, high], dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    return torch.where(out >= 8, out - 16, out).to(torch.int8)


def dequantize(packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """k = signed_nibble * group_scale in fp32 (ia.py:337-347)."""
    q = unpack_nibbles(packed).float()
    s = scale.float().repeat_interleave(group_size, dim=-1)
    return q * s


def allocate_cache(batch: int, kv_heads: int, capacity: int, head_dim: int, group_size: int):
    """Zero-filled CPU cache with the layout of _allocate_layer_cache (ia.py:423-436)."""
    groups = head_dim // group_size
    return {
        "k_packed": torch.zeros((batch, kv_heads, capacity, head_dim // 2), dtype=torch.uint8),
        "v_packed": torch.zeros((batch, kv_heads, capacity, head_dim // 2), dtype=torch.uint8),
        "k_scale": torch.zeros((batch, kv_heads, capacity, groups), dtype=torch.float32),
        "v_scale": torch.zeros((batch, kv_heads, capacity, groups), dtype=torch.float32),
        "length": 0,
    }


def pack_into(packed: torch.Tensor, scale: torch.Tensor, x: torch.Tensor,
              positions: torch.Tensor, group_size: int) -> None:
    """One launch of _pack_int4_kv_kernel (ia.py:56-111): token t of x lands in row positions[t]."""
    q, s = quantize_groups(x, group_size)
    bytes_ = pack_nibbles(q)
    for t, pos in enumerate(positions.tolist()):
        packed[:, :, pos] = bytes_[:, :, t]
        scale[:, :, pos] = s[:, :, t]


def pack_kv_into_cache(cache: dict, key_states: torch.Tensor, value_states: torch.Tensor,
                       positions: torch.Tensor, group_size: int) -> None:
    """_pack_kv_into_cache (ia.py:477-515): pack K and V, then length = max(length, max(pos)+1)."""
    pack_into(cache["k_packed"], cache["k_scale"], key_states, positions, group_size)
    pack_into(cache["v_packed"], cache["v_scale"], value_states, positions, group_size)
    cache["length"] = max(cache["length"], int(positions.max().item()) + 1)


def decode_attention(q: torch.Tensor, k_packed: torch.Tensor, v_packed: torch.Tensor,
                     k_scale: torch.Tensor, v_scale: torch.Tensor, seq_len: int,
                     num_key_value_groups: int, group_size: int,
                     mask: torch.Tensor | None = None) -> torch.Tensor:
    """q_len=1 attention over the packed cache, in float64 (ia.py:301-402).

    q: [B, Hq, D] or [B, Hq, 1, D]. Query head h reads KV head h // num_key_value_groups
    (ia.py:304). Scores s_n = (q . k_n) * log2(e)/sqrt(D) (+ mask_n), softmax in the exp2 domain
    (ia.py:310, 350-362), out = sum p_n v_n / sum p_n. Keys at or beyond the mask length get
    -inf (ia.py:352-357). A query whose keys are all masked returns NaN (0/0).
    Returns float64 [B, Hq, D].
    """
    if q.dim() == 4:
        q = q[:, :, 0]
    bsz, hq, d = q.shape
    k = dequantize(k_packed[:, :, :seq_len], k_scale[:, :, :seq_len], group_size).double()
    v = dequantize(v_packed[:, :, :seq_len], v_scale[:, :, :seq_len], group_size).double()
    kv_index = torch.arange(hq) // num_key_value_groups
    k = k[:, kv_index]  # [B, Hq, S, D]
    v = v[:, kv_index]
    scale_sm = 1.4426950408889634 / math.sqrt(d)
    s = torch.einsum("bhd,bhsd->bhs", q.double(), k) * scale_sm
    if mask is not None:
        bias = torch.full((bsz, seq_len), -math.inf, dtype=torch.float64)
        lm = min(mask.shape[-1], seq_len)
        bias[:, :lm] = mask.reshape(bsz, -1)[:, :lm].double()
        s = s + bias[:, None, :]
    m = s.amax(dim=-1, keepdim=True)
    p = torch.exp2(s - m)
    return torch.einsum("bhs,bhsd->bhd", p, v) / p.sum(dim=-1, keepdim=True)


def prefill_attention(q: torch.Tensor, k_packed: torch.Tensor, v_packed: torch.Tensor,
                      k_scale: torch.Tensor, v_scale: torch.Tensor, num_key_value_groups: int,
                      group_size: int) -> torch.Tensor:
    """Causal multi-token attention over the packed cache, in float64 (ia.py:114-251, launched by
    _prefill_attention at ia.py:594-625).

    q: [B, Hq, L, D]. Query position t of head h attends to cache keys 0 .. t of KV head
    h // num_key_value_groups (causal_len = q_pos + 1, ia.py:166-170; the cache holds the prompt
    from position 0). Scores (q . k_n) * log2(e)/sqrt(D), exp2-domain softmax (ia.py:162,
    209-213), out = sum p_n v_n / sum p_n (ia.py:243). Returns float64 [B, Hq, L, D].
    """
    bsz, hq, q_len, d = q.shape
    k = dequantize(k_packed[:, :, :q_len], k_scale[:, :, :q_len], group_size).double()
    v = dequantize(v_packed[:, :, :q_len], v_scale[:, :, :q_len], group_size).double()
    kv_index = torch.arange(hq) // num_key_value_groups
    k = k[:, kv_index]  # [B, Hq, L, D]
    v = v[:, kv_index]
    scale_sm = 1.4426950408889634 / math.sqrt(d)
    s = torch.matmul(q.double(), k.transpose(-1, -2).contiguous()) * scale_sm  # [B, Hq, L, L]
    future = torch.ones(q_len, q_len, dtype=torch.bool).triu(1)
    s = s.masked_fill(future, -math.inf)
    m = s.amax(dim=-1, keepdim=True)
    p = torch.exp2(s - m)
    return torch.matmul(p, v) / p.sum(dim=-1, keepdim=True)


def prefill_flops(batch: int, n_q_heads: int, q_len: int, head_dim: int) -> int:
    """Algorithmic flops of one causal prefill call: 2*D for q.k and 2*D for p*v per visible
    (query, key) pair, L (L + 1) / 2 pairs per head."""
    return 4 * head_dim * batch * n_q_heads * (q_len * (q_len + 1) // 2)


def decode_attention_mask(attention_mask: torch.Tensor | None, batch: int,
                          seq_len: int) -> torch.Tensor | None:
    """_decode_attention_mask (ia.py:569-591): keep-mask or 4-D mask -> fp32 bias [B,1,1,S]."""
    if attention_mask is None:
        return None
    if attention_mask.dim() == 4:
        mask = attention_mask[:, :, -1:, :seq_len]
        if mask.dtype == torch.bool:
            bias = torch.zeros(mask.shape, dtype=torch.float32)
            return bias.masked_fill(~mask, -float("inf")).contiguous()
        return mask.to(dtype=torch.float32).contiguous()
    if attention_mask.dim() == 2:
        mask = attention_mask[:, -seq_len:]
        keep = mask if mask.dtype == torch.bool else mask != 0
        bias = torch.zeros((batch, 1, 1, seq_len), dtype=torch.float32)
        return bias.masked_fill(~keep[:, None, None, :], -float("inf"))
    raise ValueError(
        f"INT4 decode attention only supports 2D or 4D attention_mask, got {attention_mask.dim()}D")


def algorithmic_bytes(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int, seq_len: int,
                      group_size: int, q_bytes: int = 2, out_bytes: int = 2,
                      mask: bool = False) -> int:
    """Unique bytes one decode-attention call must move: K and V nibbles, fp32 scales, q, out."""
    kv = 2 * batch * n_kv_heads * seq_len * (head_dim // 2)
    scales = 2 * batch * n_kv_heads * seq_len * (head_dim // group_size) * 4
    qo = batch * n_q_heads * head_dim * (q_bytes + out_bytes)
    return kv + scales + qo + (batch * seq_len * 4 if mask else 0)


def pack_algorithmic_bytes(batch: int, n_kv_heads: int, n_tokens: int, head_dim: int,
                           group_size: int, x_bytes: int = 2) -> int:
    """Unique bytes of one pack call (K or V): read x, write packed bytes and scales."""
    return batch * n_kv_heads * n_tokens * (head_dim * x_bytes + head_dim // 2
                                            + 4 * (head_dim // group_size))


def numpy_pack_reference(x: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Same quantization in float32 numpy (np.rint = round half to even); an independent path."""
    d = x.shape[-1]
    xf = x.astype(np.float32).reshape(*x.shape[:-1], d // group_size, group_size)
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    scale = np.maximum(amax / np.float32(7.0), np.float32(SCALE_FLOOR)).astype(np.float32)
    q = np.clip(np.rint(xf / scale), INT4_MIN, INT4_MAX).astype(np.int32).reshape(x.shape)
    nib = q & 15
    packed = (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)
    return packed, scale[..., 0]
