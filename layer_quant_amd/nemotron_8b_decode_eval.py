"""Decode-evaluation glue for Nemotron-H (reference hybrid_quant/nemotron_8b_decode_eval.py).

Re-provided so that the reference's driver imports resolve against this package; it holds no
kernel. Cited as de.py:line below.
"""
from __future__ import annotations

import contextlib
from types import MethodType

import torch


def _block_forward_with_cache(self, hidden_states, cache_params=None, cache_position=None,
                              attention_mask=None):
    """Residual block that hands the hybrid cache to attention mixers too (de.py:8-50).

    Runs on the device's default stream, like the reference (CPU tensors run as they are).
    """
    stream_ctx = (torch.cuda.stream(torch.cuda.default_stream(hidden_states.device))
                  if hidden_states.is_cuda else contextlib.nullcontext())
    with stream_ctx:
        residual = hidden_states
        hidden_states = self.norm(hidden_states.to(dtype=self.norm.weight.dtype))
        if self.residual_in_fp32:
            residual = residual.to(torch.float32)
        kind = self.block_type
        if kind == "mamba":
            hidden_states = self.mixer(hidden_states, cache_params=cache_params,
                                       cache_position=cache_position,
                                       attention_mask=attention_mask)
        elif kind == "attention":
            hidden_states = self.mixer(hidden_states, attention_mask=attention_mask,
                                       past_key_value=cache_params,
                                       use_cache=cache_params is not None,
                                       cache_position=cache_position)[0]
        elif kind == "mlp":
            hidden_states = self.mixer(hidden_states)
        else:
            raise ValueError(f"Invalid block_type: {kind}")
        return residual + hidden_states


def patch_attention_cache_in_blocks(model) -> None:
    """Patch every block once so attention layers receive the cache (de.py:8-50)."""
    for block in model.backbone.layers:
        if getattr(block, "_decode_eval_block_patched", False):
            continue
        block.forward = MethodType(_block_forward_with_cache, block)
        block._decode_eval_block_patched = True


class DeviceList(list):
    """A list that also carries a `.device` attribute (de.py:53-56)."""

    def __init__(self, values, device):
        super().__init__(values)
        self.device = device


def make_hybrid_cache(model, batch_size: int):
    """bf16 HybridMambaAttentionDynamicCache of the remote module (de.py:59-66)."""
    remote = __import__(model.__class__.__module__, fromlist=["HybridMambaAttentionDynamicCache"])
    cache = remote.HybridMambaAttentionDynamicCache(model.config, batch_size, torch.bfloat16,
                                                    device=model.device)
    cache.conv_kernel_size = model.config.conv_kernel
    cache.conv_states = DeviceList(cache.conv_states, model.device)
    cache.ssm_states = DeviceList(cache.ssm_states, model.device)
    return cache


def layer_groups(config) -> tuple[list[int], list[int], list[int]]:
    """Indices of Mamba ('M'), attention ('*') and MLP ('-') layers (de.py:69-74)."""
    pattern = config.hybrid_override_pattern
    by_kind = {"M": [], "*": [], "-": []}
    for idx, kind in enumerate(pattern):
        if kind in by_kind:
            by_kind[kind].append(idx)
    return by_kind["M"], by_kind["*"], by_kind["-"]


def adjacent_mamba_layers(mamba_layers: list[int], attention_layers: list[int]) -> set[int]:
    """The nearest Mamba layer before and after each attention layer (de.py:77-86)."""
    adjacent: set[int] = set()
    ordered = sorted(mamba_layers)
    for attn in attention_layers:
        before = [idx for idx in ordered if idx < attn]
        after = [idx for idx in ordered if idx > attn]
        if before:
            adjacent.add(before[-1])
        if after:
            adjacent.add(after[0])
    return adjacent
