"""MX8 / MX4 block-quantized Mamba2 recurrent state with a fused decode update.

API-compatible with the reference module hybrid_quant/mamba_state_8b_kernel.py (cited as
ms.py:line): same public names, argument meaning and error messages. The Triton kernels and the
torch initial encoder are replaced by HIP kernels for gfx950 behind the C ABI
(include/layer_quant.h):

    _state_update_requant_mx8_row_kernel          -> lq_mx_state_update, format_bits 8 (ms.py:33-222)
    _state_update_mx8_kernel + _requantize_mx4_kernel -> lq_mx_state_update, format_bits 4
                                                     (ms.py:225-443, 494-544), one pass
    _quantize_initial_state_mx (torch)            -> lq_mx_encode, nearest-even (ms.py:547-572)
    mamba-ssm selective_state_update (the fallback -> lq_selective_state_update (bf16/fp16/fp32
    for unregistered layers, ms.py:738-747)           state), `selective_state_update` here

Stochastic rounding. The reference draws Triton's tl.rand per element at offset
step*B*H*P*N + element index. This module keeps those offsets and, by default, draws from the
library's counter-based generator (LQ_ROUND_SR_COUNTER, 16-bit uniforms from a hash of
(seed, offset)). `rng="philox"` draws the reference's own stream instead (LQ_ROUND_SR_PHILOX:
tl.rand's Philox4x32-10 and the reference's u < frac test, bit for bit, at about 2.7x the counter
mode's time). Passing `uniform=` (an fp32 tensor shaped like the state) rounds with those
uniforms, for bit-exact comparison with any other implementation given the same tensor.
`stochastic=False` selects the reference's deterministic floor(q + 0.5) writeback.
"""
from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace

import torch

from . import _abi

MX8_BLOCK_SIZE = 16
MX8_PAIR_SIZE = 2
MX8_MANTISSA_MAX = 63.0
MX4_BLOCK_SIZE = 16
MX4_PAIR_SIZE = 2
MX4_MANTISSA_MAX = 7.0

_MANTISSA_MAX = {8: MX8_MANTISSA_MAX, 4: MX4_MANTISSA_MAX}


@dataclass
class MambaStateKernelCache:
    """MX state of one layer (ms.py:19-25): q_state int8 [B,H,P,N] (one byte per mantissa in
    both formats), shared_exp uint8 [B,H,P,N/16], micro_exp uint8 [B,H,P,N/2], the format, and
    the host-side step counter that offsets the stochastic-rounding stream."""

    q_state: torch.Tensor
    shared_exp: torch.Tensor
    micro_exp: torch.Tensor
    format_bits: int = 8
    step: int = 0
    layout: str = "reference"
    # optional step counter on the device (int64 [1], see enable_device_step): the counter and
    # Philox roundings then read it in the kernel and advance it with a tensor add, so a decode
    # step captured in a graph draws anew on every replay
    device_step: torch.Tensor | None = None

    @property
    def state_shape(self) -> tuple[int, ...]:
        """[B, H, P, N] of the state this cache holds (N = 16 * the exponent dimension)."""
        return (*self.shared_exp.shape[:-1], self.shared_exp.shape[-1] * MX8_BLOCK_SIZE)


# State layouts. "reference": q_state int8 [..., N] (one byte per mantissa, both formats),
# micro_exp uint8 [..., N/2] (one byte per pair) -- the reference's, interchangeable with it.
# "compact" (no reference counterpart): micro_exp uint8 [..., N/16] with bit k of byte j the
# micro-exponent of pair 8j + k; MX4 q_state uint8 [..., N/2] with two two's-complement nibbles
# per byte (value 2p low, 2p + 1 high); MX8 q_state as in the reference. shared_exp is the same.
# Same arithmetic and bit-identical states in either layout; compact MX4 moves 80 bytes per
# 128-value row instead of 200.
STATE_LAYOUTS = ("reference", "compact")


def _empty_mx_tensors(shape, device, format_bits: int = 8, layout: str = "reference"):
    *lead, n = shape
    if layout not in STATE_LAYOUTS:
        raise ValueError(f"Unknown MX state layout {layout!r}; expected one of {STATE_LAYOUTS}")
    if layout == "compact":
        if format_bits == 4:
            q = torch.empty((*lead, n // 2), dtype=torch.uint8, device=device)
        else:
            q = torch.empty(shape, dtype=torch.int8, device=device)
        m = torch.empty((*lead, n // MX8_BLOCK_SIZE), dtype=torch.uint8, device=device)
    else:
        q = torch.empty(shape, dtype=torch.int8, device=device)
        m = torch.empty((*lead, n // MX8_PAIR_SIZE), dtype=torch.uint8, device=device)
    return q, torch.empty((*lead, n // MX8_BLOCK_SIZE), dtype=torch.uint8, device=device), m


def _quantize_initial_state_mx(state: torch.Tensor, *, format_bits: int, block_size: int,
                               pair_size: int, mantissa_max: float, layout: str = "reference"):
    """Nearest-even MX encode of a float state [..., N] (ms.py:547-572).

    Runs lq_mx_encode on the state's GPU. The block and pair sizes and the mantissa maximum are
    fixed by the format (16, 2 and 63 or 7); other values raise ValueError.
    """
    if state.shape[-1] % block_size != 0:
        raise ValueError(
            f"MX{format_bits} state dim must be divisible by {block_size}, got {state.shape[-1]}")
    if (block_size, pair_size) != (MX8_BLOCK_SIZE, MX8_PAIR_SIZE) or \
            _MANTISSA_MAX.get(format_bits) != float(mantissa_max):
        raise ValueError(
            f"MX{format_bits} kernels use 16-value blocks, pairs and mantissa max "
            f"{_MANTISSA_MAX.get(format_bits)}; got block_size={block_size}, "
            f"pair_size={pair_size}, mantissa_max={mantissa_max}")
    lead = state.shape[:-1]
    state4 = state.reshape(-1, 1, 1, state.shape[-1]) if state.dim() != 4 else state
    q, e, m = _empty_mx_tensors(tuple(state4.shape), state.device, format_bits, layout)
    _abi.mx_encode(state4, q, e, m, format_bits, _abi.ROUND_NEAREST_EVEN)
    return (q.reshape(*lead, q.shape[-1]), e.reshape(*lead, e.shape[-1]),
            m.reshape(*lead, m.shape[-1]))


def allocate_state_kernel_cache(ssm_state_4d: torch.Tensor, group_size: int = MX8_BLOCK_SIZE,
                                format_bits: int = 8, *,
                                layout: str = "reference") -> MambaStateKernelCache:
    """Encode a layer's state [B,H,P,N] into a new MX cache (ms.py:575-598); `layout` selects the
    reference's tensors (default) or the compact ones (see STATE_LAYOUTS)."""
    if format_bits == 8:
        if group_size != MX8_BLOCK_SIZE:
            raise ValueError(
                f"MX8 uses a fixed {MX8_BLOCK_SIZE}-value block, got group_size={group_size}")
        q, e, m = _quantize_initial_state_mx(ssm_state_4d, format_bits=8,
                                             block_size=MX8_BLOCK_SIZE, pair_size=MX8_PAIR_SIZE,
                                             mantissa_max=MX8_MANTISSA_MAX, layout=layout)
        return MambaStateKernelCache(q_state=q, shared_exp=e, micro_exp=m, format_bits=8,
                                     layout=layout)
    if format_bits == 4:
        if group_size != MX4_BLOCK_SIZE:
            raise ValueError(
                f"MX4 uses a fixed {MX4_BLOCK_SIZE}-value block, got group_size={group_size}")
        q, e, m = _quantize_initial_state_mx(ssm_state_4d, format_bits=4,
                                             block_size=MX4_BLOCK_SIZE, pair_size=MX4_PAIR_SIZE,
                                             mantissa_max=MX4_MANTISSA_MAX, layout=layout)
        return MambaStateKernelCache(q_state=q, shared_exp=e, micro_exp=m, format_bits=4,
                                     layout=layout)
    raise ValueError(
        f"Only MX8 and MX4 state quantization are supported, got format_bits={format_bits}")


def dequantize_state_cache(cache: MambaStateKernelCache,
                           dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decoded state q * 2^(e - 127 + micro) [B,H,P,N] (no reference counterpart; the
    reference decodes only inside its update kernels, ms.py:132, 322)."""
    out = torch.empty(cache.state_shape, dtype=dtype, device=cache.q_state.device)
    return _abi.mx_decode(cache.q_state, cache.shared_exp, cache.micro_exp, out)


def convert_state_cache_layout(cache: MambaStateKernelCache, layout: str) -> MambaStateKernelCache:
    """The same MX state in the other layout (bit-exact, lossless; the step counter is kept).
    No reference counterpart: the compact layout is this build's."""
    if layout not in STATE_LAYOUTS:
        raise ValueError(f"Unknown MX state layout {layout!r}; expected one of {STATE_LAYOUTS}")
    if layout == cache.layout:
        return cache
    q, e, m = cache.q_state, cache.shared_exp, cache.micro_exp
    *lead, n = cache.state_shape
    shifts = torch.arange(8, device=m.device, dtype=torch.int32)
    if layout == "compact":
        if cache.format_bits == 4:
            u = q.view(torch.uint8).to(torch.int32) & 0x0F
            q2 = (u[..., 0::2] | (u[..., 1::2] << 4)).to(torch.uint8)
        else:
            q2 = q.clone()
        bits = m.reshape(*lead, n // MX8_BLOCK_SIZE, 8).to(torch.int32) & 1
        m2 = (bits << shifts).sum(dim=-1).to(torch.uint8)
    else:
        if cache.format_bits == 4:
            u = q.to(torch.int32)
            lo, hi = u & 0x0F, (u >> 4) & 0x0F
            q2 = torch.stack((lo, hi), dim=-1).reshape(*lead, n)
            q2 = torch.where(q2 > 7, q2 - 16, q2).to(torch.int8)
        else:
            q2 = q.clone()
        m2 = ((m.to(torch.int32)[..., None] >> shifts) & 1).reshape(*lead, n // 2).to(torch.uint8)
    return MambaStateKernelCache(q_state=q2.contiguous(), shared_exp=e.clone(),
                                 micro_exp=m2.contiguous(), format_bits=cache.format_bits,
                                 step=cache.step, layout=layout)


def _dt_bias_as_read(dt_bias: torch.Tensor | None, D: torch.Tensor | None, nheads: int,
                     dim: int) -> torch.Tensor | None:
    """The dt_bias values the reference kernels read: they index dt_bias with D's strides,
    or with strides (0, 0) when D is None (ms.py:137, 335, 624)."""
    if dt_bias is None:
        return None
    strides = tuple(D.stride()) if D is not None else (0, 0)
    if tuple(dt_bias.shape) == (nheads, dim) and tuple(dt_bias.stride()) == strides:
        return dt_bias
    reach = dt_bias.storage_offset() + (nheads - 1) * max(strides[0], 0) + (dim - 1) * max(
        strides[1], 0)
    if reach >= dt_bias.untyped_storage().nbytes() // dt_bias.element_size():
        raise ValueError(
            "dt_bias read with D's strides would leave dt_bias's storage; pass dt_bias and D "
            "with the same layout")
    return dt_bias.as_strided((nheads, dim), strides)


def mx_state_selective_update(cache: MambaStateKernelCache, x: torch.Tensor, dt: torch.Tensor,
                              A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                              D: torch.Tensor | None = None, z: torch.Tensor | None = None,
                              dt_bias: torch.Tensor | None = None, dt_softplus: bool = False,
                              stochastic: bool = True, seed: int = 1234, *,
                              uniform: torch.Tensor | None = None,
                              rng: str = "counter") -> torch.Tensor:
    """One fused decode step on the MX state, in place; returns y [B,H,P] in x's dtype
    (ms.py:601-721).

    h = dequant(state); dt (+ dt_bias, read with D's strides); softplus if dt_softplus;
    h' = h*exp(A*dt) + B*dt*x; y = sum_n h'*C (+ x*D) (* z); the state is re-encoded in its
    format with stochastic rounding (the counter generator, rng="philox" for the reference's
    tl.rand stream, or `uniform`) or, with stochastic=False, floor(q + 0.5). cache.step
    advances by one.
    """
    if rng not in ("counter", "philox"):
        raise ValueError(f"rng must be 'counter' or 'philox', got {rng!r}")
    if cache.q_state.ndim != 4:
        raise ValueError(f"Expected q_state [B,H,P,N], got {tuple(cache.q_state.shape)}")
    batch, nheads, dim, dstate = cache.state_shape
    if x.shape != (batch, nheads, dim):
        raise ValueError(f"Expected x shape {(batch, nheads, dim)}, got {tuple(x.shape)}")
    if B.ndim != 3 or C.ndim != 3:
        raise ValueError("Expected B and C with shape [batch, ngroups, dstate] for decode update.")
    if cache.format_bits not in (8, 4):
        raise ValueError(f"Unsupported MX state format_bits={cache.format_bits}")
    out = torch.empty_like(x)
    if not stochastic:
        mode = _abi.ROUND_HALF_UP
    elif uniform is not None:
        mode = _abi.ROUND_SR_UNIFORM
    elif rng == "philox":
        mode = _abi.ROUND_SR_PHILOX
    else:
        mode = _abi.ROUND_SR_COUNTER
    on_device = cache.device_step is not None and mode in (_abi.ROUND_SR_COUNTER,
                                                           _abi.ROUND_SR_PHILOX)
    rng_offset = 0 if on_device else cache.step * batch * nheads * dim * dstate
    _abi.mx_state_update(cache.q_state, cache.shared_exp, cache.micro_exp, x, dt,
                         _dt_bias_as_read(dt_bias, D, nheads, dim), A, B, C, D, z, out,
                         cache.format_bits, dt_softplus, mode,
                         uniform=uniform if mode == _abi.ROUND_SR_UNIFORM else None,
                         seed=seed, rng_offset=rng_offset,
                         step=cache.device_step if on_device else None)
    if cache.device_step is not None:
        cache.device_step.add_(1)
    cache.step += 1
    return out


def enable_device_step(cache: MambaStateKernelCache) -> MambaStateKernelCache:
    """Keep the cache's stochastic-rounding step counter on the device as well (int64 [1],
    starting at cache.step): the counter- and Philox-mode updates then take their offset
    step * B*H*P*N from that tensor in the kernel and advance it with a tensor add, which a
    captured HIP graph replays, so every replay rounds with fresh draws. cache.step still counts
    the host-side calls. No counterpart in the reference (a host integer there, ms.py:659,
    716)."""
    cache.device_step = torch.tensor([cache.step], dtype=torch.int64, device=cache.q_state.device)
    return cache


def mx8_state_selective_update(*args, **kwargs) -> torch.Tensor:
    return mx_state_selective_update(*args, **kwargs)


def mx4_state_selective_update(*args, **kwargs) -> torch.Tensor:
    return mx_state_selective_update(*args, **kwargs)


def selective_state_update(state: torch.Tensor, x: torch.Tensor, dt: torch.Tensor,
                           A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                           D: torch.Tensor | None = None, z: torch.Tensor | None = None,
                           dt_bias: torch.Tensor | None = None, dt_softplus: bool = False,
                           state_batch_indices: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step of an unquantized (bf16 / fp16 / fp32) Mamba2 state, in place, with
    mamba-ssm 2.3.2.post1's selective_state_update interface: state [B,H,P,N] or [B,P,N];
    x, dt, z [B,H,P] or [B,P]; A [H,P,N] or [P,N]; B, C [B,G,N] or [B,N]; D, dt_bias [H,P] or
    [P]. fp32 arithmetic (h' = h*exp(A*dt) + (B*dt)*x, y = C.h' + D*x, y *= silu(z)); the state
    is rounded back to its dtype. Returns y in x's dtype. This is the update the reference runs
    for unregistered layers and as its bf16-state baseline (ms.py:738-747)."""
    if state_batch_indices is not None:
        raise NotImplementedError("state_batch_indices is not supported")
    has_heads = state.dim() > 3
    if state.dim() == 3:
        state = state.unsqueeze(1)
    if x.dim() == 2:
        x = x.unsqueeze(1)
    if dt.dim() == 2:
        dt = dt.unsqueeze(1)
    if A.dim() == 2:
        A = A.unsqueeze(0)
    if B.dim() == 2:
        B = B.unsqueeze(1)
    if C.dim() == 2:
        C = C.unsqueeze(1)
    if D is not None and D.dim() == 1:
        D = D.unsqueeze(0)
    if z is not None and z.dim() == 2:
        z = z.unsqueeze(1)
    if dt_bias is not None and dt_bias.dim() == 1:
        dt_bias = dt_bias.unsqueeze(0)
    out = torch.empty_like(x)
    _abi.selective_state_update(state, x, dt, dt_bias, A, B, C, D, z, out, dt_softplus)
    return out if has_heads else out.squeeze(1)


def patch_nemotron_h_mamba_decode_state_kernel(model, group_size: int = MX8_BLOCK_SIZE,
                                               stochastic: bool = True, seed: int = 1234, *,
                                               rng: str = "counter") -> None:
    """Rebind the remote module's selective_state_update (ms.py:732-767).

    States registered through register_mamba_state_kernel_caches (looked up by id) take the MX
    update; any other state falls through to the original function. The rounding mode, seed and
    generator (rng="philox" for the reference's tl.rand stream) live on the module and may be
    changed by calling this again.
    """
    if rng not in ("counter", "philox"):
        raise ValueError(f"rng must be 'counter' or 'philox', got {rng!r}")
    module = __import__(model.__class__.__module__, fromlist=["selective_state_update"])
    original = getattr(module, "_mx_state_kernel_original", module.selective_state_update)
    if original is None:  # the remote module found no mamba-ssm kernel: use the HIP update
        original = selective_state_update
    module._mx_state_kernel_stochastic = stochastic
    module._mx_state_kernel_seed = seed
    module._mx_state_kernel_rng = rng

    def selective_state_update_mx(ssm_state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                                  dt_softplus=False):
        registry = getattr(module, "_mamba_decode_state_kernel_caches", {})
        mx_cache = registry.get(id(ssm_state))
        if mx_cache is None:
            return original(ssm_state, x, dt, A, B, C, D=D, z=z, dt_bias=dt_bias,
                            dt_softplus=dt_softplus)
        return mx_state_selective_update(
            mx_cache, x, dt, A, B, C, D=D, z=z, dt_bias=dt_bias, dt_softplus=dt_softplus,
            stochastic=getattr(module, "_mx_state_kernel_stochastic", True),
            seed=getattr(module, "_mx_state_kernel_seed", 1234),
            rng=getattr(module, "_mx_state_kernel_rng", "counter"))

    if not getattr(module, "_mx_state_kernel_patched", False):
        module.selective_state_update = selective_state_update_mx
        module._mx_state_kernel_original = original
        module._mx_state_kernel_patched = True
    model._mx_state_kernel_group_size = group_size


def register_mamba_state_kernel_caches(model, cache_params, mode_by_layer: dict[int, str], *,
                                       layout: str = "reference") -> None:
    """Encode each listed layer's ssm_state into an MX cache keyed by id(ssm_state)
    (ms.py:770-796); publishes the registry on the model and on the remote module. `layout`
    (keyword only, no reference counterpart) selects the compact cache layout."""
    registry = {}
    for layer_idx, mode in mode_by_layer.items():
        if mode not in {"mx8", "mx4"}:
            raise ValueError(f"Only MX8 and MX4 state caches are supported, got mode={mode!r}")
        mixer = model.backbone.layers[layer_idx].mixer
        ssm_state = cache_params.ssm_states[layer_idx]
        state_4d = ssm_state.view(ssm_state.shape[0], mixer.num_heads, mixer.head_dim,
                                  mixer.ssm_state_size)
        bits = 8 if mode == "mx8" else 4
        registry[id(ssm_state)] = allocate_state_kernel_cache(
            state_4d, group_size=MX8_BLOCK_SIZE if bits == 8 else MX4_BLOCK_SIZE,
            format_bits=bits, layout=layout)
    model._mamba_decode_state_kernel_caches = registry
    module = __import__(model.__class__.__module__, fromlist=["selective_state_update"])
    module._mamba_decode_state_kernel_caches = dict(registry)
    model._mamba_decode_state_kernel_meta = {
        idx: SimpleNamespace(mode=mode, block_size=16, format_bits=8 if mode == "mx8" else 4)
        for idx, mode in mode_by_layer.items()
    }
