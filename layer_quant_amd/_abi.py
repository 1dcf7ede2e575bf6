"""ctypes binding of liblayer_quant.so (the C ABI in include/layer_quant.h).

Only plain pointers, sizes and strides cross the boundary: each torch tensor is described by an
LQTensor (data pointer, dtype code, rank, shape, strides in elements). Every compute entry point
launches on the caller's current HIP stream and never synchronizes. There is no CPU fallback:
the library must be built (python -m layer_quant_amd.build) and tensors must live on a GPU.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liblayer_quant.so"

LQ_OK = 0
LQ_ERR_INVALID_ARG = -1
LQ_ERR_UNSUPPORTED = -2
LQ_ERR_WORKSPACE = -3
LQ_ERR_HIP = -4

ROUND_NEAREST_EVEN = 0
ROUND_HALF_UP = 1
ROUND_SR_UNIFORM = 2
ROUND_SR_COUNTER = 3
ROUND_SR_PHILOX = 4

# LQ_DIAG_* bits of the library's diagnostic switches, by their environment-variable names
DIAG_BITS = {
    "LQ_ATTN_FORCE_GENERIC": 1 << 0,
    "LQ_ATTN_REQUIRE_FAST": 1 << 1,
    "LQ_PREFILL_FORCE_GENERIC": 1 << 2,
    "LQ_PREFILL_REQUIRE_MFMA": 1 << 3,
    "LQ_MX_FORCE_GENERIC": 1 << 4,
    "LQ_MX_REQUIRE_ROWS": 1 << 5,
    "LQ_SSM_FORCE_GENERIC": 1 << 6,
    "LQ_SSM_REQUIRE_ROWS": 1 << 7,
    "LQ_ATTN_FOLD_MERGE": 1 << 8,
}

DTYPE_CODES = {
    torch.uint8: 0,
    torch.int8: 1,
    torch.float16: 2,
    torch.bfloat16: 3,
    torch.float32: 4,
    torch.int32: 5,
    torch.int64: 6,
}

# every symbol that include/layer_quant.h declares
EXPORTED_SYMBOLS = (
    "lq_abi_version",
    "lq_last_error",
    "lq_diagnostics",
    "lq_set_diagnostics",
    "lq_int4_pack_kv",
    "lq_int4_pack_kv_pair",
    "lq_int4_decode_attention_workspace",
    "lq_int4_decode_attention",
    "lq_int4_decode_attention_pack",
    "lq_int4_decode_attention_noalloc",
    "lq_int4_prefill_attention",
    "lq_mx_encode",
    "lq_mx_decode",
    "lq_mx_state_update",
    "lq_mx_state_update_device_step",
    "lq_selective_state_update",
)


class LQTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


class LQError(RuntimeError):
    """A non-zero return code of the C ABI; .code holds it."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_P = ctypes.POINTER(LQTensor)
_lib = None
_lib_lock = threading.Lock()


def _declare(lib: ctypes.CDLL) -> None:
    lib.lq_abi_version.restype = ctypes.c_int
    lib.lq_abi_version.argtypes = []
    lib.lq_last_error.restype = ctypes.c_char_p
    lib.lq_last_error.argtypes = []
    lib.lq_diagnostics.restype = ctypes.c_uint32
    lib.lq_diagnostics.argtypes = []
    lib.lq_set_diagnostics.restype = ctypes.c_uint32
    lib.lq_set_diagnostics.argtypes = [ctypes.c_uint32]
    lib.lq_int4_pack_kv.restype = ctypes.c_int
    lib.lq_int4_pack_kv.argtypes = [_P, _P, _P, _P, ctypes.c_int, ctypes.c_void_p]
    lib.lq_int4_pack_kv_pair.restype = ctypes.c_int
    lib.lq_int4_pack_kv_pair.argtypes = [_P] * 7 + [ctypes.c_int, ctypes.c_void_p]
    lib.lq_int4_decode_attention_workspace.restype = ctypes.c_size_t
    lib.lq_int4_decode_attention_workspace.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int]
    lib.lq_int4_decode_attention.restype = ctypes.c_int
    lib.lq_int4_decode_attention.argtypes = [_P] * 7 + [
        ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
        ctypes.c_void_p]
    lib.lq_int4_decode_attention_pack.restype = ctypes.c_int
    lib.lq_int4_decode_attention_pack.argtypes = [_P] * 9 + [
        ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
        ctypes.c_void_p]
    lib.lq_int4_decode_attention_noalloc.restype = ctypes.c_int
    lib.lq_int4_decode_attention_noalloc.argtypes = [_P] * 7 + [
        ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.lq_int4_prefill_attention.restype = ctypes.c_int
    lib.lq_int4_prefill_attention.argtypes = [_P] * 6 + [ctypes.c_int, ctypes.c_int,
                                                          ctypes.c_void_p]
    lib.lq_mx_encode.restype = ctypes.c_int
    lib.lq_mx_encode.argtypes = [_P] * 4 + [ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64,
                                            ctypes.c_uint64, ctypes.c_void_p]
    lib.lq_mx_decode.restype = ctypes.c_int
    lib.lq_mx_decode.argtypes = [_P] * 4 + [ctypes.c_void_p]
    lib.lq_mx_state_update.restype = ctypes.c_int
    lib.lq_mx_state_update.argtypes = [_P] * 12 + [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64, ctypes.c_uint64,
        ctypes.c_void_p]
    lib.lq_mx_state_update_device_step.restype = ctypes.c_int
    lib.lq_mx_state_update_device_step.argtypes = [_P] * 12 + [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64, ctypes.c_uint64, _P,
        ctypes.c_void_p]
    lib.lq_selective_state_update.restype = ctypes.c_int
    lib.lq_selective_state_update.argtypes = [_P] * 10 + [ctypes.c_int, ctypes.c_void_p]


def lib() -> ctypes.CDLL:
    """Load liblayer_quant.so once (the in-tree build, or the file LQ_LIBRARY names); raise if
    it has not been built."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                path = Path(os.environ.get("LQ_LIBRARY") or LIB_PATH)
                if not path.exists():
                    raise RuntimeError(
                        f"{path} is not built; run `python -m layer_quant_amd.build` "
                        "(or __graft_entry__.build()) first")
                handle = ctypes.CDLL(str(path))
                _declare(handle)
                _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().lq_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != LQ_OK:
        raise LQError(rc, f"{what} failed ({rc}): {last_error()}")


def desc(t: torch.Tensor | None):
    """LQTensor describing `t` (a pointer to it), or None for a missing optional tensor."""
    if t is None:
        return None
    if t.dim() > 4:
        raise ValueError(f"tensor of rank {t.dim()} exceeds the ABI's 4 dimensions")
    if t.dtype not in DTYPE_CODES:
        raise ValueError(f"dtype {t.dtype} is not supported by the ABI")
    d = LQTensor()
    d.data = t.data_ptr()
    d.dtype = DTYPE_CODES[t.dtype]
    d.ndim = t.dim()
    for i, (n, s) in enumerate(zip(t.shape, t.stride())):
        d.shape[i] = n
        d.stride[i] = s
    return ctypes.pointer(d)


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("layer_quant_amd kernels run on the GPU only; got a "
                               f"{t.device} tensor (no CPU fallback exists)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor argument")
    return dev


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def abi_version() -> int:
    return int(lib().lq_abi_version())


def diagnostics() -> set[str]:
    """Names of the diagnostic switches that are on (the library read them from the environment
    when it was loaded; set_diagnostics changes them)."""
    flags = int(lib().lq_diagnostics())
    return {name for name, bit in DIAG_BITS.items() if flags & bit}


def set_diagnostics(names) -> set[str]:
    """Turn on exactly the switches in `names` (LQ_MX_REQUIRE_ROWS, ...); returns the previous
    set. Process-wide: call it between kernel calls."""
    flags = 0
    for name in names:
        if name not in DIAG_BITS:
            raise ValueError(f"unknown diagnostic switch {name!r}")
        flags |= DIAG_BITS[name]
    prev = int(lib().lq_set_diagnostics(flags))
    return {name for name, bit in DIAG_BITS.items() if prev & bit}


@contextlib.contextmanager
def diagnostic(*names: str, on: bool = True):
    """Add the switches `names` for the block (nothing when `on` is false), then restore."""
    if not on:
        yield
        return
    prev = set_diagnostics(diagnostics() | set(names))
    try:
        yield
    finally:
        set_diagnostics(prev)


def int4_pack_kv(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                 positions: torch.Tensor, group_size: int) -> None:
    """Quantize x [B, Hkv, T, D] into rows `positions` of the packed cache (in place)."""
    dev = _require_gpu(x, packed, scale, positions)
    rc = lib().lq_int4_pack_kv(desc(x), desc(packed), desc(scale), desc(positions),
                               int(group_size), _stream(dev))
    check(rc, "lq_int4_pack_kv")


def int4_pack_kv_pair(k: torch.Tensor, v: torch.Tensor, k_packed: torch.Tensor,
                      v_packed: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                      positions: torch.Tensor, group_size: int) -> None:
    """int4_pack_kv of a layer's K and V in one launch."""
    dev = _require_gpu(k, v, k_packed, v_packed, k_scale, v_scale, positions)
    rc = lib().lq_int4_pack_kv_pair(desc(k), desc(v), desc(k_packed), desc(v_packed),
                                    desc(k_scale), desc(v_scale), desc(positions),
                                    int(group_size), _stream(dev))
    check(rc, "lq_int4_pack_kv_pair")


class _Workspace:
    """Per (device, stream) scratch buffer for the split-K partials, grown on demand. Allocated
    zeroed: the library's arrival counters at its start must be zero before first use (every
    call leaves them zero)."""

    def __init__(self):
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


_workspace = _Workspace()


def int4_decode_attention_workspace(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int,
                                    seq_len: int, group_size: int) -> int:
    return int(lib().lq_int4_decode_attention_workspace(batch, n_q_heads, n_kv_heads, head_dim,
                                                        seq_len, group_size))


def int4_decode_attention(q: torch.Tensor, k_packed: torch.Tensor, v_packed: torch.Tensor,
                          k_scale: torch.Tensor, v_scale: torch.Tensor,
                          mask: torch.Tensor | None, out: torch.Tensor, seq_len: int,
                          num_key_value_groups: int, group_size: int) -> torch.Tensor:
    """q_len=1 attention of q [B, Hq, 1, D] (or [B, Hq, D]) over the packed cache -> out."""
    dev = _require_gpu(q, k_packed, v_packed, k_scale, v_scale, mask, out)
    stream = _stream(dev)
    need = int4_decode_attention_workspace(q.shape[0], q.shape[1], k_packed.shape[1],
                                           q.shape[-1], seq_len, group_size)
    ws = _workspace.get(dev, stream, need)
    rc = lib().lq_int4_decode_attention(
        desc(q), desc(k_packed), desc(v_packed), desc(k_scale), desc(v_scale), desc(mask),
        desc(out), int(seq_len), int(num_key_value_groups), int(group_size),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream)
    check(rc, "lq_int4_decode_attention")
    return out


def int4_decode_attention_pack(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                               k_packed: torch.Tensor, v_packed: torch.Tensor,
                               k_scale: torch.Tensor, v_scale: torch.Tensor,
                               mask: torch.Tensor | None, out: torch.Tensor, seq_len: int,
                               num_key_value_groups: int, group_size: int) -> torch.Tensor:
    """int4_pack_kv_pair of the new token k_new, v_new [B, Hkv, 1, D] into cache row
    seq_len - 1, then int4_decode_attention over keys [0, seq_len) -> out; one launch on the MFMA
    path."""
    dev = _require_gpu(q, k_new, v_new, k_packed, v_packed, k_scale, v_scale, mask, out)
    stream = _stream(dev)
    need = int4_decode_attention_workspace(q.shape[0], q.shape[1], k_packed.shape[1],
                                           q.shape[-1], seq_len, group_size)
    ws = _workspace.get(dev, stream, need)
    rc = lib().lq_int4_decode_attention_pack(
        desc(q), desc(k_new), desc(v_new), desc(k_packed), desc(v_packed), desc(k_scale),
        desc(v_scale), desc(mask), desc(out), int(seq_len), int(num_key_value_groups),
        int(group_size), None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        stream)
    check(rc, "lq_int4_decode_attention_pack")
    return out


def int4_decode_attention_noalloc(q: torch.Tensor, k_packed: torch.Tensor,
                                  v_packed: torch.Tensor, k_scale: torch.Tensor,
                                  v_scale: torch.Tensor, mask: torch.Tensor | None,
                                  out: torch.Tensor, seq_len: int, num_key_value_groups: int,
                                  group_size: int) -> torch.Tensor:
    """int4_decode_attention with the split-K partials in the library's static per-device
    scratch: allocates nothing (for callers that cannot allocate). Calls overlapping on one GPU
    share that scratch and race."""
    dev = _require_gpu(q, k_packed, v_packed, k_scale, v_scale, mask, out)
    rc = lib().lq_int4_decode_attention_noalloc(
        desc(q), desc(k_packed), desc(v_packed), desc(k_scale), desc(v_scale), desc(mask),
        desc(out), int(seq_len), int(num_key_value_groups), int(group_size), _stream(dev))
    check(rc, "lq_int4_decode_attention_noalloc")
    return out


def int4_prefill_attention(q: torch.Tensor, k_packed: torch.Tensor, v_packed: torch.Tensor,
                           k_scale: torch.Tensor, v_scale: torch.Tensor, out: torch.Tensor,
                           num_key_value_groups: int, group_size: int) -> torch.Tensor:
    """Causal attention of q [B, Hq, L, D] over cache keys 0 .. t for position t -> out."""
    dev = _require_gpu(q, k_packed, v_packed, k_scale, v_scale, out)
    rc = lib().lq_int4_prefill_attention(desc(q), desc(k_packed), desc(v_packed), desc(k_scale),
                                         desc(v_scale), desc(out), int(num_key_value_groups),
                                         int(group_size), _stream(dev))
    check(rc, "lq_int4_prefill_attention")
    return out


def mx_encode(state: torch.Tensor, q_state: torch.Tensor, shared_exp: torch.Tensor,
              micro_exp: torch.Tensor, format_bits: int,
              round_mode: int = ROUND_NEAREST_EVEN, uniform: torch.Tensor | None = None,
              seed: int = 0, rng_offset: int = 0) -> None:
    dev = _require_gpu(state, q_state, shared_exp, micro_exp, uniform)
    rc = lib().lq_mx_encode(desc(state), desc(q_state), desc(shared_exp), desc(micro_exp),
                            int(format_bits), int(round_mode), desc(uniform),
                            int(seed) & ((1 << 64) - 1), int(rng_offset), _stream(dev))
    check(rc, "lq_mx_encode")


def mx_decode(q_state: torch.Tensor, shared_exp: torch.Tensor, micro_exp: torch.Tensor,
              out: torch.Tensor) -> torch.Tensor:
    dev = _require_gpu(q_state, shared_exp, micro_exp, out)
    rc = lib().lq_mx_decode(desc(q_state), desc(shared_exp), desc(micro_exp), desc(out),
                            _stream(dev))
    check(rc, "lq_mx_decode")
    return out


def mx_state_update(q_state, shared_exp, micro_exp, x, dt, dt_bias, A, B, C, D, z, out,
                    format_bits: int, dt_softplus: bool, round_mode: int,
                    uniform: torch.Tensor | None = None, seed: int = 1234,
                    rng_offset: int = 0, step: torch.Tensor | None = None) -> torch.Tensor:
    """The fused MX update in place. With `step` (an int64 [1] tensor on the device) the counter
    offset is rng_offset + step * B*H*P*N, read by the kernel (lq_mx_state_update_device_step):
    graph-capturable, with the caller advancing `step`."""
    dev = _require_gpu(q_state, shared_exp, micro_exp, x, dt, dt_bias, A, B, C, D, z, out,
                       uniform, step)
    args = (desc(q_state), desc(shared_exp), desc(micro_exp), desc(x), desc(dt), desc(dt_bias),
            desc(A), desc(B), desc(C), desc(D), desc(z), desc(out), int(format_bits),
            1 if dt_softplus else 0, int(round_mode), desc(uniform), int(seed) & ((1 << 64) - 1),
            int(rng_offset))
    if step is None:
        rc = lib().lq_mx_state_update(*args, _stream(dev))
        check(rc, "lq_mx_state_update")
    else:
        if step.dtype != torch.int64 or step.numel() < 1:
            raise ValueError("step must be an int64 tensor holding one value")
        rc = lib().lq_mx_state_update_device_step(*args, desc(step.view(-1)[:1]), _stream(dev))
        check(rc, "lq_mx_state_update_device_step")
    return out


def selective_state_update(state, x, dt, dt_bias, A, B, C, D, z, out,
                           dt_softplus: bool) -> torch.Tensor:
    dev = _require_gpu(state, x, dt, dt_bias, A, B, C, D, z, out)
    rc = lib().lq_selective_state_update(
        desc(state), desc(x), desc(dt), desc(dt_bias), desc(A), desc(B), desc(C), desc(D),
        desc(z), desc(out), 1 if dt_softplus else 0, _stream(dev))
    check(rc, "lq_selective_state_update")
    return out
