"""The C ABI without a GPU: the library loads, exports every symbol include/*.h declares, and
rejects invalid arguments before any HIP call."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from layer_quant_amd import _abi

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(lq_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    declared = _declared_symbols()
    assert declared, "no declarations found"
    assert declared == set(_abi.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_empty_error():
    assert _abi.abi_version() == 1
    assert isinstance(_abi.last_error(), str)


def test_diagnostic_switches():
    """The switches are set and read through the ABI; unknown bits are dropped; the context
    manager restores the previous set. (That the library reads them from the environment at
    load time is checked in a child process, whose library load sees a set variable.)"""
    import subprocess
    import sys

    lib = _abi.lib()
    prev = _abi.diagnostics()
    try:
        assert lib.lq_set_diagnostics(0xFFFFFFFF) == sum(_abi.DIAG_BITS[n] for n in prev)
        assert lib.lq_diagnostics() == sum(_abi.DIAG_BITS.values())
        _abi.set_diagnostics([])
        with _abi.diagnostic("LQ_MX_REQUIRE_ROWS", "LQ_SSM_FORCE_GENERIC"):
            assert _abi.diagnostics() == {"LQ_MX_REQUIRE_ROWS", "LQ_SSM_FORCE_GENERIC"}
            with _abi.diagnostic("LQ_ATTN_REQUIRE_FAST", on=False):
                assert "LQ_ATTN_REQUIRE_FAST" not in _abi.diagnostics()
        assert _abi.diagnostics() == set()
        with pytest.raises(ValueError):
            _abi.set_diagnostics(["LQ_NOT_A_SWITCH"])
    finally:
        _abi.set_diagnostics(prev)
    code = "from layer_quant_amd import _abi; print(sorted(_abi.diagnostics()))"
    env = {k: v for k, v in __import__("os").environ.items() if not k.startswith("LQ_")}
    env.update(LQ_PREFILL_REQUIRE_MFMA="1", LQ_MX_FORCE_GENERIC="0")
    out = subprocess.run([sys.executable, "-c", code], env=env, cwd=ROOT, capture_output=True,
                         text=True, check=True).stdout
    assert out.strip() == "['LQ_PREFILL_REQUIRE_MFMA']"


def _fake(shape, dtype, data=0x1000):
    """A descriptor with a non-null fake device address (never dereferenced by validation)."""
    t = _abi.LQTensor()
    t.data = data
    t.dtype = _abi.DTYPE_CODES[dtype]
    t.ndim = len(shape)
    stride = 1
    for i in reversed(range(len(shape))):
        t.shape[i] = shape[i]
        t.stride[i] = stride
        stride *= shape[i]
    return ctypes.pointer(t)


def test_pack_rejects_bad_arguments():
    lib = _abi.lib()
    x = _fake((2, 8, 1, 128), torch.bfloat16)
    packed = _fake((2, 8, 16, 64), torch.uint8)
    scale = _fake((2, 8, 16, 4), torch.float32)
    pos = _fake((1,), torch.int64)
    assert lib.lq_int4_pack_kv(None, packed, scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    assert lib.lq_int4_pack_kv(x, packed, scale, pos, 31, None) == _abi.LQ_ERR_INVALID_ARG
    assert "even" in _abi.last_error()
    assert lib.lq_int4_pack_kv(x, packed, scale, pos, 48, None) == _abi.LQ_ERR_INVALID_ARG
    assert "divisible" in _abi.last_error()
    bad_scale = _fake((2, 8, 16, 2), torch.float32)
    assert lib.lq_int4_pack_kv(x, packed, bad_scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    two_pos = _fake((2,), torch.int64)
    assert lib.lq_int4_pack_kv(x, packed, scale, two_pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    assert "q_len" in _abi.last_error()


def test_pack_pair_rejects_bad_arguments():
    """Each of the two triples goes through the single-tensor checks before anything launches."""
    lib = _abi.lib()
    x = _fake((2, 8, 1, 128), torch.bfloat16)
    packed = _fake((2, 8, 16, 64), torch.uint8)
    scale = _fake((2, 8, 16, 4), torch.float32)
    pos = _fake((1,), torch.int64)
    f = lib.lq_int4_pack_kv_pair
    assert f(None, x, packed, packed, scale, scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    assert f(x, None, packed, packed, scale, scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    assert f(x, x, packed, packed, scale, scale, pos, 31, None) == _abi.LQ_ERR_INVALID_ARG
    assert "even" in _abi.last_error()
    bad_scale = _fake((2, 8, 16, 2), torch.float32)
    assert f(x, x, packed, packed, scale, bad_scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    assert "scale must be" in _abi.last_error()
    bad_packed = _fake((2, 8, 16, 32), torch.uint8)
    assert f(x, x, packed, bad_packed, scale, scale, pos, 32, None) == _abi.LQ_ERR_INVALID_ARG
    two_pos = _fake((2,), torch.int64)
    assert f(x, x, packed, packed, scale, scale, two_pos, 32, None) == _abi.LQ_ERR_INVALID_ARG


def test_attention_rejects_bad_arguments():
    lib = _abi.lib()
    kp = _fake((2, 8, 64, 64), torch.uint8)
    ks = _fake((2, 8, 64, 4), torch.float32)
    out = _fake((2, 32, 128), torch.bfloat16)
    q2 = _fake((2, 32, 2, 128), torch.bfloat16)
    assert lib.lq_int4_decode_attention(q2, kp, kp, ks, ks, None, out, 10, 4, 32, None, 0,
                                        None) == _abi.LQ_ERR_INVALID_ARG
    assert "q_len=1" in _abi.last_error()
    q = _fake((2, 32, 1, 128), torch.bfloat16)
    assert lib.lq_int4_decode_attention(q, kp, kp, ks, ks, None, out, 65, 4, 32, None, 0,
                                        None) == _abi.LQ_ERR_INVALID_ARG
    assert lib.lq_int4_decode_attention(q, kp, kp, ks, ks, None, out, 10, 3, 32, None, 0,
                                        None) == _abi.LQ_ERR_INVALID_ARG
    # a long context needs split-K partials: no workspace is an error, not a fault
    kp2 = _fake((2, 8, 16384, 64), torch.uint8)
    ks2 = _fake((2, 8, 16384, 4), torch.float32)
    assert _abi.int4_decode_attention_workspace(2, 32, 8, 128, 16384, 32) > 0
    assert lib.lq_int4_decode_attention(q, kp2, kp2, ks2, ks2, None, out, 16384, 4, 32, None,
                                        0, None) == _abi.LQ_ERR_WORKSPACE


def test_fused_pack_attention_rejects_bad_arguments():
    """lq_int4_decode_attention_pack checks its token tensors as lq_int4_pack_kv_pair does (one
    token, into row seq_len - 1) and the rest as lq_int4_decode_attention does."""
    lib = _abi.lib()
    f = lib.lq_int4_decode_attention_pack
    kp = _fake((2, 8, 64, 64), torch.uint8)
    ks = _fake((2, 8, 64, 4), torch.float32)
    out = _fake((2, 32, 128), torch.bfloat16)
    q = _fake((2, 32, 1, 128), torch.bfloat16)
    kn = _fake((2, 8, 1, 128), torch.bfloat16)
    assert f(q, None, kn, kp, kp, ks, ks, None, out, 10, 4, 32, None, 0,
             None) == _abi.LQ_ERR_INVALID_ARG
    assert "k_new" in _abi.last_error()
    two = _fake((2, 8, 2, 128), torch.bfloat16)
    assert f(q, two, two, kp, kp, ks, ks, None, out, 10, 4, 32, None, 0,
             None) == _abi.LQ_ERR_INVALID_ARG
    assert "one token" in _abi.last_error()
    heads = _fake((2, 4, 1, 128), torch.bfloat16)
    assert f(q, heads, kn, kp, kp, ks, ks, None, out, 10, 4, 32, None, 0,
             None) == _abi.LQ_ERR_INVALID_ARG
    assert f(q, kn, kn, kp, kp, ks, ks, None, out, 65, 4, 32, None, 0,
             None) == _abi.LQ_ERR_INVALID_ARG
    assert "capacity" in _abi.last_error()
    ints = _fake((2, 8, 1, 128), torch.int32)
    assert f(q, kn, ints, kp, kp, ks, ks, None, out, 10, 4, 32, None, 0,
             None) == _abi.LQ_ERR_INVALID_ARG


def test_prefill_rejects_bad_arguments():
    lib = _abi.lib()
    kp = _fake((2, 8, 64, 64), torch.uint8)
    ks = _fake((2, 8, 64, 4), torch.float32)
    q = _fake((2, 32, 48, 128), torch.bfloat16)
    out = _fake((2, 32, 48, 128), torch.bfloat16)
    long_q = _fake((2, 32, 65, 128), torch.bfloat16)
    long_out = _fake((2, 32, 65, 128), torch.bfloat16)
    assert lib.lq_int4_prefill_attention(long_q, kp, kp, ks, ks, long_out, 4, 32,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert "capacity" in _abi.last_error()
    assert lib.lq_int4_prefill_attention(q, kp, kp, ks, ks, out, 3, 32,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert lib.lq_int4_prefill_attention(q, kp, kp, ks, ks, out, 4, 31,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    short_out = _fake((2, 32, 47, 128), torch.bfloat16)
    assert lib.lq_int4_prefill_attention(q, kp, kp, ks, ks, short_out, 4, 32,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert "out must be" in _abi.last_error()
    bad_ks = _fake((2, 8, 64, 2), torch.float32)
    assert lib.lq_int4_prefill_attention(q, kp, kp, bad_ks, ks, out, 4, 32,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    q3 = _fake((2, 32, 128), torch.bfloat16)
    assert lib.lq_int4_prefill_attention(q3, kp, kp, ks, ks, out, 4, 32,
                                         None) == _abi.LQ_ERR_INVALID_ARG


def test_mx_rejects_bad_arguments():
    lib = _abi.lib()
    qs = _fake((2, 4, 8, 128), torch.int8)
    e = _fake((2, 4, 8, 8), torch.uint8)
    m = _fake((2, 4, 8, 64), torch.uint8)
    x = _fake((2, 4, 8), torch.bfloat16)
    A = _fake((4, 8, 128), torch.float32)
    B = _fake((2, 2, 128), torch.bfloat16)
    out = _fake((2, 4, 8), torch.bfloat16)
    args = [qs, e, m, x, x, None, A, B, B, None, None, out]
    assert lib.lq_mx_state_update(*args, 6, 1, 1, None, 0, 0, None) == _abi.LQ_ERR_INVALID_ARG
    assert "format_bits=6" in _abi.last_error()
    assert lib.lq_mx_state_update(*args, 8, 1, 2, None, 0, 0, None) == _abi.LQ_ERR_INVALID_ARG
    assert lib.lq_mx_state_update(*args, 8, 1, 3, None, 0, 1, None) == _abi.LQ_ERR_INVALID_ARG
    assert "even" in _abi.last_error()
    bad_x = _fake((2, 4, 7), torch.bfloat16)
    args_bad = [qs, e, m, bad_x, x, None, A, B, B, None, None, out]
    assert lib.lq_mx_state_update(*args_bad, 8, 1, 1, None, 0, 0, None) == _abi.LQ_ERR_INVALID_ARG
    assert "Expected x shape" in _abi.last_error()
    B2 = _fake((2, 128), torch.bfloat16)
    args_b = [qs, e, m, x, x, None, A, B2, B, None, None, out]
    assert lib.lq_mx_state_update(*args_b, 8, 1, 1, None, 0, 0, None) == _abi.LQ_ERR_INVALID_ARG
    assert "[batch, ngroups, dstate]" in _abi.last_error()
    q_odd = _fake((2, 4, 8, 40), torch.int8)
    assert lib.lq_mx_encode(_fake((2, 4, 8, 40), torch.float32), q_odd, e, m, 8, 0, None, 0, 0,
                            None) == _abi.LQ_ERR_INVALID_ARG
    assert "divisible by 16" in _abi.last_error()


def test_compute_wrappers_refuse_cpu_tensors():
    x = torch.zeros(1, 1, 1, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        _abi.int4_pack_kv(x, torch.zeros(1, 1, 4, 64, dtype=torch.uint8), torch.zeros(1, 1, 4, 4),
                          torch.zeros(1, dtype=torch.long), 32)


def test_selective_state_update_rejects_bad_arguments():
    lib = _abi.lib()
    st = _fake((2, 4, 8, 128), torch.bfloat16)
    x = _fake((2, 4, 8), torch.bfloat16)
    A = _fake((4, 8, 128), torch.float32)
    B = _fake((2, 2, 128), torch.bfloat16)
    out = _fake((2, 4, 8), torch.bfloat16)
    assert lib.lq_selective_state_update(None, x, x, None, A, B, B, None, None, out, 1,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    st_int = _fake((2, 4, 8, 128), torch.int8)
    assert lib.lq_selective_state_update(st_int, x, x, None, A, B, B, None, None, out, 1,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert "not f32/f16/bf16" in _abi.last_error()
    st40 = _fake((2, 4, 8, 40), torch.bfloat16)
    assert lib.lq_selective_state_update(st40, x, x, None, A, B, B, None, None, out, 1,
                                         None) == _abi.LQ_ERR_UNSUPPORTED
    assert "multiple of 16" in _abi.last_error()
    bad_dt = _fake((2, 4, 9), torch.bfloat16)
    assert lib.lq_selective_state_update(st, x, bad_dt, None, A, B, B, None, None, out, 1,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert "dt must be [2, 4, 8]" in _abi.last_error()
    B3 = _fake((2, 3, 128), torch.bfloat16)
    assert lib.lq_selective_state_update(st, x, x, None, A, B3, B3, None, None, out, 1,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    assert "not divisible by ngroups=3" in _abi.last_error()
    D_bad = _fake((4, 7), torch.float32)
    assert lib.lq_selective_state_update(st, x, x, None, A, B, B, D_bad, None, out, 1,
                                         None) == _abi.LQ_ERR_INVALID_ARG
    with pytest.raises(RuntimeError, match="GPU only"):
        _abi.selective_state_update(torch.zeros(1, 1, 1, 16), torch.zeros(1, 1, 1),
                                    torch.zeros(1, 1, 1), None, torch.zeros(1, 1, 16),
                                    torch.zeros(1, 1, 16), torch.zeros(1, 1, 16), None, None,
                                    torch.zeros(1, 1, 1), False)
