"""lq_int4_decode_attention_noalloc: the split-K partials in the library's static per-device
scratch instead of a caller workspace. Its outputs must equal lq_int4_decode_attention's, on
consecutive calls (the second smaller, so it reads a scratch still holding the first call's
partials), on both kernels and with a mask; shapes whose partials exceed the scratch are rejected
before anything launches."""
import ctypes

import pytest
import torch

from layer_quant_amd import _abi


def _cache(gpu, gen, b, hkv, s, d, g):
    kp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    vp = torch.randint(0, 256, (b, hkv, s, d // 2), dtype=torch.uint8, device=gpu, generator=gen)
    ks = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) * 0.5 + 0.01
    vs = torch.rand(b, hkv, s, d // g, device=gpu, generator=gen) * 0.5 + 0.01
    return kp, vp, ks, vs


# b, hkv, nrep, s, g, q dtype, masked: each row's partials go through the scratch (split-K)
CASES = [
    (2, 8, 4, 16384, 32, torch.bfloat16, False),   # MFMA kernel, 32 splits
    (1, 8, 4, 3000, 64, torch.bfloat16, False),    # smaller: fewer splits over stale partials
    (3, 2, 4, 5000, 32, torch.bfloat16, True),     # masked MFMA instance
    (2, 4, 2, 2500, 32, torch.float32, False),     # generic kernel (fp32 queries)
    (1, 2, 2, 700, 32, torch.float32, True),       # generic, masked, smaller again
]


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(gpu):
    gen = torch.Generator(device=gpu).manual_seed(123)
    d = 128
    for b, hkv, nrep, s, g, qdt, masked in CASES:
        need = _abi.int4_decode_attention_workspace(b, hkv * nrep, hkv, d, s, g)
        assert 0 < need <= 8 << 20, (b, s, need)
        kp, vp, ks, vs = _cache(gpu, gen, b, hkv, s, d, g)
        q = torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen).to(qdt)
        mask = None
        if masked:
            mask = torch.randn(b, 1, 1, s, device=gpu, generator=gen) * 2
            mask[0, :, :, :100] = float("-inf")
        ref = torch.empty(b, hkv * nrep, d, device=gpu)
        _abi.int4_decode_attention(q, kp, vp, ks, vs, mask, ref, s, nrep, g)
        for _ in range(2):
            out = torch.full_like(ref, float("nan"))
            _abi.int4_decode_attention_noalloc(q, kp, vp, ks, vs, mask, out, s, nrep, g)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), (b, hkv, nrep, s, g, qdt, masked)
        assert torch.isfinite(ref).all()


@pytest.mark.gpu
def test_noalloc_single_split_needs_no_scratch(gpu):
    """B * Hkv large enough for one split per (batch, KV head): no partials at all."""
    gen = torch.Generator(device=gpu).manual_seed(7)
    b, hkv, nrep, s, g, d = 64, 8, 4, 4096, 32, 128
    assert _abi.int4_decode_attention_workspace(b, hkv * nrep, hkv, d, s, g) == 0
    kp, vp, ks, vs = _cache(gpu, gen, b, hkv, s, d, g)
    q = torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen).to(torch.bfloat16)
    ref = torch.empty(b, hkv * nrep, d, device=gpu)
    out = torch.empty_like(ref)
    _abi.int4_decode_attention(q, kp, vp, ks, vs, None, ref, s, nrep, g)
    _abi.int4_decode_attention_noalloc(q, kp, vp, ks, vs, None, out, s, nrep, g)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def _fake(shape, dtype, data=0x1000):
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


def test_noalloc_rejects_partials_larger_than_scratch():
    """2047 batch rows x 1 query head at head_dim 512 (generic kernel, 2 splits) needs about
    8.4 MB of partials: rejected with LQ_ERR_WORKSPACE before any HIP call (runs without a GPU)."""
    b, hq, d, s, g = 2047, 1, 512, 128, 128
    assert _abi.int4_decode_attention_workspace(b, hq, 1, d, s, g) > 8 << 20
    lib = _abi.lib()
    q = _fake((b, hq, 1, d), torch.float32)
    kp = _fake((b, 1, s, d // 2), torch.uint8)
    ks = _fake((b, 1, s, d // g), torch.float32)
    out = _fake((b, hq, d), torch.float32)
    rc = lib.lq_int4_decode_attention_noalloc(q, kp, kp, ks, ks, None, out, s, 1, g, None)
    assert rc == _abi.LQ_ERR_WORKSPACE
    assert "static scratch" in _abi.last_error()
    # invalid arguments are rejected exactly as by lq_int4_decode_attention
    rc = lib.lq_int4_decode_attention_noalloc(q, kp, kp, ks, ks, None, out, s + 1, 1, g, None)
    assert rc == _abi.LQ_ERR_INVALID_ARG and "seq_len" in _abi.last_error()
