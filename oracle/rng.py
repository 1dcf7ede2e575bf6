"""Counter-based uniform generator of LQ_ROUND_SR_COUNTER -- TEST INFRASTRUCTURE ONLY.

The reference draws one Triton `tl.rand(seed, offset)` (Philox4x32-10) per element, with
offset = step*B*H*P*N + row*N + n (hybrid_quant/mamba_state_8b_kernel.py:196-199, 659, 716).
Triton's stream is version dependent and too costly at the HBM roofline, so the HIP kernels use
their own counter-based generator, restated here bit for bit:

    K        = lowbias32(seed_lo ^ lowbias32(seed_hi ^ 0x9E3779B9))       (per seed, on the host)
    counter  = rng_offset + ((b*H + h)*P + p)*N + n                         (same offsets as above)
    pair     = counter >> 1,  half = counter & 1
    bits32   = lowbias32(lo32(pair) ^ lowbias32(hi32(pair) ^ K))
    u16      = (bits32 >> (16*half)) & 0xFFFF                               (16-bit uniform integer)

lowbias32 is the 32-bit integer mixer x ^= x>>16; x *= 0x7feb352d; x ^= x>>15; x *= 0x846ca68b;
x ^= x>>16 (C. Wellons, "hash prospector", public domain). The even element of a pair takes the
low half. oracle.mx_state adds u16 * 2^-16 to the scaled value on a 2^-16 grid and floors
(bias within 2^-17 of one level step).

Pinning (tests/test_oracle_mx.py): the vectorized numpy version against a scalar pure-Python
version, known-answer vectors in tests/golden/rng_vectors.json, lowbias32 bijectivity on a
sample, and uniformity of the 16-bit output.
"""
from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
GOLDEN = 0x9E3779B9


def lowbias32_scalar(x: int) -> int:
    x &= M32
    x ^= x >> 16
    x = (x * 0x7FEB352D) & M32
    x ^= x >> 15
    x = (x * 0x846CA68B) & M32
    x ^= x >> 16
    return x


def lowbias32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint32)
    with np.errstate(over="ignore"):
        x = x ^ (x >> np.uint32(16))
        x = x * np.uint32(0x7FEB352D)
        x = x ^ (x >> np.uint32(15))
        x = x * np.uint32(0x846CA68B)
        x = x ^ (x >> np.uint32(16))
    return x


def seed_key(seed: int) -> int:
    """Per-seed key K (computed on the host and passed to the kernels)."""
    seed &= (1 << 64) - 1
    return lowbias32_scalar((seed & M32) ^ lowbias32_scalar(((seed >> 32) & M32) ^ GOLDEN))


def pair_bits_scalar(key: int, pair: int) -> int:
    return lowbias32_scalar((pair & M32) ^ lowbias32_scalar(((pair >> 32) & M32) ^ key))


def uniform_scalar(seed: int, counter: int) -> float:
    bits = pair_bits_scalar(seed_key(seed), counter >> 1)
    return float((bits >> (16 * (counter & 1))) & 0xFFFF) / 65536.0


def uniforms_u16(seed: int, counters: np.ndarray) -> np.ndarray:
    """Vectorized generator: counters (uint64 array) -> 16-bit uniform integers (uint32)."""
    c = np.asarray(counters, dtype=np.uint64)
    key = np.uint32(seed_key(seed))
    pair = c >> np.uint64(1)
    lo = (pair & np.uint64(M32)).astype(np.uint32)
    hi = (pair >> np.uint64(32)).astype(np.uint32)
    bits = lowbias32(lo ^ lowbias32(hi ^ key))
    half = (c & np.uint64(1)).astype(np.uint32)
    return (bits >> (np.uint32(16) * half)) & np.uint32(0xFFFF)


def uniforms(seed: int, counters: np.ndarray) -> np.ndarray:
    """The same draws as float32 uniforms u16 * 2^-16 in [0, 1)."""
    return (uniforms_u16(seed, counters).astype(np.float32) * np.float32(1.0 / 65536.0)).astype(
        np.float32)


def state_u16(seed: int, rng_offset: int, shape: tuple[int, ...]) -> np.ndarray:
    """16-bit draws (uint32) for an MX state of `shape` = (B, H, P, N) at the given offset."""
    n = int(np.prod(shape))
    counters = np.uint64(rng_offset) + np.arange(n, dtype=np.uint64)
    return uniforms_u16(seed, counters).reshape(shape)


def state_uniforms(seed: int, rng_offset: int, shape: tuple[int, ...]) -> np.ndarray:
    """Float32 uniforms for an MX state of `shape` = (B, H, P, N) at the given offset."""
    return (state_u16(seed, rng_offset, shape).astype(np.float32) * np.float32(1.0 / 65536.0))
