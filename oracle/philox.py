"""Triton's tl.rand stream (Philox4x32-10) -- TEST INFRASTRUCTURE ONLY.

The reference's stochastic writeback draws u = tl.rand(RNG_SEED, RNG_OFFSET + index) per state
element (hybrid_quant/mamba_state_8b_kernel.py:196-199, 399-406, 478-480, 528-530), with
RNG_OFFSET = step*B*H*P*N (:659, 699, 716) and index = ((b*H + h)*P + p)*N + n. tl.rand lives in
a third-party library, Triton (torch 2.8.0 of the reference's requirements.txt pins Triton
3.4.0; triton-rocm 3.6.0 is installed here), triton/language/random.py. Restated here from the
published algorithm (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
SC'11, the Random123 Philox4x32 with 10 rounds) and Triton's conversion:

    counter  (c0, c1, c2, c3) = (lo32(offset), hi32(offset), 0, 0)
    key      (k0, k1)         = (lo32(seed), hi32(seed))
    round    c0' = mulhi(0xCD9E8D57, c2) ^ c1 ^ k0    c1' = lo32(0xCD9E8D57 * c2)
             c2' = mulhi(0xD2511F53, c0) ^ c3 ^ k1    c3' = lo32(0xD2511F53 * c0)
             k0 += 0x9E3779B9, k1 += 0xBB67AE85        (10 rounds; the first uses the seed key)
    bits     = c0 after the last round
    uniform  x = int32(bits); x = x < 0 ? -x - 1 : x; u = fp32(x) * fp32(4.6566127342e-10)
             (fp32(x) rounds to nearest even; the scale is 0x1.fffffep-32; u in [0, 1 - 2^-24])

Offsets: the reference adds its constexpr RNG_OFFSET to int32 indices, so its offsets are int32
(a sum past 2^31 wraps, which leaves the same low word and a zero high word); with Triton 3.6 a
constexpr RNG_OFFSET of 2^31 or more is rejected when the kernel compiles ("Scalar ... is out of
range for type int32"). tl.rand of int64 offsets uses (lo32, hi32) as above, which equals the
int32 form wherever that one compiles; LQ_ROUND_SR_PHILOX defines every offset that way.

Pinning (tests/test_oracle_philox.py): philox4x32 against the Random123 known-answer vectors
(counter/key all zeros, all ones, and the pi digits), tl.randint and tl.rand against Triton's own
outputs (tests/golden/philox_tl_rand.json, written by tests/golden/make_philox_vectors.py with
Triton's CPU interpreter) for five seeds (one above 2^32) and offsets up to 2^62, a scalar
pure-Python restatement against the vectorized one, and the conversion's end points.
"""
from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
ROUND_A = 0xD2511F53  # multiplies c0
ROUND_B = 0xCD9E8D57  # multiplies c2
KEY_A = 0x9E3779B9
KEY_B = 0xBB67AE85
ROUNDS = 10
SCALE = np.float32(4.6566127342e-10)  # 0x1.fffffep-32


def philox4x32_scalar(c: tuple[int, int, int, int], k: tuple[int, int],
                      rounds: int = ROUNDS) -> tuple[int, int, int, int]:
    c0, c1, c2, c3 = (x & M32 for x in c)
    k0, k1 = (x & M32 for x in k)
    for _ in range(rounds):
        pa = ROUND_A * c0
        pb = ROUND_B * c2
        c0, c1, c2, c3 = ((pb >> 32) ^ c1 ^ k0, pb & M32, (pa >> 32) ^ c3 ^ k1, pa & M32)
        k0 = (k0 + KEY_A) & M32
        k1 = (k1 + KEY_B) & M32
    return c0, c1, c2, c3


def philox4x32(c0, c1, c2, c3, k0: int, k1: int, rounds: int = ROUNDS):
    """Vectorized Philox4x32 (uint32 arrays in, uint32 arrays out)."""
    c = [np.asarray(x, dtype=np.uint64) & np.uint64(M32) for x in (c0, c1, c2, c3)]
    c = np.broadcast_arrays(*c)
    c0, c1, c2, c3 = (np.array(x, dtype=np.uint64) for x in c)
    k0 = np.uint64(k0 & M32)
    k1 = np.uint64(k1 & M32)
    m32 = np.uint64(M32)
    s32 = np.uint64(32)
    for _ in range(rounds):
        pa = np.uint64(ROUND_A) * c0
        pb = np.uint64(ROUND_B) * c2
        c0, c1, c2, c3 = ((pb >> s32) ^ c1 ^ k0, pb & m32, (pa >> s32) ^ c3 ^ k1, pa & m32)
        k0 = (k0 + np.uint64(KEY_A)) & m32
        k1 = (k1 + np.uint64(KEY_B)) & m32
    return tuple(x.astype(np.uint32) for x in (c0, c1, c2, c3))


def randint(seed: int, offsets) -> np.ndarray:
    """tl.randint(seed, offsets) for offsets in [0, 2^64): the first Philox word (uint32)."""
    off = np.asarray(offsets, dtype=np.uint64)
    seed &= (1 << 64) - 1
    lo = off & np.uint64(M32)
    hi = off >> np.uint64(32)
    return philox4x32(lo, hi, 0, 0, seed & M32, seed >> 32)[0]


def to_uniform(bits) -> np.ndarray:
    """Triton's uint_to_uniform_float for 32-bit words."""
    x = np.asarray(bits, dtype=np.uint32).view(np.int32)
    x = np.where(x < 0, ~x, x)  # -x - 1 without overflow
    return (x.astype(np.float32) * SCALE).astype(np.float32)


def to_uniform_scalar(bits: int) -> float:
    x = bits & M32
    if x >= 1 << 31:
        x = (1 << 32) - 1 - x  # -int32(bits) - 1
    return float(np.float32(np.float32(x) * SCALE))


def rand(seed: int, offsets) -> np.ndarray:
    """tl.rand(seed, offsets): float32 uniforms in [0, 1)."""
    return to_uniform(randint(seed, offsets))


def state_uniforms(seed: int, rng_offset: int, shape: tuple[int, ...]) -> np.ndarray:
    """Uniforms of LQ_ROUND_SR_PHILOX for a state of `shape` = (B, H, P, N): element
    (b, h, p, n) draws tl.rand(seed, rng_offset + ((b*H + h)*P + p)*N + n)."""
    n = int(np.prod(shape))
    offsets = np.uint64(rng_offset) + np.arange(n, dtype=np.uint64)
    return rand(seed, offsets).reshape(shape)
