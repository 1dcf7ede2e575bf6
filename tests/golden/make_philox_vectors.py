"""Writes tests/golden/philox_tl_rand.json: Triton's own tl.randint / tl.rand outputs for
(seed, offset) pairs, the stream the reference's stochastic writeback draws
(hybrid_quant/mamba_state_8b_kernel.py:198, 405, 479, 529: tl.rand(RNG_SEED, RNG_OFFSET + index)).

Triton is a third-party library of the reference (torch 2.8.0 pins Triton 3.4.0; this container
has triton-rocm 3.6.0). Its kernels run here in Triton's CPU interpreter (TRITON_INTERPRET=1), so
no GPU is needed; the reference itself is not imported. Two launch forms:

  * "constexpr": the offset base is a tl.constexpr added to an int32 arange, as in the
    reference's kernels (bases below 2^31 only: Triton 3.6 rejects a larger constexpr there
    with "Scalar ... is out of range for type int32");
  * "int64": the base is a runtime int64 argument, so the offsets are int64 and tl.randint
    splits them into the counter words (lo32, hi32).

Run: python tests/golden/make_philox_vectors.py
"""
from __future__ import annotations

import json
import os
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

N = 8


@triton.jit
def _rand_constexpr(bits_ptr, u_ptr, SEED: tl.constexpr, OFF: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    tl.store(bits_ptr + offs, tl.randint(SEED, OFF + offs).to(tl.int32, bitcast=True))
    tl.store(u_ptr + offs, tl.rand(SEED, OFF + offs))


@triton.jit
def _rand_int64(bits_ptr, u_ptr, SEED: tl.constexpr, off, BLOCK: tl.constexpr):
    offs = off + tl.arange(0, BLOCK).to(tl.int64)
    tl.store(bits_ptr + tl.arange(0, BLOCK), tl.randint(SEED, offs).to(tl.int32, bitcast=True))
    tl.store(u_ptr + tl.arange(0, BLOCK), tl.rand(SEED, offs))


def _run(kernel, seed: int, base: int) -> dict:
    bits = torch.empty(N, dtype=torch.int32)
    u = torch.empty(N, dtype=torch.float32)
    kernel[(1,)](bits, u, seed, base, BLOCK=N)
    return {
        "seed": seed,
        "base": base,
        "offsets": [base + i for i in range(N)],
        "bits": [int(b) & 0xFFFFFFFF for b in bits.tolist()],
        "uniform_f32_bits": [int(x) & 0xFFFFFFFF for x in u.view(torch.int32).tolist()],
    }


def main() -> None:
    seeds = [1234, 0, 0xFFFFFFFF, (1 << 32) + 7, (1 << 62) + 12345]
    bases32 = [0, 1000, (1 << 31) - 4]
    bases64 = [0, (1 << 31) - 4, (1 << 32) - 3, (1 << 32) + 12345, 5 * (1 << 33) + 77, (1 << 62) + 3]
    cases = []
    for seed in seeds:
        for base in bases32:
            cases.append(dict(_run(_rand_constexpr, seed, base), form="constexpr"))
        for base in bases64:
            cases.append(dict(_run(_rand_int64, seed, base), form="int64"))
    out = {
        "source": f"triton {triton.__version__} tl.randint / tl.rand, CPU interpreter",
        "cases": cases,
    }
    path = Path(__file__).with_name("philox_tl_rand.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
