"""Writes tests/golden/rng_vectors.json: known-answer vectors of the counter-based generator of
LQ_ROUND_SR_COUNTER, computed with the scalar pure-Python implementation (oracle/rng.py's
lowbias32_scalar / uniform_scalar), for regression of the vectorized oracle and the HIP kernels.

    python tests/golden/make_rng_vectors.py
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import rng  # noqa: E402

CASES = [
    (1234, [0, 1, 2, 3, 4, 5, 6, 7, 100, 101, 8589934590, 8589934591, 8589934592, 8589934593]),
    (0, [0, 1, 1 << 32, (1 << 32) + 1, (1 << 40) + 3, 2**63]),
    (2**40 + 7, [10, 11, 12, 13, 999999999]),
]


def main():
    out = {
        "generator": "u = ((lowbias32(lo32(c>>1) ^ lowbias32(hi32(c>>1) ^ K)) >> 16*(c&1)) & 0xFFFF) / 65536",
        "lowbias32": {str(x): rng.lowbias32_scalar(x) for x in (0, 1, 2, 0xFFFFFFFF, 0x9E3779B9)},
        "cases": [
            {"seed": seed, "counters": counters,
             "uniforms": [rng.uniform_scalar(seed, c) for c in counters]}
            for seed, counters in CASES
        ],
    }
    path = Path(__file__).with_name("rng_vectors.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()
