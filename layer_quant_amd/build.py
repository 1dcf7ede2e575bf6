"""Build liblayer_quant.so for gfx950 with hipcc (in-tree, no JIT cache).

    python -m layer_quant_amd.build          # compile every csrc/*.hip and link the library

Every HIP source is compiled with packed-fp32 instruction selection disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops) and default IEEE fp32 division, which the
bit-exact encoders rely on.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB_PATH = LIB_DIR / "liblayer_quant.so"
BUILD_DIR = PKG.parent / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source additions. The decode attention keeps its MFMA accumulators in VGPRs: with the
# default AGPR form the compiler copied all 36 of them to VGPRs at the top of every 32-key tile
# (for the rarely taken softmax rescale), 36 extra instructions per tile.
SOURCE_FLAGS = {
    "int4_attention_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    noise = "'-packed-fp32-ops' is not a recognized feature"
    for line in (res.stdout + res.stderr).splitlines():
        if line.strip() and noise not in line and verbose:
            print(line)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link liblayer_quant.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
