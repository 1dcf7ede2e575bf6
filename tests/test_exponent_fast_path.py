"""The MX encoders' fast block-exponent path, checked exhaustively on the CPU.

block_exponent_fast (layer_quant_amd/csrc/mx_state.hip) skips the exact ceil(log2) rule of
mamba_state_8b_kernel.py:172, 560 for blocks whose absmax makes the rule's outcome certain.
tests/native/exponent_fast_path.c verifies that claim for every fp32 absmax in the fast range
against the correctly rounded quotient; the constants are read from the shipped source.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "layer_quant_amd" / "csrc" / "mx_state.hip"
CHECK = ROOT / "tests" / "native" / "exponent_fast_path.c"


def _constants():
    text = SRC.read_text()
    out = []
    for name in ("FAST_AMAX_LO", "FAST_AMAX_HI", "FAST_MANT_LO", "FAST_MANT_HI"):
        m = re.search(rf"constexpr uint32_t {name} = (0x[0-9a-fA-F]+|\d+)u;", text)
        assert m, name
        out.append(m.group(1))
    return out


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fast_exponent_path_exhaustive(tmp_path):
    exe = tmp_path / "exponent_fast_path"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(CHECK)],
                   check=True)
    res = subprocess.run([str(exe), *_constants()], capture_output=True, text=True, timeout=600)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    for line in res.stdout.splitlines():
        assert " bad=0 " in line, line
