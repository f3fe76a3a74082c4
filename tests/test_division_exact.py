"""The kernels' fast division (one multiply + two FMAs with a correctly rounded reciprocal) is
bit-identical to IEEE float32 division for bf16 operands: exhaustive over mantissas and signs.

The exponent window covers every quotient exponent the kernels use the fast path for
(quotients in [2^-90, 2^100] with smoothing scales in [2^-17, 2^19] and the constant 7);
outside it the kernels switch to IEEE division.  Compiled with gcc, run on the CPU.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "native" / "div_exhaustive.c"


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    out = tmp_path_factory.mktemp("div") / "div_exhaustive"
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", str(SRC), "-o", str(out), "-lm"], check=True)
    return out


@pytest.mark.parametrize("window", [
    (100, 160, 110, 146),   # activations around 1 and smoothing scales 2^-17 .. 2^19
    (27, 40, 127, 131),     # tiny activations (2^-100 ..) over s in [1, 16)
    (214, 227, 120, 127),   # huge activations (.. 2^100) over s in [2^-7, 1)
    (20, 240, 129, 129),    # the scale computation amax / 7 over the whole useful range
])
def test_division_is_exact(exe, window):
    res = subprocess.run([str(exe), *map(str, window)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith("mismatches=0 ")
