"""The kernels' fast divisions are bit-identical to the reference arithmetic for bf16 operands.

The quantizer's division (one multiply + two FMAs with a correctly rounded reciprocal) is
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


SMOOTH_SRC = Path(__file__).resolve().parent / "native" / "smooth_exhaustive.c"


@pytest.fixture(scope="module")
def smooth_exe(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    out = tmp_path_factory.mktemp("smooth") / "smooth_exhaustive"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(SMOOTH_SRC), "-o", str(out), "-lm"], check=True)
    return out


@pytest.mark.parametrize("window", [
    (0, 254, 1, 254),       # every finite bf16 x (zero and subnormals included) over every normal s
    (0, 254, 0, 0),         # subnormal s (pairs whose RN(1/s) is infinite go to IEEE division)
])
def test_smoothing_single_multiply_is_exact(smooth_exe, window):
    """bf16(x * RN(1/s)) == bf16(RN(x / s)) wherever the quotient is in [2^-90, 2^100] and RN(1/s)
    is finite: the activation pass's smoothing fast path (about 1.3e9 pairs, a few seconds)."""
    res = subprocess.run([str(smooth_exe), *map(str, window)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith("mismatches=0 ")
    checked = int(res.stdout.split("checked=")[1].split()[0])
    assert checked > 2_000_000
