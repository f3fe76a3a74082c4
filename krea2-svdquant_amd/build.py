"""Build ``_lib/libsvdq_gfx950.so`` from ``csrc/`` with hipcc for gfx950 (in-tree).

The library links ``libamdhip64.so.7`` by soname only; loaded after ``import torch`` it
binds to the HIP runtime torch already has in the process.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libsvdq_gfx950.so"
SOURCES = ["svdq_act.hip", "svdq_gemm.hip", "svdq_block.hip", "svdq_attn.hip", "svdq_capi.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed FP32 instructions (v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32) anywhere.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE float32 division where the source writes '/', as the bit-exact paths require.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    root = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(root) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    cc = hipcc()
    LIB_DIR.mkdir(exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="svdq_build_") as tmp:
        objs = []
        cmds = []
        for src in SOURCES:
            obj = Path(tmp) / (Path(src).stem + ".o")
            objs.append(str(obj))
            cmds.append([cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
                if verbose:
                    print(" ".join(cmd))
                fut.result()
        tmp_lib = LIB_DIR / (LIB_PATH.name + ".tmp")
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp_lib)])
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
