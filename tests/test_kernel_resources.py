"""No kernel with asynchronous inline-asm loads into VGPRs may spill.

The W4A16 kernels issue their global loads as inline asm (`global_load_dwordx4 %0, ...`) so that
the compiler neither waits for them nor reorders them; the kernels wait with explicit
`s_waitcnt vmcnt(N)`.  The compiler takes such a load's destination as written when the asm
issues, so a spill or copy of that register placed before the wait saves whatever the register
held before the load lands (a build of the 256-row W4A16 tile with 117 spilled VGPRs returned NaN).
This test reads the kernel metadata of the library built in this repository (its code objects'
AMDGPU notes) and requires zero scratch and zero VGPR spills for every such kernel.
"""
import re
import subprocess
import tempfile

import pytest

from tests.test_dma_hazards import LIB, _gfx950_code_objects

READOBJ = "/opt/rocm/llvm/bin/llvm-readobj"
ASYNC_VGPR_LOAD_KERNELS = ("w4a16_kernel", "w4a16_wide_kernel", "w4a16_ws_kernel")


def _kernel_metadata() -> dict[str, dict[str, int]]:
    out = {}
    for code in _gfx950_code_objects(LIB):
        with tempfile.NamedTemporaryFile(suffix=".o") as f:
            f.write(code)
            f.flush()
            text = subprocess.run([READOBJ, "--notes", f.name], capture_output=True, text=True, check=True).stdout
        for block in re.split(r"\n\s*- \.agpr_count:", text)[1:]:
            name = re.search(r"\.name:\s+(\S+)", block)
            if not name:
                continue
            fields = {}
            for key in ("private_segment_fixed_size", "vgpr_spill_count", "vgpr_count"):
                m = re.search(rf"\.{key}:\s+(\d+)", block)
                if m:
                    fields[key] = int(m.group(1))
            out[name.group(1)] = fields
    return out


@pytest.mark.skipif(not LIB.exists(), reason="library not built")
def test_async_load_kernels_do_not_spill():
    meta = _kernel_metadata()
    checked = {k: v for k, v in meta.items() if any(s in k for s in ASYNC_VGPR_LOAD_KERNELS)}
    assert len(checked) >= 10, f"expected the W4A16 kernels in the metadata, found {sorted(meta)[:5]}..."
    bad = {k: v for k, v in checked.items()
           if v.get("private_segment_fixed_size", -1) != 0 or v.get("vgpr_spill_count", -1) != 0}
    assert not bad, f"kernels with in-flight asm loads spill: {bad}"


# Kernels on the denoise step's path (every group-64 activation pass, the grouped GEMM, the
# attention and the streaming passes around them): a spill there (a mis-sized register array, a
# loop the compiler could not keep in registers) costs more than it saves.
NO_SCRATCH_KERNELS = ("mid_finalize_kernel", "gate_op_kernel", "rms_norm_modulate_kernel", "head_rms_rope",
                      "attn_fast_kernel", "attn_combine_kernel", "act_kernelILi64E", "w4a4_e3m2_siblings_kernel",
                      "act_siblings_kernel", "act_shared_x_kernel", "mid_finalize_siblings_kernel")


@pytest.mark.skipif(not LIB.exists(), reason="library not built")
def test_streaming_kernels_use_no_scratch():
    meta = _kernel_metadata()
    checked = {k: v for k, v in meta.items() if any(s in k for s in NO_SCRATCH_KERNELS)}
    assert len(checked) >= 12, f"expected the kernels in the metadata, found {sorted(meta)[:5]}..."
    bad = {k: v for k, v in checked.items()
           if v.get("private_segment_fixed_size", -1) != 0 or v.get("vgpr_spill_count", -1) != 0}
    assert not bad, f"kernels with scratch or spills: {bad}"
