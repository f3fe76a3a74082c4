"""Instruction-order rules of the fast attention kernel, checked on the built library.

`attn_fast_kernel` (csrc/svdq_attn.hip) issues its MFMAs as inline asm and interleaves softmax
VALU work between them, so the compiler's hazard recognizer does not guard the MFMA operands.
The kernel's source keeps two rules, which this test checks in the gfx950 disassembly of our own
build (llvm-objdump), in instruction order:

* no VALU instruction between two consecutive MFMAs that read the same A operand (an earlier
  layout that put softmax work there gave wrong results for the second MFMA of every pair; the
  cause was not found -- the same sequence in a standalone probe is exact -- so the kernel keeps
  to the layouts that test exact);
* no instruction writes an MFMA's A or B source registers (VALU, LDS or global load destination)
  until two more MFMAs have issued or 32 wait states of `s_nop` have passed (the kernel holds each
  fragment two MFMAs past its last use and ends each phase with a 32-wait-state fence);
* no VALU instruction writes a source register of an MFMA (A, B or C, VGPR or AGPR) fewer than 2
  wait states before it: the CDNA3 ISA's required independent instructions between a VALU write
  of a VGPR and an MFMA read of it (LLVM's hazard recognizer inserts them for the MFMAs it sees,
  not for inline asm).  The compiler writes the output accumulators back to AGPRs with
  v_accvgpr_write after the softmax rescale and may place the last write right before the next
  output MFMA; an earlier layout that put softmax work between the two MFMAs of a fragment had
  such writes 0 and 1 wait states before the second MFMA of a pair, whose results were wrong.

Planted listings with violations of each kind must be caught.
"""
import re
from pathlib import Path

import pytest

from tests.test_dma_hazards import LIB, OBJDUMP, _disassemble, _functions, _gfx950_code_objects

KERNEL = "_ZN4svdq12_GLOBAL__N_116attn_fast_kernelENS0_8AttnArgsE"
HOLD_MFMAS = 2
HOLD_WAITS = 32
VALU_TO_MFMA_WAITS = 2


def _vregs(tok: str) -> set:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _operands(text: str) -> list[str]:
    return [a.strip() for a in text.split(None, 1)[1].split(",")] if " " in text else []


def _writes_vgprs(op: str) -> bool:
    if op.startswith("v_"):
        return not op.startswith(("v_cmp", "v_readfirstlane", "v_readlane", "v_mfma", "v_accvgpr_write"))
    return op.startswith(("ds_read", "global_load_dword", "buffer_load", "flat_load"))


def _regs(tok: str) -> set:
    """VGPRs and AGPRs of an operand, as ("v", n) / ("a", n)."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def valu_to_mfma_violations(func: dict) -> list[str]:
    """VALU writes of an MFMA source register (A, B or C) fewer than VALU_TO_MFMA_WAITS wait states
    before the MFMA (every instruction in between is one wait state, `s_nop n` n + 1)."""
    ins = [text for _, text, _ in func["ins"]]
    bad = []
    for i, text in enumerate(ins):
        if not text.startswith("v_mfma"):
            continue
        srcs = set().union(*(_regs(a) for a in _operands(text)[1:4]))
        waits = 0
        for j in range(i - 1, -1, -1):
            if waits >= VALU_TO_MFMA_WAITS:
                break
            prev = ins[j]
            op = prev.split()[0]
            if op == "s_nop":
                waits += int(prev.split()[1], 0) + 1
                continue
            if op.startswith("v_") and not op.startswith(("v_mfma", "v_cmp", "v_readfirstlane", "v_readlane")):
                args = _operands(prev)
                if args and _regs(args[0]) & srcs:
                    bad.append(f"{prev!r} writes a source of {text!r} {waits} wait states before it")
            waits += 1
    return bad


def order_violations(func: dict) -> tuple[int, list[str]]:
    """(number of MFMAs, descriptions of the violations) of one function, in instruction order."""
    mfmas, bad = 0, []
    pending = []        # [A|B registers, MFMAs since, wait states since, text]
    last_a, valu_since = None, False
    for _, text, _ in func["ins"]:
        op = text.split()[0]
        if op.startswith("v_mfma"):
            mfmas += 1
            args = _operands(text)
            a = _vregs(args[1])
            if last_a is not None and a == last_a and valu_since:
                bad.append(f"VALU work between two MFMAs reading {args[1]}: {text!r}")
            for p in pending:
                p[1] += 1
            pending = [p for p in pending if p[1] < HOLD_MFMAS and p[2] < HOLD_WAITS]
            pending.append([a | _vregs(args[2]), 0, 0, text])
            last_a, valu_since = a, False
            continue
        if op == "s_nop":
            w = int(text.split()[1], 0) + 1
            for p in pending:
                p[2] += w
            pending = [p for p in pending if p[2] < HOLD_WAITS]
            continue
        if op.startswith("v_"):
            valu_since = True
        if _writes_vgprs(op):
            args = _operands(text)
            dst = _vregs(args[0]) if args else set()
            for p in pending:
                if dst & p[0]:
                    bad.append(f"{text!r} writes a source of {p[3]!r} {p[1]} MFMAs / {p[2]} wait states later")
    return mfmas, bad + valu_to_mfma_violations(func)


PLANTED = """0000000000001000 <k>:
\tds_read_b128 v[10:13], v1 // 000000001000: 0
\tv_mfma_f32_32x32x16_bf16 v[20:35], v[10:13], v[40:43], 0 // 000000001004: 0
\tv_cvt_pk_bf16_f32 v50, v0, v1 // 00000000100C: 0
\tv_mfma_f32_32x32x16_bf16 v[60:75], v[10:13], v[44:47], 0 // 000000001010: 0
\tv_exp_f32_e32 v12, v2 // 000000001018: 0
\tv_mfma_f32_32x32x16_bf16 v[20:35], v[14:17], v[40:43], v[20:35] // 00000000101C: 0
\tv_mfma_f32_32x32x16_bf16 v[60:75], v[14:17], v[44:47], v[60:75] // 000000001024: 0
\tv_mfma_f32_32x32x16_bf16 v[20:35], v[80:83], v[40:43], v[20:35] // 00000000102C: 0
\tds_read_b128 v[14:17], v1 offset:64 // 000000001034: 0
\ts_nop 15 // 000000001038: 0
\ts_nop 15 // 00000000103C: 0
\tv_mov_b32_e32 v80, 0 // 000000001040: 0
\ts_endpgm // 000000001044: 0
"""


def test_order_check_catches_planted_violations():
    (func,) = _functions(PLANTED.splitlines())
    mfmas, bad = order_violations(func)
    assert mfmas == 5
    # the cvt between the two MFMAs that read v[10:13]; the exp writing v12 right after both of its
    # readers; v[14:17] (last read by the 4th MFMA) rewritten after only one more MFMA; v80
    # rewritten after 32 wait states is clean
    assert len(bad) == 4, bad
    assert "VALU work between two MFMAs reading v[10:13]" in bad[0]
    assert "v_exp_f32_e32 v12" in bad[1] and "v[10:13], v[40:43]" in bad[1]
    assert "v_exp_f32_e32 v12" in bad[2] and "v[10:13], v[44:47]" in bad[2]
    assert "ds_read_b128 v[14:17]" in bad[3] and "v[14:17], v[44:47]" in bad[3]


PLANTED_RAW = """0000000000002000 <k2>:
\tv_accvgpr_write_b32 a15, v3 // 000000002000: 0
\tv_mfma_f32_32x32x16_bf16 a[0:15], v[10:13], v[40:43], a[0:15] // 000000002004: 0
\tv_accvgpr_write_b32 a31, v4 // 00000000200C: 0
\ts_waitcnt lgkmcnt(0) // 000000002010: 0
\tv_mfma_f32_32x32x16_bf16 a[16:31], v[14:17], v[44:47], a[16:31] // 000000002014: 0
\tv_cvt_pk_bf16_f32 v50, v0, v1 // 00000000201C: 0
\ts_nop 1 // 000000002020: 0
\tv_mfma_f32_32x32x16_bf16 v[60:75], v[20:23], v[48:51], 0 // 000000002024: 0
\tv_mov_b32_e32 v52, v0 // 00000000202C: 0
\ts_nop 0 // 000000002030: 0
\tv_add_f32_e32 v5, v6, v7 // 000000002034: 0
\tv_mfma_f32_32x32x16_bf16 v[76:91], v[24:27], v[52:55], 0 // 000000002038: 0
\tv_mov_b32_e32 v56, v0 // 000000002040: 0
\ts_nop 0 // 000000002044: 0
\tv_mfma_f32_32x32x16_bf16 v[92:107], v[28:31], v[56:59], 0 // 000000002048: 0
\ts_endpgm // 000000002050: 0
"""


def test_valu_to_mfma_check_catches_planted_violations():
    (func,) = _functions(PLANTED_RAW.splitlines())
    bad = valu_to_mfma_violations(func)
    # a15 0 wait states before its MFMA, a31 1 (the s_waitcnt); v52 written 2 wait states before
    # its reader is clean; v56 1 wait state (one s_nop 0) before its reader
    assert len(bad) == 3, bad
    assert "a15" in bad[0] and "0 wait states" in bad[0]
    assert "a31" in bad[1] and "1 wait states" in bad[1]
    assert "v56" in bad[2] and "1 wait states" in bad[2]
    mfmas, all_bad = order_violations(func)
    assert mfmas == 5 and all_bad == bad


@pytest.mark.skipif(not LIB.exists() or not OBJDUMP.exists(),
                    reason="needs the built library and ROCm's llvm-objdump")
def test_fast_attention_kernel_keeps_its_mfma_order_rules():
    found, mfmas, bad = False, 0, []
    for code in _gfx950_code_objects(LIB):
        for func in _functions(_disassemble(code)):
            if func["name"] != KERNEL:
                continue
            found = True
            n, b = order_violations(func)
            mfmas += n
            bad += b
    assert found, f"{KERNEL} not in the library"
    assert mfmas >= 64, "the fast attention kernel's MFMAs were not found"
    assert not bad, f"{len(bad)} violations, e.g. {bad[:3]}"
