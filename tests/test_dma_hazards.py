"""No global->LDS DMA of the built library can read an SGPR or M0 that was written too recently.

The GEMMs issue their global->LDS DMA (`global_load_lds_dword[x4]`) as inline asm, whose operands
the compiler's hazard recognizer does not see.  Two gfx9 rules apply to it:

* 5 wait states between a VALU instruction that writes an SGPR and a VMEM instruction that reads
  it.  Under SGPR pressure the compiler restores a spilled base pointer with `v_readlane` right
  before such a DMA, which then reads a stale address; builds in which that happened faulted the
  GPU.  Kernels whose builds do that start each DMA with `s_nop 4`.
* 1 wait state between an SALU instruction that writes M0 and an LDS DMA (which reads its LDS
  address from M0).  The compiler sets M0 with `s_mov_b32 m0, ...` right before the asm block;
  every DMA starts with at least `s_nop 0`.

This test disassembles the gfx950 code objects of the library built in this repository
(llvm-objdump on our own build) and walks back from every LDS DMA over every predecessor path
(fall-through and branches): within 5 wait states (`s_nop N` counts N + 1) no VALU instruction may
name one of the DMA's base SGPRs or M0, within 1 wait state no SALU instruction may write M0, and
no path may reach the start of the function.  Planted hazards of both kinds in a small
hand-written listing must be caught.
"""
import re
import struct
import subprocess
import tempfile
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parents[1] / "krea2-svdquant_amd" / "_lib" / "libsvdq_gfx950.so"
OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _gfx950_code_objects(lib: Path) -> list[bytes]:
    """The gfx950 entries of the clang offload bundles embedded in the library."""
    data = lib.read_bytes()
    out = []
    for m in re.finditer(re.escape(BUNDLE_MAGIC), data):
        base = m.start()
        (count,) = struct.unpack_from("<Q", data, base + len(BUNDLE_MAGIC))
        pos = base + len(BUNDLE_MAGIC) + 8
        for _ in range(count):
            off, size, idlen = struct.unpack_from("<QQQ", data, pos)
            pos += 24
            target = data[pos:pos + idlen].decode()
            pos += idlen
            if "gfx950" in target and size:
                out.append(data[base + off:base + off + size])
    return out


def _disassemble(code: bytes) -> list[str]:
    with tempfile.NamedTemporaryFile(suffix=".o") as f:
        f.write(code)
        f.flush()
        res = subprocess.run([str(OBJDUMP), "-d", "--mcpu=gfx950", f.name], capture_output=True, text=True,
                             check=True)
    return res.stdout.splitlines()


def _sregs(tok: str) -> set:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {f"s{r}" for r in range(int(m.group(1)), int(m.group(2)) + 1)}
    return {tok} if re.fullmatch(r"s\d+", tok) else set()


def _functions(lines: list[str]) -> list[dict]:
    """Functions of an llvm-objdump listing: start address and (address, text, line) per instruction."""
    funcs, cur = [], None
    for line in lines:
        m = re.match(r"^([0-9a-f]+) <(.+)>:$", line)
        if m:
            cur = {"name": m.group(2), "start": int(m.group(1), 16), "ins": []}
            funcs.append(cur)
            continue
        m = re.match(r"^\s+(.*?)\s*//\s*([0-9A-Fa-f]+):", line)
        if cur is not None and m:
            cur["ins"].append((int(m.group(2), 16), m.group(1).strip(), line))
    return funcs


def _writes_m0(text: str) -> bool:
    """An SALU instruction whose destination is M0 (s_mov_b32 m0, ...; s_add_u32 m0, ...)."""
    parts = text.replace(",", " ").split()
    return (parts[0].startswith("s_") and not parts[0].startswith(("s_nop", "s_waitcnt", "s_barrier"))
            and len(parts) > 1 and parts[1] == "m0")


def dma_hazards(func: dict) -> tuple[int, list[str]]:
    """(number of LDS DMAs, descriptions of the hazardous ones) of one function."""
    ins = func["ins"]
    index = {a: i for i, (a, _, _) in enumerate(ins)}
    preds = {i: [] for i in range(len(ins))}
    for i, (_, text, line) in enumerate(ins):
        op = text.split()[0]
        if op.startswith(("s_branch", "s_cbranch")):
            m = re.search(r"<.+\+0x([0-9a-f]+)>", line)
            tgt = func["start"] + int(m.group(1), 16) if m else None
            if tgt in index:
                preds[index[tgt]].append(i)
        if i + 1 < len(ins) and op not in ("s_branch", "s_endpgm", "s_setpc_b64"):
            preds[i + 1].append(i)
    count, bad = 0, []
    for i, (_, text, _) in enumerate(ins):
        if not text.startswith("global_load_lds"):
            continue
        count += 1
        base = _sregs(text.split()[-1].rstrip(",")) | {"m0"}
        stack, seen, reason = [(p, 0) for p in preds[i]] or [(None, 0)], set(), None
        while stack and reason is None:
            j, waits = stack.pop()
            if j is None:
                reason = "the function start is within 5 wait states"
                break
            if (j, waits) in seen:
                continue
            seen.add((j, waits))
            t = ins[j][1]
            op = t.split()[0]
            if op == "s_nop":
                w = int(t.split()[1], 0) + 1
            else:
                w = 1
                if op.startswith("v_") and any(
                        (_sregs(x.rstrip(",")) | ({"m0"} if x.rstrip(",") == "m0" else set())) & base
                        for x in t.split()[1:]):
                    reason = f"{t!r} {waits} wait states before"
                    break
                if waits < 1 and _writes_m0(t):
                    reason = f"{t!r} (SALU write of M0) {waits} wait states before"
                    break
            if waits + w < 5:
                if not preds[j]:
                    reason = "the function start is within 5 wait states"
                    break
                stack.extend((q, waits + w) for q in preds[j])
        if reason:
            bad.append(f"{func['name']}: {text!r} after {reason}")
    return count, bad


PLANTED = """0000000000001000 <k>:
\ts_load_dwordx2 s[4:5], s[0:1], 0x0 // 000000001000: 0
\ts_cbranch_scc1 3 // 000000001008: 0 <k+0x18>
\tv_readlane_b32 s5, v1, 0 // 00000000100C: 0
\ts_mov_b32 m0, s8 // 000000001010: 0
\ts_nop 1 // 000000001014: 0
\tglobal_load_lds_dwordx4 v2, s[4:5] // 000000001018: 0
\ts_nop 4 // 00000000101C: 0
\tglobal_load_lds_dwordx4 v3, s[4:5] // 000000001020: 0
\ts_mov_b32 m0, s9 // 000000001024: 0
\tglobal_load_lds_dword v4, s[4:5] // 000000001028: 0
\ts_add_u32 m0, s9, 0x400 // 00000000102C: 0
\ts_nop 0 // 000000001030: 0
\tglobal_load_lds_dword v5, s[4:5] // 000000001034: 0
\ts_nop 3 // 000000001038: 0
\tv_readfirstlane_b32 m0, v6 // 00000000103C: 0
\ts_nop 3 // 000000001040: 0
\tglobal_load_lds_dword v7, s[4:5] // 000000001044: 0
\ts_endpgm // 000000001048: 0
"""


def test_hazard_walk_catches_planted_hazards():
    (func,) = _functions(PLANTED.splitlines())
    count, bad = dma_hazards(func)
    assert count == 5
    # v2: v_readlane wrote s5 three wait states earlier on the fall-through path; v3: 5 wait
    # states after it, clean; v4: the SALU write of M0 right before it; v5: one s_nop 0 after the
    # M0 write, clean; v7: a VALU write of M0 four wait states before
    assert len(bad) == 3, bad
    assert "v2, s[4:5]" in bad[0] and "v_readlane" in bad[0]
    assert "v4, s[4:5]" in bad[1] and "SALU write of M0" in bad[1]
    assert "v7, s[4:5]" in bad[2] and "v_readfirstlane_b32 m0" in bad[2]


@pytest.mark.skipif(not LIB.exists() or not OBJDUMP.exists(),
                    reason="needs the built library and ROCm's llvm-objdump")
def test_no_lds_dma_reads_a_recently_written_sgpr_or_m0():
    code_objects = _gfx950_code_objects(LIB)
    assert code_objects, "no gfx950 code object in the library"
    dma, bad = 0, []
    for code in code_objects:
        for func in _functions(_disassemble(code)):
            n, b = dma_hazards(func)
            dma += n
            bad += b
    assert dma > 0, "the GEMM kernels issue LDS DMA; none found in the disassembly"
    assert not bad, f"{len(bad)} hazardous LDS DMA, e.g. {bad[:3]}"
