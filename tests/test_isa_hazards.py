"""Wait states around the inline-assembly DPP multiply-adds of the Mamba-1 lane backward.

`fmac_row` in csrc/selscan.hip issues `v_fmac_f32_dpp` (a row broadcast as the DPP source)
from inline assembly, because the compiler folds DPP into multiplies but not into fmac.  The
hardware needs two wait states between a vector write of a register and a DPP read of it, and
the compiler inserts none for inline assembly: the code is correct only while every such
instruction's DPP source was written at least two instructions earlier (or the instruction
carries its own `s_nop 1`).  This test disassembles the gfx950 code object of the selscan.o
that `build()` produced (this build's own code) and checks every one of them, so a compiler
that schedules differently fails here on the CPU instead of giving wrong gradients on a GPU.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OBJ = os.path.join(ROOT, "metal-kernelops_amd", "_build", "selscan.o")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

INSN = re.compile(r"^\s+([a-z_0-9]+)(.*?)\s*//\s*([0-9A-F]+):")
FUNC = re.compile(r"^([0-9a-f]+) <([^>]+)>:")
TARGET = re.compile(r"<([^>+]+)\+0x([0-9a-f]+)>")


def _disassemble(tmp_path):
    if not os.path.exists(OBJ):
        pytest.skip("selscan.o not built (run __graft_entry__.build() first)")
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not available")
    obj = tmp_path / "selscan.o"
    shutil.copy(OBJ, obj)
    subprocess.run([OBJDUMP, "--offloading", str(obj)], check=True, capture_output=True, cwd=tmp_path)
    dev = [p for p in tmp_path.iterdir() if "amdgcn" in p.name and "gfx950" in p.name]
    assert dev, "no gfx950 code object in selscan.o"
    out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(dev[0])], check=True, capture_output=True, text=True)
    return out.stdout.splitlines()


def _written(mnemonic, operands):
    """Vector registers an instruction writes (its first operand, for vector ALU ops)."""
    if not mnemonic.startswith("v_") or mnemonic.startswith(("v_cmp", "v_readlane", "v_readfirstlane")):
        return set()
    dst = operands.split(",")[0].strip()
    m = re.fullmatch(r"v(\d+)", dst)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", dst)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _problems(lines):
    """(number of v_fmac_f32_dpp checked, the ones whose DPP source may not have settled)."""
    funcs, insns = {}, []
    for line in lines:
        m = FUNC.match(line)
        if m:
            funcs[m.group(2)] = int(m.group(1), 16)
            continue
        m = INSN.match(line)
        if m:
            insns.append((int(m.group(3), 16), m.group(1), m.group(2), line))
    targets = set()
    for _, mn, _, line in insns:
        if mn.startswith(("s_branch", "s_cbranch")):
            t = TARGET.search(line)
            if t and t.group(1) in funcs:
                targets.add(funcs[t.group(1)] + int(t.group(2), 16))
    checked, problems = 0, []
    for i, (addr, mn, ops, line) in enumerate(insns):
        if mn != "v_fmac_f32_dpp":
            continue
        checked += 1
        src = int(re.match(r"\s*v\d+,\s*v(\d+),", ops).group(1))
        if addr in targets:
            problems.append(f"branch target at {line.strip()}")
            continue
        waits, j = 0, i - 1
        while waits < 2 and j >= 0:
            a, m2, o2, l2 = insns[j]
            if src in _written(m2, o2):
                problems.append(f"v{src} written {waits} wait states before: {l2.strip()} -> {line.strip()}")
                break
            waits += int(o2.split()[0]) + 1 if m2 == "s_nop" else 1
            if waits < 2 and a in targets:
                problems.append(f"branch target inside the window: {l2.strip()} -> {line.strip()}")
                break
            j -= 1
    return checked, problems


def _listing(body):
    out = ["0000000000001000 <k>:"]
    for n, text in enumerate(body):
        out.append(f"\t{text:58s} // {0x1000 + 4 * n:012X}: 00000000")
    return out


def test_checker_finds_an_unsettled_source():
    """The check itself: a source written one instruction before the DPP read is reported, the
    same source behind s_nop 1 or two other instructions is not, and a branch landing between
    the write and the read makes the read unverifiable."""
    fmac = "v_fmac_f32_dpp v10, v4, v5 row_newbcast:3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
    bad = _listing(["v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", fmac])
    nop = _listing(["v_mul_f32_e32 v4, v1, v2", "s_nop 1", fmac])
    far = _listing(["v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", "v_add_f32_e32 v8, v1, v2", fmac])
    jump = _listing(["s_branch 1 <k+0xc>", "v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", fmac])
    assert _problems(bad)[1] and not _problems(nop)[1] and not _problems(far)[1]
    assert _problems(jump)[1] and _problems(far)[0] == 1


def test_dpp_fmac_sources_are_settled(tmp_path):
    checked, problems = _problems(_disassemble(tmp_path))
    assert checked > 0, "no v_fmac_f32_dpp found: fmac_row is no longer used, drop this test"
    assert not problems, "\n".join(problems[:10])
