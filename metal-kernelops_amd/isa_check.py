"""Checks of the built device code: the wait states of the Mamba-1 backward's inline-assembly
DPP multiply-adds, and the one rounding convention for float16 results.

``fmac_row`` in csrc/selscan.hip issues ``v_fmac_f32_dpp`` (a row broadcast as the DPP
source) from inline assembly, because the compiler folds DPP into multiplies but not into
fmac.  The compiler inserts no hazard waits for inline assembly, so the code is correct only
while the schedule around each such instruction already meets the two DPP rules of
gfx9-family parts (the ones LLVM's hazard recognizer enforces for compiled DPP):

* two wait states between any write of a VGPR and a DPP instruction that reads it (for
  ``v_fmac_f32_dpp`` that is the DPP source, the multiplier and the tied accumulator);
* five wait states between a vector instruction that writes EXEC (``v_cmpx_*``) and a DPP
  instruction.

``check_object`` disassembles the gfx950 code object of an object file that this build
produced (``_build/selscan.o``, whose device code is what ``libmko.so`` carries) with ROCm's
``llvm-objdump`` and checks every ``v_fmac_f32_dpp`` in it.  ``build.py`` runs it after
compiling and fails the build on a problem; ``tests/test_isa_hazards.py`` checks the checker.

``check_f16_rounding`` fails an object that holds a mixed-precision multiply-add with a
float16 result (``v_fma_mixlo_f16`` / ``v_fma_mixhi_f16``, and the ``v_mad_mix`` forms).  Such an
instruction rounds an exact product once to float16, where the kernels' convention (every
float16 value is an fp32 value rounded to float16, ``from_f32`` and ``pack2`` in
csrc/common.hpp) rounds twice; the SSD backward's cancelling row and column sums need every
kernel to round the same products the same way.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
DPP_VGPR_WAITS = 2
DPP_EXEC_WAITS = 5

INSN = re.compile(r"^\s+([a-z_0-9]+)(.*?)\s*//\s*([0-9A-F]+):")
FUNC = re.compile(r"^([0-9a-f]+) <([^>]+)>:")
TARGET = re.compile(r"<([^>+]+)\+0x([0-9a-f]+)>")
VREG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")

# loads whose first operand is the destination
_LOADS = ("ds_read", "ds_load", "global_load", "buffer_load", "flat_load", "scratch_load")
# vector instructions whose first operand is a scalar destination, not a VGPR
_SCALAR_DST = ("v_cmp", "v_readlane", "v_readfirstlane")
# vector instructions that write their first two operands
_TWO_DST = ("v_permlane16_swap", "v_permlane32_swap", "v_swap_b32")


def _regs(operand):
    """The VGPR numbers an operand names (v7 or v[4:5]; anything else names none)."""
    m = VREG.match(operand.strip())
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def _operands(text):
    return [o.strip() for o in text.split(",")] if text.strip() else []


def written(mnemonic, operands):
    """VGPRs an instruction writes."""
    ops = _operands(operands)
    if not ops:
        return set()
    if mnemonic.startswith(_TWO_DST):
        return _regs(ops[0]) | (_regs(ops[1]) if len(ops) > 1 else set())
    if mnemonic.startswith(_LOADS):
        return _regs(ops[0])
    if mnemonic.startswith("v_") and not mnemonic.startswith(_SCALAR_DST):
        return _regs(ops[0].split()[0])
    return set()


def writes_exec(mnemonic):
    return mnemonic.startswith("v_cmpx")


def _wait_states(mnemonic, operands):
    return int(operands.split()[0]) + 1 if mnemonic == "s_nop" else 1


def problems(lines):
    """(number of v_fmac_f32_dpp checked, descriptions of the ones whose inputs may not have
    settled) for a disassembly listing."""
    funcs, insns = {}, []
    for line in lines:
        m = FUNC.match(line)
        if m:
            funcs[m.group(2)] = int(m.group(1), 16)
            continue
        m = INSN.match(line)
        if m:
            insns.append((int(m.group(3), 16), m.group(1), m.group(2), line))
    targets = {}  # branch target address -> indices of the branches that jump there
    for k, (_, mn, _, line) in enumerate(insns):
        if mn.startswith(("s_branch", "s_cbranch")):
            t = TARGET.search(line)
            if t and t.group(1) in funcs:
                targets.setdefault(funcs[t.group(1)] + int(t.group(2), 16), []).append(k)

    def exec_written_before(k, budget):
        # a v_cmpx within `budget` wait states up to and including instruction k, on the
        # straight-line path into it (None when another branch target makes it unverifiable)
        waits = 0
        while waits < budget and k >= 0:
            a, m2, o2, l2 = insns[k]
            if writes_exec(m2):
                return l2.strip()
            waits += _wait_states(m2, o2)
            if waits < budget and a in targets:
                return None
            k -= 1
        return ""

    checked, found = 0, []
    for i, (addr, mn, ops, line) in enumerate(insns):
        if mn != "v_fmac_f32_dpp":
            continue
        checked += 1
        reads = set()
        for o in _operands(ops)[:3]:  # accumulator (tied), DPP source, multiplier
            reads |= _regs(o.split()[0])
        if addr in targets:
            found.append(f"branch target at {line.strip()}")
            continue
        waits, j = 0, i - 1
        while waits < DPP_EXEC_WAITS and j >= 0:
            a, m2, o2, l2 = insns[j]
            if waits < DPP_VGPR_WAITS:
                hit = reads & written(m2, o2)
                if hit:
                    found.append(f"v{min(hit)} written {waits} wait states before: {l2.strip()} -> {line.strip()}")
                    break
            if writes_exec(m2):
                found.append(f"EXEC written {waits} wait states before: {l2.strip()} -> {line.strip()}")
                break
            waits += _wait_states(m2, o2)
            if waits < DPP_EXEC_WAITS and a in targets:
                if waits < DPP_VGPR_WAITS:
                    found.append(f"branch target inside the window: {l2.strip()} -> {line.strip()}")
                    break
                # another path joins here with the VGPRs settled: only a v_cmpx at the end of
                # a path that jumps here could still be inside the EXEC window
                for k in targets[a]:
                    w = exec_written_before(k, DPP_EXEC_WAITS - waits)
                    if w is None or w:
                        found.append(f"EXEC may be written {waits}+ wait states before, on a path "
                                     f"into {l2.strip()}: {w or 'unverifiable'} -> {line.strip()}")
                        break
            j -= 1
    return checked, found


def disassemble(obj, required=True):
    """The gfx950 disassembly of the device code object embedded in ``obj`` (no lines for an
    object without one, unless ``required``)."""
    if not os.path.exists(OBJDUMP):
        raise RuntimeError(f"{OBJDUMP} not found: the DPP wait states of {obj} cannot be checked")
    with tempfile.TemporaryDirectory() as tmp:
        local = os.path.join(tmp, os.path.basename(obj))
        shutil.copy(obj, local)
        subprocess.run([OBJDUMP, "--offloading", local], check=True, capture_output=True, cwd=tmp)
        dev = [p for p in os.listdir(tmp) if "amdgcn" in p and "gfx950" in p]
        if not dev:
            if not required:
                return []
            raise RuntimeError(f"no gfx950 code object in {obj}")
        out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(tmp, dev[0])], check=True,
                             capture_output=True, text=True)
    return out.stdout.splitlines()


def check_object(obj):
    """Raises RuntimeError when a v_fmac_f32_dpp in ``obj`` may read an unsettled input, or
    when ``obj`` has none (then fmac_row is gone and this check should go with it)."""
    checked, found = problems(disassemble(obj))
    if checked == 0:
        raise RuntimeError(f"no v_fmac_f32_dpp in {obj}: fmac_row is no longer used, drop this check")
    if found:
        raise RuntimeError(f"{len(found)} DPP hazard(s) in {obj}:\n" + "\n".join(found[:10]))
    return checked


MIX16 = re.compile(r"\sv_(?:fma|mad)_mix(?:lo|hi)_f16\b")


def f16_rounding_problems(lines):
    """The functions of a disassembly that hold a mixed-precision multiply-add with a float16
    result, with the count of such instructions in each."""
    found, func = {}, None
    for line in lines:
        m = FUNC.match(line)
        if m:
            func = m.group(2)
            continue
        if MIX16.search(line):
            found[func] = found.get(func, 0) + 1
    return found


def check_f16_rounding(obj):
    """Raises RuntimeError when ``obj`` rounds a product to float16 in one step."""
    found = f16_rounding_problems(disassemble(obj, required=False))
    if found:
        raise RuntimeError(f"float16 results of mixed-precision multiply-adds in {obj} (route the value "
                           "through from_f32 / pack2): " + ", ".join(f"{k} ({v})" for k, v in list(found.items())[:5]))
