"""Checks on the gfx950 machine code of the built library.

`scalar_writes` finds writes through the scalar data cache, which the
library must not contain.  `exec_zero_writes` finds vector instructions
placed where the exec mask is zero.  A loop that lanes leave after different trip counts ends with
`s_cbranch_execnz` falling through once exec is zero, into a block that then
restores exec; an instruction the compiler places in that block before the
restore writes no lane.  ROCm 7.2's compiler has placed the copy of a
loop-carried value there (a register copy of a running maximum, so every lane
kept the value it had before the loop); the step kernel avoids the pattern,
and hipbuild runs this check after every build so that a regression fails
the build instead of silently corrupting results.
"""

from __future__ import annotations

import re
import shutil
import subprocess
import tempfile
from pathlib import Path

LLVM_BIN = Path("/opt/rocm/llvm/bin")
# Vector and memory instructions that depend on exec; v_writelane,
# v_readlane and v_readfirstlane address one lane explicitly and ignore it.
_VECTOR = ("v_", "ds_", "buffer_", "global_", "flat_", "scratch_")
_EXEMPT = ("v_writelane", "v_readlane", "v_readfirstlane")


def disassemble(library: Path, arch: str = "gfx950") -> str:
    """Disassembly of the `arch` code object embedded in a HIP shared library."""
    objdump = LLVM_BIN / "llvm-objdump"
    with tempfile.TemporaryDirectory() as tmp:
        copy = Path(tmp) / "lib.so"
        shutil.copy(library, copy)
        # --offloading writes each bundle next to its input
        subprocess.run([str(objdump), "--offloading", str(copy)], check=True,
                       capture_output=True)
        objects = [p for p in Path(tmp).iterdir() if p.name.endswith(arch)]
        if not objects:
            raise RuntimeError(f"{library}: no {arch} code object")
        return subprocess.run([str(objdump), "-d", f"--mcpu={arch}", str(objects[0])],
                              check=True, capture_output=True, text=True).stdout


_FUNCTION = re.compile(r"^([0-9a-f]+) <([^>]+)>:")
_INSTRUCTION = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):")
_TARGET = re.compile(r"<([^>+]+)\+0x([0-9a-f]+)>")


def _offset(pc, n, word, operand):
    """Record a literal half of the offset added to the address that
    s_getpc_b64 left in s[n:n+1]; an added register makes the address
    unknown, so the pair is no longer followed (a jump through it then adds
    no target, which can only report more, never less)."""
    try:
        pc[n][word] = int(operand, 0) & 0xFFFFFFFF
    except ValueError:
        pc.pop(n)


def exec_zero_writes(text: str):
    """(function, address, instruction) of every vector or memory instruction
    reached only by falling through `s_cbranch_execnz` (exec is zero there)
    before exec is written again."""
    functions, rows = {}, []
    current = None
    for line in text.splitlines():
        m = _FUNCTION.match(line)
        if m:
            current = m.group(2)
            functions[current] = int(m.group(1), 16)
            continue
        m = _INSTRUCTION.match(line)
        if m and current:
            rows.append((current, int(m.group(3), 16), m.group(1), m.group(2), line))
    targets = set()
    # far jumps: s_getpc_b64 s[n:n+1] (the address of the next instruction),
    # s_add_u32 sn, sn, lo; s_addc_u32 sn+1, sn+1, hi; s_setpc_b64
    pc = {}
    for _, address, op, args, line in rows:
        if op.startswith(("s_branch", "s_cbranch")):
            t = _TARGET.search(line)
            if t and t.group(1) in functions:
                targets.add(functions[t.group(1)] + int(t.group(2), 16))
        regs = [a.strip() for a in args.split(",")]
        if op == "s_getpc_b64":
            n = int(re.match(r"s\[(\d+):", regs[0]).group(1))
            pc[n] = [address + 4, 0, 0]
        elif op in ("s_add_u32", "s_addc_u32") and len(regs) == 3 and regs[0] == regs[1]:
            # only an SGPR destination sn can be half of an s_getpc pair
            # (vcc_lo, ttmp or m0 destinations are skipped)
            sgpr = re.fullmatch(r"s(\d+)", regs[0])
            if sgpr:
                n = int(sgpr.group(1))
                if op == "s_add_u32" and n in pc:
                    _offset(pc, n, 1, regs[2])
                elif op == "s_addc_u32" and n - 1 in pc:
                    _offset(pc, n - 1, 2, regs[2])
        elif op == "s_setpc_b64":
            n = int(re.match(r"s\[(\d+):", regs[0]).group(1))
            if n in pc:
                base, lo, hi = pc.pop(n)
                offset = (hi << 32) | lo
                if offset >= 1 << 63:
                    offset -= 1 << 64
                targets.add(base + offset)
    found, zero = [], False
    for function, address, op, args, _ in rows:
        if address in targets:
            zero = False  # another path enters here
        if zero:
            first = args.split(",")[0].strip() if args else ""
            if op.startswith("s_") and (first == "exec" or "saveexec" in op):
                zero = False
            elif op.startswith(_VECTOR) and not op.startswith(_EXEMPT):
                found.append((function, address, f"{op} {args}".strip()))
        if op == "s_cbranch_execnz":
            zero = True
        elif op.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            zero = False
    return found


# Writes through the scalar data cache (scalar memory stores and atomics, its
# write-back and discard): the library must contain none.
_SCALAR_WRITES = re.compile(r"^\s+(s_store_\w+|s_buffer_store_\w+|s_scratch_store_\w+|"
                            r"s_atomic_\w+|s_buffer_atomic_\w+|s_dcache_wb\w*|"
                            r"s_dcache_discard\w*)\b", re.M)


def scalar_writes(text: str):
    """Every scalar-cache write instruction in a disassembly listing."""
    return [m.group(1) for m in _SCALAR_WRITES.finditer(text)]


def check(library: Path, arch: str = "gfx950") -> None:
    """Raise if the library's code writes vector registers with exec zero, or
    writes through the scalar data cache."""
    text = disassemble(library, arch)
    scalar = scalar_writes(text)
    if scalar:
        raise RuntimeError(f"{library}: {len(scalar)} scalar-cache write instruction(s): "
                           f"{sorted(set(scalar))}")
    found = exec_zero_writes(text)
    if found:
        lines = "\n".join(f"  {f} +{a:#x}: {i}" for f, a, i in found[:20])
        raise RuntimeError(f"{library}: {len(found)} vector instruction(s) placed where exec "
                           f"is zero (after a divergent loop exit, before exec is restored):\n"
                           f"{lines}")
