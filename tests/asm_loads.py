"""Static check of the asynchronous register loads in gfx950 assembly.

The fused kernels issue some buffer loads as inline asm, so the compiler
does not know that their destination VGPRs are written long after the
instruction issues.  The kernels wait with an explicit s_waitcnt vmcnt(N)
before any use; this module checks that the compiler kept its side of the
bargain: on every control-flow path from such a load to the wait that
retires it (vmcnt(N) with N <= loads issued since), no instruction reads or
writes one of the destination VGPRs (no copy, spill or reuse of a register
that is still being filled).
"""

from __future__ import annotations

import re

_VMEM = re.compile(r"^(buffer_load|buffer_store|global_load|global_store|buffer_atomic|global_atomic|flat_load|flat_store)")
_ASM_LOAD = re.compile(r"^\s*buffer_load_dwordx4 v\[(\d+):(\d+)\], v\d+, s\[\d+:\d+\], 0 offen$")


def _vgprs(text: str) -> set[int]:
    out: set[int] = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def kernels(asm: str) -> dict[str, list[str]]:
    """Kernel symbol -> instruction lines (comments stripped)."""
    parts = re.split(r"\n(?=_Z\S+:\s)", asm)
    return {p.split(":")[0]: [ln.split(";")[0].rstrip() for ln in p.split("\n")] for p in parts[1:]}


def check_kernel(lines: list[str]) -> tuple[int, list[str]]:
    """(number of asm loads, violations) for one kernel's lines."""
    labels = {m.group(1): i for i, ln in enumerate(lines) if (m := re.match(r"^(\.LBB\w+):", ln))}
    loads, bad = 0, []
    for i, ln in enumerate(lines):
        m = _ASM_LOAD.match(ln)
        if not m:
            continue
        loads += 1
        dst = set(range(int(m.group(1)), int(m.group(2)) + 1))
        seen: set[tuple[int, int]] = set()
        stack = [(i + 1, 0)]
        while stack:
            j, younger = stack.pop()
            while j < len(lines):
                if (j, younger) in seen:
                    break
                seen.add((j, younger))
                ins = lines[j].strip()
                w = re.search(r"vmcnt\((\d+)\)", ins)
                if ins.startswith("s_waitcnt") and w and int(w.group(1)) <= younger:
                    break
                if _VMEM.match(ins):
                    younger = min(younger + 1, 63)
                if ins.startswith("s_endpgm"):
                    bad.append(f"load at line {i} ({ln.strip()}) reaches s_endpgm without a wait")
                    break
                if ins and not ins.startswith(("s_", ".")) and _vgprs(ins) & dst:
                    bad.append(f"load at line {i} ({ln.strip()}) touched at line {j}: {ins}")
                    break
                b = re.match(r"^s_(c?branch\w*)\s+(\.LBB\w+)", ins)
                if b:
                    stack.append((labels[b.group(2)], younger))
                    if b.group(1) == "branch":
                        break
                j += 1
    return loads, bad
