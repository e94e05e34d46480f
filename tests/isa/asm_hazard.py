"""Static check of the decode GEMV's hand-placed waits (test infrastructure).

The DMA GEMV loads its activations with inline-asm global_load_dwordx4 and
waits for them with a later inline-asm s_waitcnt, so the weight copies
issued in between stay in flight. The compiler believes the asm outputs are
ready at once; if it ever copies or reads one of those registers before the
wait, the kernel reads stale data (a race). This scans the gfx950 assembly
of every gemv_dma_kernel instance for a read of an in-flight load's
destination register before the next vmcnt wait."""
from __future__ import annotations

import re


def _regs(tok: str) -> set[int]:
    tok = tok.strip("|,")
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def hazards(asm: str, kernel_prefix: str = "_ZN3nuq15gemv_dma_kernel") -> tuple[int, list[str]]:
    kernels = re.findall(r"^(" + kernel_prefix + r"\S+):\s*;.*?\n(.*?)^\.Lfunc_end", asm, re.S | re.M)
    found = []
    for name, body in kernels:
        pending: set[int] = set()
        for line in (l.strip() for l in body.split("\n")):
            if not line or line.startswith(";"):
                continue
            op = line.split()[0]
            if op == "global_load_dwordx4":
                pending |= _regs(line.split()[1])
                continue
            if op == "s_waitcnt" and "vmcnt" in line:
                pending = set()
                continue
            if not pending:
                continue
            operands = [t for t in line.split()[1:]]
            sources = operands[1:] if op.startswith("v_") else operands
            used = set().union(*(_regs(t) for t in sources)) if sources else set()
            if used & pending:
                found.append(f"{name}: {line}")
                pending -= used
    return len(kernels), found
