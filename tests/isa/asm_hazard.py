"""Static check of the decode GEMV's hand-placed waits (test infrastructure).

The DMA GEMV loads its activations with inline-asm global_load_dwordx4 and
waits for them with a later inline-asm s_waitcnt, so the weight copies
issued in between stay in flight. The compiler believes the asm outputs are
ready at once; if it ever reads, copies or overwrites one of those
registers before the wait, the kernel races with the load.

This scans the gfx950 assembly of every gemv_dma_kernel instance. Vector
memory instructions (loads, stores and LDS copies: each counts in vmcnt)
enter an in-order queue with their destination VGPRs; `s_waitcnt vmcnt(N)`
retires all but the N youngest. Any later instruction that names a VGPR of
a load still in the queue, as a source or a destination, is reported. Labels
and branches keep the queue (the state flows into the branch target), and
each backward branch rescans its loop body once more with the queue it
carries at the branch, so loads issued at the bottom of a loop are checked
against the top of the next iteration."""
from __future__ import annotations

import re

_VMEM = re.compile(r"^(global_load|global_store|buffer_load|buffer_store|flat_load|flat_store|global_atomic|"
                   r"buffer_atomic|flat_atomic|scratch_load|scratch_store)")
_LOAD = re.compile(r"^(global_load|buffer_load|flat_load|scratch_load)")
_BRANCH = re.compile(r"^s_(cbranch_\w+|branch)$")


def _regs(tok: str) -> set[int]:
    tok = tok.strip("|,")
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _vmcnt(line: str) -> int | None:
    m = re.search(r"vmcnt\((\d+)\)", line)
    return int(m.group(1)) if m else None


def _scan(lines, start, end, queue, name, found, seen):
    """Linear scan of lines[start:end] from an in-flight queue (a list of
    register sets, oldest first). Returns the queue at `end`, and the
    backward branches met as (target, branch index, queue there)."""
    back = []
    for i in range(start, end):
        line = lines[i]
        op = line.split()[0]
        if op.endswith(":"):
            continue
        operands = line.split(None, 1)[1].split(",") if " " in line else []
        named = set().union(*(_regs(t.strip().split()[0]) for t in operands if t.strip())) if operands else set()
        if op == "s_waitcnt":
            n = _vmcnt(line)
            if n is not None:
                queue = queue[len(queue) - n:] if n < len(queue) else queue
                queue = [] if n == 0 else queue
            continue
        pending = set().union(*queue) if queue else set()
        if _VMEM.match(op):
            # LDS copies (global_load_lds_*, or a buffer load with the lds
            # modifier) write no VGPR
            to_lds = "_lds" in op or "lds" in line.split()[1:]
            dest = _regs(operands[0].strip()) if _LOAD.match(op) and not to_lds else set()
            srcs = named - dest if dest else named
            if (srcs | dest) & pending:
                key = (name, i)
                if key not in seen:
                    seen.add(key)
                    found.append(f"{name}: {line}")
            queue = queue + [dest]
            continue
        if named & pending:
            key = (name, i)
            if key not in seen:
                seen.add(key)
                found.append(f"{name}: {line}")
        if _BRANCH.match(op) and operands:
            back.append((operands[0].strip(), i, list(queue)))
    return queue, back


def hazards(asm: str, kernel_prefix: str = "_ZN3nuq15gemv_dma_kernel") -> tuple[int, list[str]]:
    kernels = re.findall(r"^(" + kernel_prefix + r"\S+):\s*;.*?\n(.*?)^\.Lfunc_end", asm, re.S | re.M)
    found: list[str] = []
    for name, body in kernels:
        lines = [l.split(";")[0].strip() for l in body.split("\n")]
        lines = [l for l in lines if l and (not l.startswith(".") or l.endswith(":"))]
        labels = {l[:-1]: i for i, l in enumerate(lines) if l.endswith(":")}
        seen: set = set()
        _, branches = _scan(lines, 0, len(lines), [], name, found, seen)
        for target, at, queue in branches:
            t = labels.get(target)
            if t is not None and t <= at:  # a loop: its top runs again with this queue
                _scan(lines, t, at + 1, queue, name, found, seen)
    return len(kernels), found
