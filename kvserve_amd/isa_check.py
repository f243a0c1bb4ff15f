"""Build-time check of the compiled gfx950 assembly: no spill store while EXEC is partial.

The register allocator of the ROCm 7.2 toolchain can place a VGPR spill store in the join block
of a divergent branch *before* the `s_or_b64 exec, exec, sN` that restores the full lane mask.
The store then writes only the lanes that took the branch; the lanes that did not keep whatever
the scratch slot held before, and the reload (under the full mask) hands those lanes stale
values. Where the spilled value feeds an address -- a row index of the output store, say -- the
kernel writes outside its buffers and the GPU faults. Two builds of the prefill kernel did so
(a spill of a row-index pair placed between the page-table load's `s_and_saveexec` and the
join's exec restore; the store of the output rows then faulted).

`check(asm)` finds, for every kernel of an assembly file, the scratch stores that may execute
with some lanes of a full wave disabled. (Reloads under a partial mask are emitted inside
divergent regions for uses in the same region: they refill exactly the lanes that read them.)
It is a forward dataflow over the kernel's
basic blocks: EXEC is full at entry; `s_and_saveexec_b64 sX, ...` and `s_mov_b64 sX, exec` make
sX a copy of a full mask; `s_or_b64 exec, exec, sX` and `s_mov_b64 exec, sX` restore it; any
other write of EXEC leaves it partial; joins take the weakest state. The kernels launch whole
waves, so a spill store at a point where EXEC is full writes every lane.
"""
from __future__ import annotations

import re

_LABEL = re.compile(r"^(\.LBB\d+_\d+):")
_FUNC = re.compile(r"^(_Z\w+):")
_SREG = re.compile(r"s\[(\d+):(\d+)\]|s(\d+)\b")


def _sregs(tok: str) -> set[int]:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _functions(asm: str):
    lines = asm.split("\n")
    i = 0
    while i < len(lines):
        m = _FUNC.match(lines[i])
        if m:
            j = i + 1
            while j < len(lines) and not lines[j].startswith(".Lfunc_end"):
                j += 1
            yield m.group(1), [(k + 1, lines[k]) for k in range(i + 1, j)]
            i = j
        i += 1


def _parse(body):
    """Basic blocks: list of (label, [(line, op, operands)]), in layout order."""
    blocks = [["<entry>", []]]
    for ln, raw in body:
        s = raw.split(";")[0].strip()
        if not s or s.startswith("."):
            m = _LABEL.match(s) if s else None
            if m:
                blocks.append([m.group(1), []])
            continue
        parts = s.split(None, 1)
        ops = [t.strip() for t in re.split(r",\s*", parts[1])] if len(parts) > 1 else []
        if ops:
            ops[-1] = ops[-1].split()[0]
        blocks[-1][1].append((ln, parts[0], ops))
        if parts[0].startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            blocks.append([None, []])  # instructions after a branch start a new block
    return [b for b in blocks if b[0] is not None or b[1]]


def _succ(blocks, idx, index_of):
    label, insts = blocks[idx]
    out = []
    last = insts[-1][1] if insts else ""
    if insts and last.startswith(("s_branch", "s_cbranch")):
        tgt = insts[-1][2][0] if insts[-1][2] else None
        if tgt in index_of:
            out.append(index_of[tgt])
        if last.startswith("s_branch"):
            return out
    if last.startswith(("s_endpgm", "s_setpc")):
        return out
    if idx + 1 < len(blocks):
        out.append(idx + 1)
    return out


def _transfer(state, op, ops, ln, hits, name, text):
    full, copies = state
    if op.startswith("scratch_store") and not full:
        hits.append(f"{name}: line {ln}: {text} runs with a partial EXEC mask")
    dst = ops[0] if ops else ""
    # EXEC writes
    if dst in ("exec", "exec_lo", "exec_hi"):
        src = ops[2] if op == "s_or_b64" and len(ops) > 2 and ops[1] == "exec" else (ops[1] if len(ops) > 1 else "")
        regs = frozenset(_sregs(src))
        if op in ("s_or_b64", "s_mov_b64") and regs and regs in copies:
            full = True
        elif op == "s_mov_b64" and src == "-1":
            full = True
        else:
            full = False
        return full, copies
    if op.endswith("saveexec_b64"):
        regs = frozenset(_sregs(dst))
        copies = {c for c in copies if not (c & regs)}
        if full:
            copies.add(regs)
        full = op.startswith("s_or_saveexec") and len(ops) > 1 and ops[1] == "-1"
        return full, copies
    if op == "s_mov_b64" and len(ops) > 1 and ops[1] == "exec":
        regs = frozenset(_sregs(dst))
        copies = {c for c in copies if not (c & regs)}
        if full:
            copies.add(regs)
        return full, copies
    # any other SGPR write invalidates the copies it overlaps
    written: set[int] = set()
    if op.startswith("s_") and dst.startswith("s"):
        written = _sregs(dst)
    elif op.startswith("v_") and len(ops) > 1:
        for t in ops[:2]:  # VOP3 carry-out / compare / readlane destinations
            if t.startswith("s"):
                written |= _sregs(t)
    elif op.startswith("s_load") or op.startswith("s_buffer_load"):
        written = _sregs(dst)
    if written:
        copies = {c for c in copies if not (c & written)}
    return full, copies


def check(asm: str) -> list[str]:
    """Scratch stores that may run with a partial EXEC mask, one line per finding."""
    hits: list[str] = []
    for name, body in _functions(asm):
        blocks = _parse(body)
        index_of = {b[0]: i for i, b in enumerate(blocks) if b[0]}
        succ = [_succ(blocks, i, index_of) for i in range(len(blocks))]
        start: list = [None] * len(blocks)
        start[0] = (True, frozenset())
        work = [0]
        while work:
            i = work.pop()
            full, copies = start[i]
            copies = set(copies)
            for ln, op, ops in blocks[i][1]:
                full, copies = _transfer((full, copies), op, ops, ln, [], name, "")
            out = (full, frozenset(copies))
            for s in succ[i]:
                cur = start[s]
                new = out if cur is None else (cur[0] and out[0], cur[1] & out[1])
                if new != cur:
                    start[s] = new
                    work.append(s)
        for i, (label, insts) in enumerate(blocks):
            if start[i] is None:
                continue
            full, copies = start[i][0], set(start[i][1])
            for ln, op, ops in insts:
                text = f"{op} {', '.join(ops)}"
                full, copies = _transfer((full, copies), op, ops, ln, hits, name, text)
    return hits
