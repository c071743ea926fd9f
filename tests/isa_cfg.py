"""Control-flow graphs of kernels this repository builds, from their disassembly.

Test infrastructure for the device-code invariants: basic blocks of one kernel's
instructions, its branch edges, and which instructions can reach which, so a test can
find the waits that sit between the global -> LDS transfers of a pipelined loop and
check them against the loop's budget.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

_ADDR = re.compile(r"//\s*([0-9A-Fa-f]+):")
_TARGET = re.compile(r"<[^>+]+\+0x([0-9a-fA-F]+)>")


@dataclass
class Insn:
    addr: int
    mnemonic: str
    text: str
    target_off: int | None = None  # a branch's target, as an offset from the function


@dataclass
class Block:
    index: int
    insns: list = field(default_factory=list)
    succs: list = field(default_factory=list)


def build(lines: list[str]) -> list[Block]:
    """Basic blocks of one function's disassembly lines, with successor indices."""
    insns = []
    for line in lines:
        m = _ADDR.search(line)
        if not m:
            continue
        body = line[:m.start()].strip()
        t = _TARGET.search(line)
        insns.append(Insn(int(m.group(1), 16), body.split()[0], body, int(t.group(1), 16) if t else None))
    if not insns:
        return []
    base = insns[0].addr
    leaders = {insns[0].addr}
    for i, insn in enumerate(insns):
        if insn.mnemonic.startswith(("s_branch", "s_cbranch")):
            leaders.add(base + insn.target_off)
            if i + 1 < len(insns):
                leaders.add(insns[i + 1].addr)
        elif insn.mnemonic == "s_endpgm" and i + 1 < len(insns):
            leaders.add(insns[i + 1].addr)
    blocks, at = [], {}
    for insn in insns:
        if insn.addr in leaders or not blocks:
            blocks.append(Block(len(blocks)))
            at[insn.addr] = blocks[-1].index
        blocks[-1].insns.append(insn)
    for b in blocks:
        last = b.insns[-1]
        nxt = b.index + 1 if b.index + 1 < len(blocks) else None
        if last.mnemonic == "s_endpgm":
            continue
        if last.mnemonic.startswith("s_branch"):
            b.succs.append(at[base + last.target_off])
        elif last.mnemonic.startswith("s_cbranch"):
            b.succs.append(at[base + last.target_off])
            if nxt is not None:
                b.succs.append(nxt)
        elif nxt is not None:
            b.succs.append(nxt)
    return blocks


def reachable(blocks: list[Block], starts: set[int], reverse: bool = False) -> set[int]:
    """Blocks reachable from `starts` by one or more edges (backwards with `reverse`)."""
    edges = {b.index: list(b.succs) for b in blocks}
    if reverse:
        rev = {b.index: [] for b in blocks}
        for b in blocks:
            for s in b.succs:
                rev[s].append(b.index)
        edges = rev
    seen, todo = set(), [s2 for s in starts for s2 in edges[s]]
    while todo:
        x = todo.pop()
        if x in seen:
            continue
        seen.add(x)
        todo.extend(edges[x])
    return seen


def vmcnt(insn: Insn):
    """The vmcnt field of an s_waitcnt, or None."""
    if insn.mnemonic != "s_waitcnt":
        return None
    m = re.search(r"vmcnt\((\d+)\)", insn.text)
    return int(m.group(1)) if m else None


def lgkm_zero(insn: Insn) -> bool:
    return insn.mnemonic == "s_waitcnt" and re.search(r"lgkmcnt\(0\)", insn.text) is not None


def is_dma(insn: Insn) -> bool:
    return insn.mnemonic.startswith("global_load_lds_") or (
        insn.mnemonic.startswith("buffer_load_") and " lds" in insn.text)


def is_lds_read(insn: Insn) -> bool:
    return insn.mnemonic.startswith(("ds_read", "ds_load"))


def pipeline_waits(blocks: list[Block]) -> list[int]:
    """vmcnt values of the waits that lie on a path from one transfer to another: the
    waits a pipelined loop's hand-counted budget sets (those after the last transfer of
    a non-persistent kernel, which the compiler places for its own loads, are not)."""
    dma_blocks = {b.index for b in blocks if any(is_dma(i) for i in b.insns)}
    after = reachable(blocks, dma_blocks)
    before = reachable(blocks, dma_blocks, reverse=True)
    out = []
    for b in blocks:
        seen_dma = False
        for i, insn in enumerate(b.insns):
            if is_dma(insn):
                seen_dma = True
            n = vmcnt(insn)
            if n is None:
                continue
            dma_after_here = any(is_dma(x) for x in b.insns[i + 1:]) or b.index in before
            dma_before_here = seen_dma or b.index in after
            if dma_before_here and dma_after_here:
                out.append(n)
    return out


def barriers_after_unfinished_lds_reads(blocks: list[Block]) -> list[int]:
    """Addresses of the s_barrier instructions that some path reaches with an LDS read
    issued but not waited for (no lgkmcnt(0) between them): forward data flow of the
    flag "an LDS read may be outstanding" over the graph."""
    state_in = {b.index: False for b in blocks}
    changed = True
    while changed:
        changed = False
        for b in blocks:
            s = state_in[b.index]
            for insn in b.insns:
                if is_lds_read(insn):
                    s = True
                elif lgkm_zero(insn):
                    s = False
            for t in b.succs:
                if s and not state_in[t]:
                    state_in[t] = True
                    changed = True
    bad = []
    for b in blocks:
        s = state_in[b.index]
        for insn in b.insns:
            if is_lds_read(insn):
                s = True
            elif lgkm_zero(insn):
                s = False
            elif insn.mnemonic == "s_barrier" and s:
                bad.append(insn.addr)
    return bad
