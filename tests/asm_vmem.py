"""Vector-memory counts along the paths of a gfx950 assembly function.

A kernel that loads straight into LDS (`buffer_load_dwordx4 ... lds`,
`global_load_lds_dwordx4`) has to wait for those loads itself: the compiler
does not track them, so the source states `s_waitcnt vmcnt(N)` by hand, and
N is right only while the loads issued between two waits are the ones the
source counts. `walk` follows every path of a function through its basic
blocks and records, at each `s_waitcnt` that names a vmcnt, which vector
memory operations can be in flight just before it (oldest first). vmcnt
retires in issue order on gfx950 (loads and stores share the counter), so
`vmcnt(N)` leaves exactly the newest N of them.

Each in-flight entry is (kind, line, fresh): kind "lds" for a
direct-to-LDS load and "vmem" for any other vector memory operation, the
line of the instruction in the listing, and whether it was issued after
the last `s_barrier` on the path. Paths are walked without regard to
branch conditions, so paths the kernel can never take are included: the
properties checked on them must hold whatever the branches decide.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

VMEM = re.compile(r"^(?:buffer|global|flat|scratch)_(?:load|store|atomic)\w*")
WAIT_VM = re.compile(r"\bvmcnt\((\d+)\)")
BRANCH = re.compile(r"^s_(?:c)?branch\w*\s+(\.L\w+)")
MAX_VMCNT = 63


@dataclass
class Block:
    label: str
    instrs: list = field(default_factory=list)   # (line, text)
    succ: list = field(default_factory=list)     # block indices


def function_body(asm: str, symbol: str) -> list:
    """(line, instruction) of one function, from its label to .Lfunc_end."""
    lines = asm.splitlines()
    start = next((i for i, l in enumerate(lines) if l.startswith(symbol + ":")), None)
    if start is None:
        raise KeyError(symbol)
    out = []
    for i in range(start + 1, len(lines)):
        text = lines[i].split(";", 1)[0].strip()
        if text.startswith(".Lfunc_end"):
            break
        if not text or (text.startswith(".") and not text.endswith(":")):
            continue
        out.append((i + 1, text))
    return out


def blocks(body: list) -> list:
    """Basic blocks: a label starts one; a branch or s_endpgm ends one."""
    bl = [Block("<entry>")]
    for line, text in body:
        if text.endswith(":"):
            if bl[-1].instrs or bl[-1].label != "<entry>":
                bl.append(Block(text[:-1]))
            else:
                bl[-1].label = text[:-1]
            continue
        bl[-1].instrs.append((line, text))
        if text.startswith("s_branch") or text.startswith("s_cbranch") or text.startswith("s_endpgm") \
                or text.startswith("s_setpc"):
            bl.append(Block(f"<after {line}>"))
    index = {b.label: i for i, b in enumerate(bl)}
    for i, b in enumerate(bl):
        last = b.instrs[-1][1] if b.instrs else ""
        m = BRANCH.match(last)
        if last.startswith("s_endpgm") or last.startswith("s_setpc"):
            continue
        if m:
            b.succ.append(index[m.group(1)])
            if last.startswith("s_branch"):
                continue
        if i + 1 < len(bl):
            b.succ.append(i + 1)
    return bl


@dataclass
class Walk:
    waits: dict          # line of a vmcnt wait -> {(vmcnt, in-flight tuple)}
    barriers: dict       # line of an s_barrier -> {direct-to-LDS loads issued since the last barrier}
    instr: dict          # line -> instruction text


def walk(body: list) -> Walk:
    bl = blocks(body)
    waits, barriers = {}, {}
    instr = {line: text for line, text in body}
    # state: (in-flight entries, direct-to-LDS loads issued since the last barrier)
    seen = set()
    work = [(0, ((), 0))]
    while work:
        bi, state = work.pop()
        if (bi, state) in seen:
            continue
        seen.add((bi, state))
        fly, since = state
        for line, text in bl[bi].instrs:
            if VMEM.match(text):
                kind = "lds" if re.search(r"\blds\b", text) or "load_lds" in text else "vmem"
                fly = (fly + ((kind, line, True),))[-MAX_VMCNT - 1:]
                if kind == "lds":
                    since += 1
            elif text.startswith("s_waitcnt"):
                m = WAIT_VM.search(text)
                if m:
                    n = int(m.group(1))
                    waits.setdefault(line, set()).add((n, fly))
                    fly = fly[len(fly) - n:] if n < len(fly) else fly
            elif text.startswith("s_barrier"):
                barriers.setdefault(line, set()).add(since)
                fly = tuple((k, l, False) for k, l, _ in fly)
                since = 0
        for s in bl[bi].succ:
            work.append((s, (fly, since)))
    return Walk(waits, barriers, instr)


def mangled(kernel: str, template: str, args: str) -> str:
    """Itanium name of swiftllm::(anonymous)::kernel<template>(args)."""
    return (f"_ZN8swiftllm12_GLOBAL__N_1{len(kernel)}{kernel}I{template}EEvNS0_{len(args)}{args}E")
