"""Build-time check of the AMD assembly of kernels that issue loads as inline assembly.

Inline-assembly ``buffer_load`` instructions with register destinations (the LM head's
weight stream in ``csrc/lm_head.hip``) are invisible to the compiler's wait-count pass:
it treats their destination registers as written when the asm statement ends, so it
could copy, spill or reuse them while the load is still in flight. This module checks
the compiled code instead of trusting the register allocator.

For every kernel in a ``.s`` file it runs a dataflow analysis of the vector-memory
counter over the kernel's control-flow graph: the state at each instruction is the
ordered list of vector-memory operations that may still be outstanding (youngest
last), each with the registers its data will write. ``s_waitcnt vmcnt(n)`` retires all
but the ``n`` youngest; every load, store and LDS-DMA load (``buffer_*``, ``global_*``,
``scratch_*``, ``flat_*``) is appended. States meeting at a join are merged
conservatively (aligned at the youngest entry, register sets united). An instruction
that reads or writes a register of a load that may still be outstanding is a hazard.
Compiler-generated loads pass by construction (the compiler waits before every use it
knows of), so a hazard names an inline-asm load whose destination the compiler touched
too early.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

_VMEM = re.compile(r"^(buffer|global|scratch|flat)_(load|store|atomic)")
_WAIT = re.compile(r"^s_waitcnt\b")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_BRANCH = re.compile(r"^s_(cbranch_\w+|branch)\s+(\.LBB\w+)")
_REG = re.compile(r"\b([va])(?:(\d+)|\[(\d+):(\d+)\])")
_LABEL = re.compile(r"^(\.LBB\w+):")
_FUNC = re.compile(r"^(_Z\w+):")
MAX_OUTSTANDING = 63  # the 6-bit vector-memory counter


def _regs(text: str) -> set:
    out = set()
    for kind, one, lo, hi in _REG.findall(text):
        if one:
            out.add((kind, int(one)))
        else:
            out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    return out


@dataclass
class Inst:
    line: int
    op: str
    text: str          # operands, comment stripped
    regs: set = field(default_factory=set)
    dest: frozenset = frozenset()  # registers a VMEM load writes (empty for stores and LDS-DMA)


@dataclass
class Block:
    name: str
    insts: list = field(default_factory=list)
    succ: list = field(default_factory=list)


def _parse_inst(line_no: int, raw: str) -> Inst | None:
    s = raw.split(";", 1)[0].strip()
    if not s or s.startswith(".") or s.endswith(":"):
        return None
    op, _, rest = s.partition(" ")
    inst = Inst(line_no, op, rest.strip(), _regs(rest))
    if _VMEM.match(op) and "_load" in op and " lds" not in f" {rest} ":
        first = rest.split(",", 1)[0]
        inst.dest = frozenset(_regs(first))
    return inst


def split_functions(asm: str) -> dict:
    """name -> list of (line number, text) of each function body in a .s file."""
    funcs, cur, name = {}, None, None
    for i, line in enumerate(asm.splitlines(), 1):
        m = _FUNC.match(line)
        if m:
            name, cur = m.group(1), []
            funcs[name] = cur
            continue
        if cur is not None:
            if line.strip().startswith(".Lfunc_end") or line.strip().startswith("s_endpgm"):
                if line.strip().startswith("s_endpgm"):
                    cur.append((i, line))
                cur = None if line.strip().startswith(".Lfunc_end") else cur
                continue
            cur.append((i, line))
    return funcs


def build_cfg(body: list) -> list:
    blocks = [Block("<entry>")]
    for ln, line in body:
        m = _LABEL.match(line.strip())
        if m:
            if blocks[-1].insts or blocks[-1].name == "<entry>":
                blocks.append(Block(m.group(1)))
            else:
                blocks[-1].name = m.group(1)
            continue
        inst = _parse_inst(ln, line)
        if inst is None:
            continue
        blocks[-1].insts.append(inst)
        if _BRANCH.match(inst.op + " " + inst.text) or inst.op == "s_endpgm":
            blocks.append(Block(f"<fall{ln}>"))
    index = {b.name: i for i, b in enumerate(blocks)}
    for i, b in enumerate(blocks):
        last = b.insts[-1] if b.insts else None
        fall = i + 1 < len(blocks)
        if last is not None:
            m = _BRANCH.match(last.op + " " + last.text)
            if last.op == "s_endpgm":
                fall = False
            elif m:
                tgt = m.group(2)
                if tgt in index:
                    b.succ.append(index[tgt])
                if m.group(1) == "branch":
                    fall = False
        if fall:
            b.succ.append(i + 1)
    return blocks


def _join(a: tuple, b: tuple) -> tuple:
    n = max(len(a), len(b))
    a = (frozenset(),) * (n - len(a)) + a
    b = (frozenset(),) * (n - len(b)) + b
    return tuple(x | y for x, y in zip(a, b))


def _step(state: tuple, inst: Inst, hazards: list | None, fn: str) -> tuple:
    if _WAIT.match(inst.op):
        m = _VMCNT.search(inst.text)
        if m:
            n = int(m.group(1))
            state = state[len(state) - n:] if n < len(state) else state
            if n == 0:
                state = ()
        return state
    if hazards is not None and inst.regs:
        pending = frozenset().union(*state) if state else frozenset()
        hit = inst.regs & pending
        if hit:
            hazards.append((fn, inst.line, f"{inst.op} {inst.text}", sorted(hit)[:4]))
    if _VMEM.match(inst.op):
        state = (state + (inst.dest,))[-MAX_OUTSTANDING:]
    return state


def check_function(name: str, body: list) -> list:
    """Hazards in one function: (function, line, instruction, registers)."""
    blocks = build_cfg(body)
    entry = [None] * len(blocks)
    entry[0] = ()
    work = [0]
    while work:
        i = work.pop()
        st = entry[i]
        for inst in blocks[i].insts:
            st = _step(st, inst, None, name)
        for s in blocks[i].succ:
            new = st if entry[s] is None else _join(entry[s], st)
            if new != entry[s]:
                entry[s] = new
                work.append(s)
    hazards = []
    for i, b in enumerate(blocks):
        if entry[i] is None:
            continue
        st = entry[i]
        for inst in b.insts:
            st = _step(st, inst, hazards, name)
    return hazards


def check_asm(asm: str, name_filter: str = "") -> tuple:
    """(functions checked, hazards) for every function whose name contains name_filter."""
    funcs = {k: v for k, v in split_functions(asm).items() if name_filter in k}
    hazards = []
    for name, body in funcs.items():
        hazards += check_function(name, body)
    return len(funcs), hazards
