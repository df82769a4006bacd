"""Static check of LDS / scalar-load completion in gfx950 assembly (test helper).

Some kernels issue their LDS reads as inline asm (``ds_read_b128``, ``ds_read_b64_tr_b16``) and
wait for them with explicit ``s_waitcnt lgkmcnt(N)``.  The compiler does not track those reads, so
a count that is off by one lets an instruction consume a register before its load has returned:
the hardware does not interlock on it.  This module replays the counter through the control-flow
graph of every kernel in an assembly listing and reports each instruction that reads or writes a
VGPR / AGPR while a load into that register may still be outstanding.

Model (CDNA3/CDNA4 ISA, "Data dependency resolution"): every LDS instruction (``ds_*``) and every
scalar memory instruction (``s_load*``, ``s_buffer_load*``, ``s_memtime`` ...) increments
``lgkmcnt``; LDS operations return in issue order, scalar ones in any order.  After
``s_waitcnt lgkmcnt(N)`` with T operations outstanding, of which s are scalar, at least the
T - N - s oldest LDS operations have returned (all of them when N = 0).  So whether an operation
has returned depends only on its distance from the newest one and on the scalar count: a join in
the graph keeps the states that reach it, and where too many do, widens them into one whose entry
at each distance holds the union of their registers there (scalar if any of them is).
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

_LABEL = re.compile(r"^(\.LBB[\w.]+|[A-Za-z_][\w.$]*):")
_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


@dataclass(frozen=True)
class Op:
    scalar: bool          # a scalar-memory operation (returns out of order)
    regs: frozenset       # vector registers it writes on return
    line: int = field(compare=False)  # where it was issued (for the report only)


@dataclass
class Finding:
    kernel: str
    line: int
    text: str
    pending_from: int

    def __str__(self) -> str:
        return f"{self.kernel}: line {self.line}: `{self.text}` touches a register loaded at line {self.pending_from}"


def _regs(operands: str) -> set:
    out = set()
    for m in _REG.finditer(operands):
        kind = m.group(1)
        if m.group(4) is not None:
            out.add((kind, int(m.group(4))))
        else:
            out.update((kind, r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


@dataclass
class _Block:
    name: str
    insts: list = field(default_factory=list)   # (line number, mnemonic, operands, text)
    succ: list = field(default_factory=list)


def _split_kernels(asm: str) -> dict:
    """Map each kernel symbol to its (line number, text) body."""
    lines = asm.split("\n")
    kernels = {}
    cur = None
    for i, raw in enumerate(lines, 1):
        s = raw.strip()
        m = re.match(r"^(_Z\w+):", s)
        if m and cur is None:
            cur = m.group(1)
            kernels[cur] = []
            continue
        if cur is not None:
            if s.startswith(".Lfunc_end"):
                cur = None
                continue
            kernels[cur].append((i, raw))
    return kernels


def _blocks(body: list) -> list:
    blocks = [_Block("<entry>")]
    for ln, raw in body:
        s = raw.split(";")[0].strip()
        if not s or s.startswith("."):
            m = _LABEL.match(s)
            if m and s.startswith(".LBB"):
                blocks.append(_Block(m.group(1)))
            continue
        m = _LABEL.match(s)
        if m:
            blocks.append(_Block(m.group(1)))
            continue
        parts = s.split(None, 1)
        blocks[-1].insts.append((ln, parts[0], parts[1] if len(parts) > 1 else "", s))
        if parts[0].startswith(("s_cbranch", "s_branch", "s_endpgm", "s_setpc", "s_trap")):
            blocks.append(_Block(f"<after {ln}>"))  # a branch ends its block
    index = {b.name: k for k, b in enumerate(blocks)}
    for k, b in enumerate(blocks):
        last = b.insts[-1] if b.insts else None
        falls = True
        if last is not None:
            mn, ops = last[1], last[2]
            if mn == "s_branch":
                b.succ.append(index[ops.split()[0]])
                falls = False
            elif mn.startswith("s_cbranch"):
                b.succ.append(index[ops.split()[0]])
            elif mn in ("s_endpgm", "s_setpc_b64", "s_trap"):
                falls = False
        if falls and k + 1 < len(blocks):
            b.succ.append(k + 1)
    return blocks


_LGKM_MAX = 15  # the counter's width on gfx9: issue stalls while 15 operations are outstanding


def _retire(state: tuple, n: int) -> tuple:
    if n == 0:
        return ()
    if len(state) <= n:
        return state
    scalar = sum(1 for o in state if o.scalar)
    done = max(0, len(state) - n - scalar)
    out = []
    for o in state:
        if not o.scalar and done > 0:
            done -= 1
            continue
        out.append(o)
    return tuple(out)


def _step(state: tuple, inst, kernel: str, findings: list) -> tuple:
    ln, mn, ops, text = inst
    if mn == "s_waitcnt":
        m = _LGKM.search(ops)
        if m:
            state = _retire(state, int(m.group(1)))
        elif ops.strip() == "0":
            state = ()
        return state
    lds = mn.startswith("ds_")
    writes = lds and (mn.startswith(("ds_read", "ds_load", "ds_bpermute", "ds_permute", "ds_swizzle")) or "_rtn" in mn)
    dst = _regs(ops.split(",")[0]) if writes else set()
    # An LDS load may target a register that an earlier LDS load still has in flight: they
    # return in order.  Its other operands, and every other instruction's, must have landed.
    used = _regs(ops.split(",", 1)[1]) if writes and "," in ops else _regs(ops)
    for o in state:
        if o.regs & used or (o.scalar and o.regs & dst):
            findings.append(Finding(kernel, ln, text, o.line))
            break
    if lds:
        state = _retire(state, _LGKM_MAX - 1) + (Op(False, frozenset(dst), ln),)
    elif mn.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_dcache", "s_sendmsg",
                        "s_scratch_load", "s_get_waveid")) or mn.startswith("flat_"):
        dst = _regs(ops.split(",")[0]) if mn.startswith("flat_load") else set()
        state = _retire(state, _LGKM_MAX - 1)
        if len(state) >= _LGKM_MAX:  # only scalar operations left: one of them has returned
            state = state[1:]
        state = state + (Op(True, frozenset(dst), ln),)
    return state


def _join(states) -> tuple:
    """One state covering every given one: entries aligned from the newest, registers united."""
    n = max(len(st) for st in states)
    out = []
    for d in range(n, 0, -1):  # distance from the end
        ents = [st[len(st) - d] for st in states if len(st) >= d]
        regs = frozenset().union(*(e.regs for e in ents))
        out.append(Op(any(e.scalar for e in ents), regs, ents[0].line))
    return tuple(out)


def _covers(big: tuple, small: tuple) -> bool:
    if len(small) > len(big):
        return False
    for d in range(1, len(small) + 1):
        a, b = big[-d], small[-d]
        if not b.regs <= a.regs or (b.scalar and not a.scalar):
            return False
    return True


def check_kernel(name: str, body: list, max_states: int = 64) -> list:
    blocks = _blocks(body)
    entry_states = [set() for _ in blocks]
    entry_states[0].add(())
    work = [0]
    findings: list = []
    seen_findings = set()
    while work:
        k = work.pop()
        for st in list(entry_states[k]):
            local: list = []
            s = st
            for inst in blocks[k].insts:
                s = _step(s, inst, name, local)
            for f in local:
                key = (f.line, f.pending_from)
                if key not in seen_findings:
                    seen_findings.add(key)
                    findings.append(f)
            for j in blocks[k].succ:
                have = entry_states[j]
                if s in have or any(_covers(h, s) for h in have):
                    continue
                have.add(s)
                if len(have) > max_states:
                    entry_states[j] = {_join(list(have))}
                if j not in work:
                    work.append(j)
    return findings


def check_asm(asm: str, kernel_filter=None) -> tuple:
    """Check every kernel of an assembly listing; returns (kernels checked, findings)."""
    kernels = _split_kernels(asm)
    names = [n for n in kernels if kernel_filter is None or kernel_filter(n)]
    findings = []
    for n in names:
        findings += check_kernel(n, kernels[n])
    return names, findings
