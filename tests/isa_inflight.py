"""Checks, on the gfx950 assembly of a kernel built here, that registers loaded by
inline-assembly loads are not touched before those loads have landed.

The prefill GEMM issues its weight loads from inline assembly (the compiler does not
count them) and waits for them with explicit `s_waitcnt vmcnt(N)`.  The compiler
takes such an output as written when the asm statement executes, while the hardware
writes it when the load returns: a register it then hands to another value is later
overwritten by the load.  This check walks the kernel's control-flow graph: every
`global_load_dword*` between `;;#ASMSTART` and `;;#ASMEND` puts its destination
registers in flight; each later vector-memory instruction ages them by one; an
`s_waitcnt vmcnt(N)` retires every load followed by at least N vector-memory
instructions (loads retire in issue order).  At control-flow merges a load keeps its
smallest age, and the analysis iterates to a fixed point over the loops.  Any
instruction that reads or writes an in-flight register is reported.
"""

from __future__ import annotations

import re

_VMEM = ("global_", "buffer_", "scratch_", "flat_")


def _regs(text: str) -> set:
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def kernel_names(asm: str, prefix: str) -> list:
    return [m.group(1) for m in re.finditer(r"^(%s\S*):" % re.escape(prefix), asm, re.M)]


def inflight_hazards(asm: str, func: str) -> list:
    """(line, registers, instruction) for every touch of an in-flight register."""
    text = asm.split("\n")
    start = next(i for i, l in enumerate(text) if l.startswith(func + ":"))
    end = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
    ins, labels, in_asm = [], {}, False
    for k, raw in enumerate(text[start + 1:end]):
        s = raw.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        m = re.match(r"^(\.LBB\S+):", s)
        if m:
            labels[m.group(1)] = len(ins)
            ins.append((start + k + 2, "LABEL", m.group(1), False))
            continue
        t = s.split(";")[0].strip()
        if t and not t.startswith("."):
            ins.append((start + k + 2, t.split()[0], t, in_asm))
    leaders = {0} | set(labels.values())
    for i, (_, op, _, _) in enumerate(ins):
        if op.startswith(("s_cbranch", "s_branch", "s_endpgm", "s_setpc")):
            leaders.add(i + 1)
    leaders = sorted(x for x in leaders if x < len(ins))
    blocks = {b: (b, leaders[j + 1] if j + 1 < len(leaders) else len(ins))
              for j, b in enumerate(leaders)}

    def succs(b):
        last = ins[blocks[b][1] - 1]
        e0 = blocks[b][1]
        if last[1] == "s_branch":
            return [labels[last[2].split()[1]]]
        if last[1].startswith("s_cbranch"):
            return [labels[last[2].split()[1]]] + ([e0] if e0 < len(ins) else [])
        if last[1] in ("s_endpgm", "s_setpc_b64"):
            return []
        return [e0] if e0 < len(ins) else []

    def transfer(state, b, report):
        st = dict(state)
        for i in range(*blocks[b]):
            ln, op, t, asm_ins = ins[i]
            if op == "LABEL":
                continue
            if op == "s_waitcnt":
                m = re.search(r"vmcnt\((\d+)\)", t)
                if m:
                    n = int(m.group(1))
                    st = {k: v for k, v in st.items() if v[0] < n}
                continue
            rs = _regs(t)
            if report is not None:
                live = set()
                for _, r in st.values():
                    live |= r
                if rs & live:
                    report.append((ln, sorted(rs & live), t))
            if op.startswith(_VMEM):
                st = {k: (min(64, a + 1), r) for k, (a, r) in st.items()}
                if asm_ins and op.startswith("global_load_dword") and "lds" not in op:
                    st[i] = (0, _regs(t.split(",")[0]))
        return st

    def merge(a, b):
        out = dict(a)
        for k, (age, r) in b.items():
            out[k] = (min(age, out[k][0]), r) if k in out else (age, r)
        return out

    ins_state = {b: {} for b in blocks}
    out_state = {b: None for b in blocks}
    work = list(blocks)
    while work:
        b = work.pop(0)
        o = transfer(ins_state[b], b, None)
        if o != out_state[b]:
            out_state[b] = o
            for s in succs(b):
                n = merge(ins_state[s], o)
                if n != ins_state[s]:
                    ins_state[s] = n
                    work.append(s)
    report = []
    for b in blocks:
        transfer(ins_state[b], b, report)
    return report
