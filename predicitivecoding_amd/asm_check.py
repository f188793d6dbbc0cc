"""Build-time check of the kernels' inline-asm vector loads (gfx9 assembly).

The direct-weight phase kernels load weight fragments with inline-asm
`global_load_dwordx4`, which the compiler's wait-count pass does not see: the
kernel source waits for them itself (`s_waitcnt vmcnt(N)` with the registers
as operands) and keeps the registers allocated until they have landed.  This
check verifies that on the generated code.  It walks each kernel's control
flow to a fixed point, tracking every asm load still in flight together with
the smallest number of vector-memory operations issued after it on any path;
`s_waitcnt vmcnt(N)` retires the loads with at least N younger operations.
Any instruction that reads or writes a register an in-flight asm load will
still write is an error, and so is `s_endpgm` with asm loads in flight.  DMA
loads into LDS (`global_load_lds_*`) write no register and only count.
"""
from __future__ import annotations

import re

_REG = re.compile(r'\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)')
_VMEM = re.compile(r'^(global|buffer|flat|scratch)_')
_VMCNT = re.compile(r'vmcnt\((\d+)\)')


def _regs(text: str) -> set:
    out = set()
    for m in _REG.finditer(text):
        if m.group(4) is not None:
            out.add((m.group(1), int(m.group(4))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def _parse(lines: list[str], start: int):
    """Instructions (opcode, operands, issued from inline asm) and labels of the function at `start`."""
    insts, labels, in_asm = [], {}, False
    for raw in lines[start + 1:]:
        s = raw.strip()
        if s.startswith(';;#ASMSTART'):
            in_asm = True
            continue
        if s.startswith(';;#ASMEND'):
            in_asm = False
            continue
        s = s.split(';')[0].strip()
        if not s or s.startswith('//'):
            continue
        if s.startswith('.Lfunc_end'):
            break
        if s.endswith(':'):
            labels[s[:-1]] = len(insts)
            continue
        if s.startswith('.'):
            continue
        op, _, rest = s.partition(' ')
        insts.append((op, rest.strip(), in_asm))
    return insts, labels


def _successors(i: int, insts, labels) -> list[int]:
    op, rest, _ = insts[i]
    if op == 's_endpgm':
        return []
    if op == 's_branch':
        return [labels[rest.split()[0]]]
    if op.startswith('s_cbranch'):
        return [labels[rest.split()[0]], i + 1]
    return [i + 1]


def check_function(lines: list[str], start: int) -> list[str]:
    """Problems found in the function whose label is at lines[start]."""
    insts, labels = _parse(lines, start)
    n = len(insts)
    state_in: list[dict | None] = [None] * n
    if n == 0:
        return []
    state_in[0] = {}
    work, problems = [0], set()
    while work:
        i = work.pop()
        st = dict(state_in[i])
        op, rest, in_asm = insts[i]
        if op == 's_waitcnt':
            m = _VMCNT.search(rest)
            if m:
                keep = int(m.group(1))
                st = {k: v for k, v in st.items() if v[0] < keep}
        else:
            pending = set()
            for _, regs in st.values():
                pending |= regs
            hit = _regs(rest) & pending
            if hit:
                problems.add(f'#{i} {op} {rest}: in-flight asm load target {sorted(hit)[0]}')
            if _VMEM.match(op):
                st = {k: (min(y + 1, 64), r) for k, (y, r) in st.items()}
                if in_asm and 'load' in op:
                    st[i] = (0, frozenset() if '_lds_' in op else frozenset(_regs(rest.split(',')[0])))
            if op == 's_endpgm' and st:
                problems.add(f'#{i} s_endpgm with asm loads in flight')
        for j in _successors(i, insts, labels):
            if j >= n:
                continue
            old = state_in[j]
            if old is None:
                new = dict(st)
            else:
                new = dict(old)
                for k, (y, r) in st.items():
                    new[k] = (min(new[k][0], y), r) if k in new else (y, r)
            if new != old:
                state_in[j] = new
                work.append(j)
    return sorted(problems)


def check_asm(text: str, name_filter: str = 'phase_kernel') -> dict[str, list[str]]:
    """Problems per kernel (functions whose symbol contains name_filter) of an assembly listing."""
    lines = text.split('\n')
    out = {}
    for i, line in enumerate(lines):
        m = re.match(r'^([A-Za-z_][\w.$]*):', line)
        if m and name_filter in m.group(1) and not m.group(1).startswith('.'):
            out[m.group(1)] = check_function(lines, i)
    return out
