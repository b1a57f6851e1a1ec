"""Static check of hand-scheduled gfx950 kernels: simulate the in-order vmcnt
queue over a kernel's assembly and report every instruction that reads or
writes a VGPR while a vector-memory load into it is still outstanding.

The GEMM issues its loads from inline asm and waits with explicit vmcnt
counts, so the compiler neither tracks those loads nor inserts waits for them:
a wait count that is too large, or a register the compiler reuses while a load
into it is in flight (it sees the asm write the register at once), is a race
the hardware does not catch.  Vector-memory loads return in issue order, so
`s_waitcnt vmcnt(N)` retires all but the N most recent.

The path simulated is the kernel's text in order with its K loop body
repeated: prologue, body x iters, then everything after the loop.
"""
from __future__ import annotations

import re

_VREG = re.compile(r'^v\[(\d+):(\d+)\]$|^v(\d+)$')


def _regs(tok: str) -> set:
    m = _VREG.match(tok)
    if not m:
        return set()
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


def _parse(lines):
    out = []
    for line in lines:
        line = line.split(';')[0].strip()
        if not line or line.startswith('.') or line.endswith(':'):
            continue
        parts = line.replace(',', ' ').split()
        out.append((parts[0], parts[1:], line))
    return out


def kernels(asm: str) -> dict:
    """{symbol: [lines]} for every kernel function in an assembly listing."""
    lines = asm.splitlines()
    out, name, body = {}, None, []
    for line in lines:
        m = re.match(r'^(_Z\S+):', line)
        if m and '@' in line:
            name, body = m.group(1), []
            continue
        if name is not None:
            body.append(line)
            if 's_endpgm' in line:
                out[name] = body
                name = None
    return out


def _simulate(seq):
    q, bad = [], []
    for idx, (op, ops, text) in enumerate(seq):
        if op == 's_waitcnt':
            m = re.search(r'vmcnt\((\d+)\)', text)
            if m:
                n = int(m.group(1))
                while len(q) > n:
                    q.pop(0)
            continue
        if op.startswith(('buffer_load', 'global_load')):
            if text.rstrip().endswith('lds'):
                q.append(set())  # LDS DMA: no VGPR destination
                continue
            dst = _regs(ops[0])
            if any(dst & p for p in q):
                bad.append((idx, 'load into a register with a load in flight', text))
            q.append(dst)
            continue
        if op.startswith(('buffer_store', 'global_store', 'buffer_atomic', 'global_atomic')):
            q.append(set())
            continue
        if op.startswith('s_'):
            continue
        regs = [_regs(o) for o in ops]
        if not regs:
            continue
        if op.startswith('ds_write'):
            dst, src = set(), set().union(*regs)
        else:
            dst, src = regs[0], set().union(*regs[1:]) if len(regs) > 1 else set()
        pending = set().union(*q) if q else set()
        if dst & pending:
            bad.append((idx, 'write of a register with a load in flight', text))
        if src & pending:
            bad.append((idx, 'read of a register with a load in flight', text))
    return bad


_LABEL = re.compile(r'^(\.LBB\w+):')


def _loops(body_lines):
    """{header label: (first line, last line, depth)} of every loop, from the
    compiler's block annotations: a loop is its header block, the blocks
    marked as inside it, and everything up to its last branch back into it."""
    labels = {}
    for i, l in enumerate(body_lines):
        m = _LABEL.match(l.strip())
        if m:
            labels[m.group(1)] = i
    out = {}
    for lab, i in labels.items():
        text = body_lines[i] + (body_lines[i + 1] if i + 1 < len(body_lines) else '')
        m = re.search(r'Loop Header: Depth=(\d+)', text)
        if not m:
            continue
        tag = lab.lstrip('.').replace('LBB', 'BB')
        members = [j for l2, j in labels.items()
                   if j == i or f'Header={tag} ' in body_lines[j] + ' '
                   or f'Parent Loop {tag} ' in body_lines[j] + ' ']
        names = {l2 for l2, j in labels.items() if j in members}
        start = min(members)
        last = max(j for j, l in enumerate(body_lines)
                   if ('s_cbranch' in l or 's_branch' in l) and l.split()[-1] in names
                   and j >= start)
        out[lab] = (start, last, int(m.group(1)), i)
    return out


def hazards(body_lines, iters: int = 3):
    """Hazards on the path prologue -> loop body x iters -> rest, for the
    kernel's first loop (the K loop).  When the first loop holds a nested loop
    (a tile loop around the K loop), the path is prologue -> (outer body with
    the inner body x iters) x 2 -> rest, the outer body entered at its header
    (blocks the compiler placed before the header run after it)."""
    loops = _loops(body_lines)
    if not loops:
        return _simulate(_parse(body_lines))
    outer = min(loops.values(), key=lambda v: v[0])
    start, last, depth, hdr = outer
    pre, post = _parse(body_lines[:start]), _parse(body_lines[last + 1:])
    inner = [v for v in loops.values() if v[2] == depth + 1 and start <= v[0] <= last]
    if not inner:
        body = _parse(body_lines[hdr:last + 1]) + _parse(body_lines[start:hdr])
        return _simulate(pre + body * iters + post)
    istart, ilast, _, _ = min(inner, key=lambda v: v[0])
    main = (_parse(body_lines[hdr:istart]) + _parse(body_lines[istart:ilast + 1]) * iters
            + _parse(body_lines[ilast + 1:last + 1]))
    body = main + _parse(body_lines[start:hdr])
    return _simulate(pre + body * 2 + post)
