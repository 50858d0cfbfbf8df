"""Dataflow check of kernels that issue vector-memory loads from inline asm.

The compiler does not know that a load issued from inline asm is still in
flight: the load writes its destination registers whenever it returns, and
only an ``s_waitcnt vmcnt(N)`` that retires it makes the registers safe to
read or reuse.  This check walks the gfx950 assembly of one function over its
control-flow graph and reports every instruction that reads or overwrites a
register that an outstanding load may still write.

State at each program point: the outstanding vector-memory operations,
newest first (loads carry their destination registers; stores, atomics and
direct-to-LDS loads carry none).  ``s_waitcnt vmcnt(N)`` keeps the N newest
(vmcnt retires in issue order).  At a join the states merge position by
position (a register is pending if it is pending on any predecessor), and the
blocks are iterated to a fixed point.  The check is conservative: loads the
compiler issued itself are tracked too (its own waits retire them).
"""

from __future__ import annotations

import re

MAX_QUEUE = 64  # vmcnt is a 6-bit counter


def _regs(tok: str) -> frozenset:
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return frozenset({int(m.group(1))}) if m else frozenset()


def _union(toks) -> frozenset:
    out = frozenset()
    for t in toks:
        out |= _regs(t)
    return out


def function_body(asm: str, name: str) -> list[str]:
    """The instruction lines (comments stripped) of function `name`."""
    i = asm.index(name + ":")
    j = asm.index(".Lfunc_end", i)
    return [line.split(";")[0].strip() for line in asm[i:j].split("\n")[1:]]


def _blocks(lines):
    blocks, labels, cur = [], {}, []
    for k, line in enumerate(lines):
        if not line:
            continue
        if line.startswith(".L") and line.endswith(":"):
            if cur:
                blocks.append(cur)
            labels[line[:-1]] = len(blocks)
            cur = []
            continue
        if line.startswith("."):
            continue
        cur.append((k, line))
        op = line.split()[0]
        if op.startswith("s_cbranch") or op in ("s_branch", "s_endpgm") or op.startswith("s_setpc"):
            blocks.append(cur)
            cur = []
    if cur:
        blocks.append(cur)
    succ = []
    for bi, b in enumerate(blocks):
        out = []
        last = b[-1][1] if b else ""
        op = last.split()[0] if last else ""
        if op == "s_branch":
            out.append(labels.get(last.split()[1]))
        elif op.startswith("s_cbranch"):
            out += [labels.get(last.split()[1]), bi + 1]
        elif op not in ("s_endpgm",) and not op.startswith("s_setpc"):
            out.append(bi + 1)
        succ.append([x for x in out if x is not None and x < len(blocks)])
    return blocks, succ


def _merge(a, b):
    if a is None:
        return b
    n = max(len(a), len(b))
    return tuple((a[t] if t < len(a) else frozenset()) | (b[t] if t < len(b) else frozenset()) for t in range(n))


def check_function(asm: str, name: str) -> list[tuple[int, str, str]]:
    """(line index, kind, instruction) of every read or overwrite of a
    register an outstanding load may still write, in function `name`."""
    blocks, succ = _blocks(function_body(asm, name))
    state = [None] * len(blocks)
    if blocks:
        state[0] = tuple()
    reports = {}
    changed, rounds = True, 0
    while changed and rounds < 500:
        changed, rounds = False, rounds + 1
        for bi, block in enumerate(blocks):
            if state[bi] is None:
                continue
            q = list(state[bi])
            for k, line in block:
                op = line.split()[0]
                toks = [t.strip(",") for t in line.split()[1:]]
                pend = frozenset().union(*q) if q else frozenset()
                if op == "s_waitcnt" and "vmcnt" in line:
                    q = q[: int(re.search(r"vmcnt\((\d+)\)", line).group(1))]
                    continue
                is_load = op.startswith(("global_load", "buffer_load", "flat_load"))
                if is_load and (op.startswith("global_load_lds") or " lds" in line):
                    if _union(toks) & pend:
                        reports[k] = ("address read", line)
                    q = ([frozenset()] + q)[:MAX_QUEUE]
                    continue
                if is_load:
                    dst, src = _regs(toks[0]), _union(toks[1:])
                    if src & pend:
                        reports[k] = ("address read", line)
                    if dst & pend:
                        reports[k] = ("load over a pending register", line)
                    q = ([dst] + q)[:MAX_QUEUE]
                    continue
                if op.startswith(("global_store", "buffer_store", "flat_store", "global_atomic", "buffer_atomic")):
                    if _union(toks) & pend:
                        reports[k] = ("store of a pending register", line)
                    q = ([frozenset()] + q)[:MAX_QUEUE]
                    continue
                if op.startswith(("ds_write", "ds_store")):
                    if _union(toks) & pend:
                        reports[k] = ("read", line)
                    continue
                if toks:
                    dst, src = _regs(toks[0]), _union(toks[1:])
                    if src & pend:
                        reports[k] = ("read", line)
                    if dst & pend and not op.startswith("s_"):
                        reports[k] = ("overwrite", line)
            out = tuple(q)
            for sb in succ[bi]:
                m = _merge(state[sb], out)
                if m != state[sb]:
                    state[sb] = m
                    changed = True
    if changed:
        raise RuntimeError(f"{name}: dataflow did not converge")
    return [(k, kind, line) for k, (kind, line) in sorted(reports.items())]


def functions_named(asm: str, fragment: str) -> list[str]:
    """Symbols of the functions whose (mangled) name contains `fragment`."""
    return re.findall(r"^(_Z\S*" + re.escape(fragment) + r"\S*):", asm, flags=re.M)
