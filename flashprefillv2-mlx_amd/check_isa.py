"""Static check of the kernels' asynchronous LDS reads.

The sparse-attention kernel and the owner path (head_dim 256) of the
selection kernel issue their LDS reads as inline asm (the compiler would
otherwise serialise them behind the asynchronous global->LDS fills) and
waits for them with ``s_waitcnt lgkmcnt(N)``.  The compiler treats the result
register of such a read as written when the asm statement ends, so nothing
stops it from copying or spilling that register before the data has arrived.
This checker reads the gfx950 assembly of the kernels and fails if any
instruction reads or writes the destination registers of an LDS read that is
still in flight:

* LDS operations (``ds_*``) complete in order; ``s_waitcnt lgkmcnt(N)``
  retires all but the N youngest;
* every path through the function's branches is followed (a dataflow over
  its basic blocks, loops included), and no read may stay in flight at the
  end of the function (LDS writes, which have no destination registers,
  still count towards the in-order retirement but may stay in flight);
* scalar-memory loads also count in lgkmcnt and may complete out of order,
  but a wait for at most N outstanding operations in all leaves at most N
  LDS operations outstanding, the N youngest, whatever else is in flight.

Usage: ``python check_isa.py kernel.s [symbol-substring]``; exit status 1 on
a violation.  ``build.py`` runs it on every build.
"""

from __future__ import annotations

import re
import sys

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)(?!\w))")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def _regs(operands: str) -> set[tuple[str, int]]:
    out = set()
    for kind, lo, hi, single in _REG.findall(operands):
        if single:
            out.add((kind, int(single)))
        else:
            out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    return out


_BRANCHES = ("s_branch", "s_cbranch_scc0", "s_cbranch_scc1", "s_cbranch_vccz",
             "s_cbranch_vccnz", "s_cbranch_execz", "s_cbranch_execnz")


def _step(pending: tuple, op: str, rest: str, i: int, s: str, name: str, errors: list[str]):
    """One instruction on one path's state: the tuple of in-flight LDS ops
    ``(line, dest regs)``, oldest first.  Returns the state after it."""
    if op == "s_waitcnt":
        m = _LGKM.search(rest)
        if m and len(pending) > int(m.group(1)):
            n = int(m.group(1))
            return pending[len(pending) - n:] if n else ()
        return pending
    regs = _regs(rest)
    if op.startswith("ds_"):
        # operands: dest first for reads; a DS op may not touch in-flight dests either
        dest: frozenset = frozenset()
        if op.startswith(("ds_read", "ds_bpermute", "ds_permute", "ds_swizzle")):
            first = rest.split(",")[0]
            dest = frozenset(_regs(first))
            srcs = _regs(",".join(rest.split(",")[1:]))
        else:
            srcs = regs
        for line_no, d in pending:
            if (srcs | dest) & d:
                errors.append(f"{name}: line {i} `{s}` touches registers of the LDS "
                              f"read at line {line_no} before its wait")
        return pending + ((i, dest),)
    for line_no, d in pending:
        if regs & d:
            errors.append(f"{name}: line {i} `{s}` touches registers of the LDS "
                          f"read at line {line_no} before its wait")
    return pending


def check_function(name: str, lines: list[str]) -> list[str]:
    """Dataflow over the function's basic blocks: each block's entry holds the
    set of states of the paths that reach it (the fall-through and every
    branch to its label, backward branches included), iterated until no
    set grows."""
    errors: list[str] = []
    # basic blocks: (first line, [(line, op, rest, text)], successor labels, falls through)
    blocks: list[tuple[str | None, list, list[str], bool]] = []
    label: str | None = None
    body: list = []

    def close(succ: list[str], falls: bool) -> None:
        nonlocal label, body
        blocks.append((label, body, succ, falls))
        label, body = None, []

    for i, raw in enumerate(lines):
        s = raw.split(";")[0].strip()
        if not s or (s.startswith(".") and not s.endswith(":")):
            continue
        if s.endswith(":"):
            close([], True)
            label = s[:-1]
            continue
        op, _, rest = s.partition(" ")
        if op in _BRANCHES:
            close([rest.strip()], op != "s_branch")
        elif op in ("s_endpgm", "s_setpc_b64"):
            body.append((i, op, rest, s))
            close([], False)
        else:
            body.append((i, op, rest, s))
    close([], False)
    index = {b[0]: k for k, b in enumerate(blocks) if b[0] is not None}

    entry: list[set] = [set() for _ in blocks]
    entry[0].add(())
    work = [0]
    while work:
        k = work.pop()
        _, body, succ, falls = blocks[k]
        states = set(entry[k])
        for i, op, rest, s in body:
            if op == "s_endpgm":
                if any(d for st in states for _, d in st):
                    errors.append(f"{name}: LDS read(s) in flight at s_endpgm (line {i})")
                continue
            nxt = set()
            for st in states:
                st = _step(st, op, rest, i, s, name, errors)
                if len(st) > 16:
                    # an operation with no destination registers that 16
                    # younger ones follow is retired by any wait (lgkmcnt
                    # holds at most 15): drop it, so a loop's writes do not
                    # grow the state
                    st = tuple(p for k, p in enumerate(st) if p[1] or k >= len(st) - 16)
                if len(st) > 64:
                    errors.append(f"{name}: LDS reads accumulate without a wait (line {i})")
                    st = st[-64:]
                nxt.add(st)
            states = nxt
        targets = [index[t] for t in succ if t in index]
        if falls and k + 1 < len(blocks):
            targets.append(k + 1)
        for t in targets:
            if not states <= entry[t]:
                entry[t] |= states
                work.append(t)
    return sorted(set(errors))


def check_text(text: str, symbol_filter: str = "sparse_attn_kernel") -> list[str]:
    errors: list[str] = []
    lines = text.splitlines()
    starts = [i for i, l in enumerate(lines)
              if re.match(r"^[A-Za-z_][\w.]*:\s*(;.*)?$", l) and symbol_filter in l]
    for start in starts:
        name = lines[start].split(":")[0]
        end = start + 1
        while end < len(lines) and not lines[end].startswith(".Lfunc_end"):
            end += 1
        errors += check_function(name, lines[start + 1:end])
    return errors


def main(argv: list[str]) -> int:
    text = open(argv[1]).read()
    errors = check_text(text, argv[2] if len(argv) > 2 else "sparse_attn_kernel")
    for e in errors[:50]:
        print(e)
    if errors:
        print(f"{len(errors)} violation(s)")
        return 1
    print("async LDS reads: ok")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
