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
* the text is walked linearly, so instructions on skipped branch paths are
  checked as if executed (conservative), and no read may stay in flight
  across a backward branch (loop back-edge) or the end of a function (LDS
  writes, which have no destination registers, still count towards the
  in-order retirement but may stay in flight);
* scalar-memory loads also count in lgkmcnt and may complete out of order; a
  wait with N > 0 while such a load is outstanding retires no LDS read.

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


def check_function(name: str, lines: list[str]) -> list[str]:
    errors: list[str] = []
    pending: list[tuple[int, set]] = []  # in-flight LDS ops: (line, dest regs)
    smem_outstanding = 0
    labels: dict[str, int] = {}
    for i, raw in enumerate(lines):
        s = raw.split(";")[0].strip()
        if not s:
            continue
        if s.endswith(":"):
            labels[s[:-1]] = i
            continue
        if s.startswith("."):
            continue
        op, _, rest = s.partition(" ")
        if op == "s_waitcnt":
            m = _LGKM.search(rest)
            if m:
                n = int(m.group(1))
                if n == 0:
                    pending.clear()
                    smem_outstanding = 0
                elif smem_outstanding == 0:
                    while len(pending) > n:
                        pending.pop(0)
            continue
        if op.startswith("s_load") or op.startswith("s_buffer_load"):
            smem_outstanding += 1
        if op in ("s_branch", "s_cbranch_scc0", "s_cbranch_scc1", "s_cbranch_vccz",
                  "s_cbranch_vccnz", "s_cbranch_execz", "s_cbranch_execnz"):
            target = rest.strip()
            if target in labels and any(d for _, d in pending):
                errors.append(f"{name}: LDS read(s) from line(s) {[p[0] for p in pending if p[1]]} "
                              f"in flight across the back-edge at line {i}: {s}")
            continue
        if op == "s_endpgm" and any(d for _, d in pending):
            errors.append(f"{name}: LDS read(s) in flight at s_endpgm (line {i})")
            continue
        regs = _regs(rest)
        if op.startswith("ds_"):
            # operands: dest first for reads; a DS op may not touch in-flight dests either
            dest: set = set()
            if op.startswith("ds_read") or op.startswith("ds_bpermute") or op.startswith("ds_permute") \
                    or op.startswith("ds_swizzle"):
                first = rest.split(",")[0]
                dest = _regs(first)
                srcs = _regs(",".join(rest.split(",")[1:]))
            else:
                srcs = regs
            for line_no, d in pending:
                if (srcs | dest) & d:
                    errors.append(f"{name}: line {i} `{s}` touches registers of the LDS "
                                  f"read at line {line_no} before its wait")
            pending.append((i, dest))
            continue
        for line_no, d in pending:
            if regs & d:
                errors.append(f"{name}: line {i} `{s}` touches registers of the LDS "
                              f"read at line {line_no} before its wait")
    return errors


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
