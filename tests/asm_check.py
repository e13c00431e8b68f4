"""Static check of compiled gfx950 assembly: no instruction may read or write
a VGPR that a still-pending global/buffer load is filling.

Kernels that issue loads as inline asm place their vmcnt waits by hand; a
miscounted wait lets code use (or reuse, e.g. as an address) a register the
load has not written yet. vmcnt counts vector memory operations in issue
order, so after `s_waitcnt vmcnt(n)` only the n most recent ones may still be
in flight. The walk is linear (branch-free hot paths), which is what the
kernels checked here are.
"""
import re

_RANGE = re.compile(r"v\[(\d+):(\d+)\]")
_ONE = re.compile(r"v(\d+)")


def _regs(tok):
    m = _RANGE.fullmatch(tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _ONE.fullmatch(tok)
    return {int(m.group(1))} if m else set()


def check_kernel(lines):
    """lines: assembly lines of one kernel. Returns a list of violations."""
    pending = []  # (registers, line) per outstanding vector memory op, oldest first
    bad = []
    for ln, line in lines:
        s = line.split(";")[0].strip()
        if not s or s.endswith(":") or s.startswith("."):
            continue
        parts = s.replace(",", " ").split()
        op, ops = parts[0], parts[1:]
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", s)
            if m:
                n = int(m.group(1))
                pending = pending[len(pending) - n:] if len(pending) > n else pending
            continue
        touched = set().union(*[_regs(o) for o in ops]) if ops else set()
        for regs, at in pending:
            if regs & touched:
                bad.append((ln, s, at))
        if op.startswith("global_load_lds") or (op.startswith("buffer_load") and " lds" in s):
            pending.append((set(), ln))  # DMA into LDS: no destination VGPR
        elif op.startswith(("global_load", "buffer_load", "flat_load")):
            pending.append((_regs(ops[0]), ln))
        elif op.startswith(("global_store", "buffer_store", "global_atomic", "buffer_atomic", "flat_store", "flat_atomic")):
            pending.append((set(), ln))
    return bad


def check_file(text, name_filter=""):
    """Returns {kernel name: violations} for kernels whose name contains name_filter."""
    out, cur, buf = {}, None, []
    for i, l in enumerate(text.splitlines(), 1):
        m = re.match(r"^(_Z\S+):", l)
        if m:
            cur, buf = m.group(1), []
            continue
        if cur:
            buf.append((i, l))
            if "s_endpgm" in l:
                if name_filter in cur:
                    out[cur] = check_kernel(buf)
                cur = None
    return out
