"""Static check of compiled gfx950 assembly: no instruction may read or write
a VGPR that a still-pending global/buffer load is filling.

Kernels that issue loads as inline asm place their vmcnt waits by hand; a
miscounted wait lets code use (or reuse, e.g. as an address) a register the
load has not written yet. vmcnt counts vector memory operations in issue
order, so after `s_waitcnt vmcnt(n)` only the n most recent ones may still be
in flight; LDS reads (inline-asm fragment loads) count the same way under
lgkmcnt. The pending queues are propagated over the kernel's control-flow
graph, so every path to an instruction is checked.
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


_WAIT = re.compile(r"(vmcnt|lgkmcnt)\((\d+)\)")
_CAP = 64  # longest pending queue tracked (hardware counters are smaller)
# Largest count lgkmcnt's 4-bit field can express on gfx950. A path that
# leaves more LDS reads (operations that fill registers) outstanding than that
# relies on how the counter behaves past its field, so it is reported. LDS
# writes are not counted: the compiler itself issues long runs of them and
# drains them with a full wait. (vmcnt has 6 bits; the deepest hand-placed
# vector-load queue here is 32, and loops of LDS DMAs with run-time trip
# counts make a static vmcnt depth meaningless, so it is not checked.)
_LG_LIMIT = 15


def _loads(q):
    return sum(1 for regs, _ in q if regs)


def _parse(lines):
    """Instructions and basic blocks of one kernel: returns (insts, blocks,
    label index) with insts = [(line number, text)], blocks = [(first, end)]
    (end exclusive) and the successor rule applied in _succ."""
    insts, labels = [], {}
    for ln, line in lines:
        s = line.split(";")[0].strip()
        if not s or s.startswith("."):
            m = re.match(r"^(\.L\w+):", s)
            if m:
                labels[m.group(1)] = len(insts)
            continue
        if s.endswith(":"):
            labels[s[:-1]] = len(insts)
            continue
        insts.append((ln, s))
    starts = {0} | set(labels.values())
    for k, (_, s) in enumerate(insts):
        if s.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            starts.add(k + 1)
    starts = sorted(x for x in starts if x < len(insts))
    blocks = [(a, b) for a, b in zip(starts, starts[1:] + [len(insts)])]
    return insts, blocks, labels


def _succ(insts, blocks, labels, bi):
    a, b = blocks[bi]
    s = insts[b - 1][1]
    op = s.split()[0]
    nxt = [bi + 1] if bi + 1 < len(blocks) else []
    start_of = {blk[0]: k for k, blk in enumerate(blocks)}
    if op == "s_branch":
        return [start_of[labels[s.split()[1]]]]
    if op.startswith("s_cbranch"):
        return [start_of[labels[s.split()[1]]]] + nxt
    if op in ("s_endpgm", "s_setpc_b64"):
        return []
    return nxt


def _classify(op, s):
    """(queue, destination operand index or None) of a memory instruction, or
    None. Queues: 'vm' (vector memory, completes in issue order) and 'lg'
    (LDS and scalar memory)."""
    if op.startswith("global_load_lds") or (op.startswith("buffer_load") and " lds" in s):
        return ("vm", None)  # DMA into LDS: no destination VGPR
    if op.startswith(("global_load", "buffer_load", "scratch_load")):
        return ("vm", 0)
    if op.startswith("flat_load"):
        return ("vmlg", 0)
    if op.startswith(("global_store", "buffer_store", "scratch_store", "global_atomic",
                      "buffer_atomic", "flat_store", "flat_atomic")):
        return ("vm", None)
    if op.startswith("ds_"):
        if op.startswith(("ds_write", "ds_store")) or op in ("ds_nop",):
            return ("lg", None)
        return ("lg", 0)  # ds_read / ds_load / ds_bpermute / returning atomics
    if op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_dcache")):
        return ("lg", None)
    return None


def _merge(x, y):
    """Pending queues of two paths, aligned at the newest entry: entry i from
    the end holds the union of both paths' entries (so a wait that keeps n
    entries is sound for both)."""
    n = max(len(x), len(y))
    out = []
    for i in range(n, 0, -1):
        a = x[-i] if i <= len(x) else None
        b = y[-i] if i <= len(y) else None
        if a is None:
            out.append(b)
        elif b is None:
            out.append(a)
        else:
            out.append((a[0] | b[0], min(a[1], b[1])))
    return tuple(out[-_CAP:])


_SPAIR = re.compile(r"^(s\[\d+:\d+\]|vcc)$")


_TRACKED = set()  # flag pairs the current kernel feeds to s_and(n)2_b64 vcc, exec, X


def _flags(consts, op, ops):
    """Known values of 64-bit scalar flags: the compiler lowers an if/else that
    both paths share into `s_mov_b64 sX, -1|0` then `s_and(n2)_b64 vcc, exec,
    sX` and `s_cbranch_vcc(n)z`. Tracking those constants keeps a path's waits
    tied to the branch it takes."""
    d = dict(consts)
    dst = ops[0] if ops else ""
    if op == "s_mov_b64" and dst in _TRACKED and len(ops) > 1 and ops[1] in ("-1", "0"):
        d[dst] = int(ops[1])
    elif op in ("s_and_b64", "s_andn2_b64") and dst == "vcc" and len(ops) > 2 and ops[1] == "exec":
        v = d.get(ops[2])
        d.pop("vcc", None)
        if v is not None:
            nz = (v == -1) if op == "s_and_b64" else (v == 0)
            d["vcc"] = "nz" if nz else "z"
    else:
        if op.startswith("v_cmp") or dst == "vcc":
            d.pop("vcc", None)
        w = _sregs(dst)
        if w:
            for k in [k for k in d if k != "vcc" and _sregs(k) & w]:
                d.pop(k)
    return tuple(sorted(d.items()))


def _sregs(tok):
    """Scalar registers named by an operand (sN or s[a:b])."""
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _step(state, ln, s, bad):
    vm, lg, consts = state
    parts = s.replace(",", " ").split()
    op, ops = parts[0], parts[1:]
    if op == "s_waitcnt":
        for kind, n in _WAIT.findall(s):
            n = int(n)
            if kind == "vmcnt":
                vm = vm[len(vm) - n:] if len(vm) > n else vm
            else:
                lg = lg[len(lg) - n:] if len(lg) > n else lg
        return (vm, lg, consts)
    if op.startswith("s_"):
        consts = _flags(consts, op, ops)
    elif op.startswith("v_cmp"):
        consts = _flags(consts, op, ops)
    cls = _classify(op, s)
    dest = set()
    if cls and cls[1] is not None and ops:
        dest = _regs(ops[0])
        srcs = ops[1:]
    else:
        srcs = ops
    touched = set().union(*[_regs(o) for o in srcs]) if srcs else set()
    for qname, q in (("vm", vm), ("lg", lg)):
        # a load's destination may overlap pending loads of its own queue
        # (same-queue results land in issue order); anything else may not
        hit = touched | (dest if not (cls and qname in cls[0]) else set())
        for regs, at in q:
            if regs & hit:
                bad.append((ln, s, at))
                break
    if cls:
        entry = (frozenset(dest), ln)
        if "vm" in cls[0]:
            vm = (vm + (entry,))[-_CAP:]
        if "lg" in cls[0]:
            lg = (lg + (entry,))[-_CAP:]
            if dest and _loads(lg) > _LG_LIMIT:
                bad.append((ln, s, "lgkmcnt overflow"))
    return (vm, lg, consts)


def _feasible(state, insts, blocks, labels, bi):
    """Successor blocks of block bi that the state's known flags allow."""
    succ = _succ(insts, blocks, labels, bi)
    s = insts[blocks[bi][1] - 1][1]
    op = s.split()[0]
    vcc = dict(state[2]).get("vcc")
    if vcc is not None and op in ("s_cbranch_vccnz", "s_cbranch_vccz") and len(succ) == 2:
        taken = (vcc == "nz") == (op == "s_cbranch_vccnz")
        return [succ[0]] if taken else [succ[1]]
    return succ


_MAXSTATES = 128  # distinct flag sets kept per block before all are merged


def _join(states):
    """States reaching one block: those with the same known flags have their
    queues merged (the flags are what ties a wait to a branch); past
    _MAXSTATES flag sets everything is merged into one state."""
    by = {}
    for vm, lg, c in states:
        if c in by:
            ovm, olg = by[c]
            by[c] = (_merge(ovm, vm), _merge(olg, lg))
        else:
            by[c] = (vm, lg)
    if len(by) > _MAXSTATES:
        vm, lg = (), ()
        for ovm, olg in by.values():
            vm, lg = _merge(vm, ovm), _merge(lg, olg)
        return {(vm, lg, ())}
    return {(vm, lg, c) for c, (vm, lg) in by.items()}


def check_kernel(lines):
    """lines: [(line number, text)] of one kernel. Returns the violations
    [(line, instruction, line of the pending load)]: instructions that read or
    overwrite a VGPR a still-pending load (vector memory under vmcnt, LDS
    under lgkmcnt) is filling. Sets of pending-queue states are propagated
    over the control-flow graph to a fixed point (loops included), with the
    compiler's constant branch flags tracked so that a wait placed on one
    side of an if/else is credited to the path that took it."""
    insts, blocks, labels = _parse(lines)
    if not insts:
        return []
    _TRACKED.clear()
    for _, s in insts:
        p = s.replace(",", " ").split()
        if p[0] in ("s_and_b64", "s_andn2_b64") and len(p) > 3 and p[1] == "vcc" and p[2] == "exec":
            _TRACKED.add(p[3])
    entry = {0: {((), (), ())}}
    work = [0]
    while work:
        bi = work.pop()
        a, b = blocks[bi]
        outs = {}
        for st in entry[bi]:
            for ln, s in insts[a:b]:
                st = _step(st, ln, s, [])
            for nb in _feasible(st, insts, blocks, labels, bi):
                outs.setdefault(nb, set()).add(st)
        for nb, sts in outs.items():
            old = entry.get(nb, set())
            new = _join(old | sts)
            if new != old:
                entry[nb] = new
                work.append(nb)
    bad = []
    for bi, sts in sorted(entry.items()):
        a, b = blocks[bi]
        for st in sts:
            for ln, s in insts[a:b]:
                st = _step(st, ln, s, bad)
    return sorted(set(bad))


def check_file(text, name_filter=""):
    """Returns {kernel name: violations} for kernels whose name contains name_filter."""
    out, cur, buf = {}, None, []
    for i, l in enumerate(text.splitlines(), 1):
        m = re.match(r"^(_Z\S+):", l)
        if m:
            cur, buf = m.group(1), []
            continue
        if cur:
            if l.startswith(".Lfunc_end"):  # a kernel may hold several s_endpgm
                if name_filter in cur:
                    out[cur] = check_kernel(buf)
                cur = None
                continue
            buf.append((i, l))
    return out
