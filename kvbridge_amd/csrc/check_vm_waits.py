"""Static check of the hand-counted vector-memory waits in the device
assembly: a wait `s_waitcnt vmcnt(N) ; kvb-keep G` (lds_stream.h
wait_vm_keep) must leave no load of an older tile DMA group in flight than
the G most recent groups, on every path that reaches it.

N counts emitted instructions, which the source cannot see: if a toolchain
emitted fewer vector-memory instructions per tile than the kernel assumes,
such a wait would release a tile before its data landed (wrong results, no
fault).  Each tile's DMA group starts at an assembler comment `;kvb-dma-group`
(lds_stream.h dma_group_mark); every LDS-DMA load (`buffer_load_* ... lds`,
`global_load_lds_*`) after it belongs to that group until the next mark.
The vector-memory counter (vmcnt; on gfx9-family chips loads, stores and
atomics alike) retires in issue order, so `vmcnt(N)` completes all but the N
most recent operations.

The analysis follows the control-flow graph with a set of abstract states
per block entry, so paths are not merged.  Groups are aged by the marks (0 =
the group of the most recent mark); a state records, for each age g, how
many vector-memory operations were issued after the newest pending LDS-DMA
load of age >= g (a wait vmcnt(N) completes that load iff the number is at
least N).  Every
hand-written `s_waitcnt vmcnt(N)` with N > 0 (inside `;;#ASMSTART` /
`;;#ASMEND`) must carry a kvb-keep annotation; a wait without one, or one
that may leave in flight an LDS-DMA load issued before any mark, is
reported.

Usage: python check_vm_waits.py FILE.s ...   (exit status 1 on findings)
"""
import re
import sys

_LABEL = re.compile(r"^(\.LBB\w+):")
_TARGET = re.compile(r"^s_c?branch\w*\s+(\.LBB\w+)")
_VMEM = re.compile(r"^(buffer_|global_|flat_|scratch_|tbuffer_|image_)")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_KEEP = re.compile(r"kvb-keep\s+(\d+)")
_MARK = "kvb-dma-group"
MAX_PENDING = 63  # the counter's range: a wave cannot have more in flight
MAX_AGE = 64
UNMARKED = -2     # an LDS-DMA load issued before any group mark


def _is_dma(t):
    return (t.startswith("buffer_load") and re.search(r"\slds(\s|$)", t) is not None) or t.startswith("global_load_lds")


def parse(lines):
    """Basic blocks of one function: {"label", "ins": [(line, kind, text,
    arg)], "succ": [labels], "falls"}; kind is mark / wait / dma / vmem."""
    blocks, cur = [], None
    in_asm = False

    def new(label=None):
        return {"label": label, "ins": [], "succ": [], "falls": True}

    for i, raw in enumerate(lines):
        code, _, comment = raw.partition(";")
        t = code.strip()
        stripped = raw.strip()
        if stripped == ";;#ASMSTART":
            in_asm = True
            continue
        if stripped == ";;#ASMEND":
            in_asm = False
            continue
        m = _LABEL.match(t)
        if m:
            if cur is not None:
                blocks.append(cur)
            cur = new(m.group(1))
            continue
        if cur is None:
            cur = new()
        if in_asm and _MARK in raw:
            cur["ins"].append((i, "mark", stripped, None))
            continue
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        if t.startswith("s_waitcnt"):
            w = _VMCNT.search(t)
            if w is not None:
                k = _KEEP.search(comment)
                cur["ins"].append((i, "wait", t, (int(w.group(1)), in_asm, int(k.group(1)) if k else None)))
        elif t.startswith("s_swappc"):
            cur["ins"].append((i, "call", t, None))
        elif _VMEM.match(t):
            cur["ins"].append((i, "dma" if _is_dma(t) else "vmem", t, None))
        tm = _TARGET.match(t)
        if tm:
            cur["succ"].append(tm.group(1))
            if t.startswith("s_branch"):
                cur["falls"] = False
        if t.startswith(("s_endpgm", "s_setpc")):
            cur["falls"] = False
        if tm or t.startswith(("s_endpgm", "s_setpc")):
            blocks.append(cur)
            cur = new()
    if cur is not None:
        blocks.append(cur)
    return blocks


def _step(state, ins, findings, checked, ages):
    """Abstract transfer of one instruction.  state = (seen, after): seen =
    a mark was executed on the path; after[g] (g = 0 .. ages) = number of
    vector-memory operations issued after the newest pending LDS-DMA load
    whose group age is >= g, None if no such load is pending; after[ages + 1]
    the same for LDS-DMA loads issued before any mark.  A wait vmcnt(N)
    completes such a load iff at least N operations were issued after it."""
    seen, after = state
    line, kind, text, arg = ins
    if kind == "call":  # the callee's memory operations are not in this function's text
        findings.add((line, text, "calls another function: its vector-memory operations cannot be counted"))
        return seen, after
    if kind == "mark":  # every group gets one older: age >= g now means age >= g - 1 before
        return True, (after[0],) + after[0:ages] + (after[ages + 1],)
    if kind in ("dma", "vmem"):
        bump = tuple(None if x is None or x + 1 >= MAX_PENDING else x + 1 for x in after)
        if kind == "dma":  # the newest load of group age 0 (or an unmarked one)
            bump = bump[:ages + 1] + (0,) if not seen else (0,) + bump[1:]
        return seen, bump
    n, hand, keep = arg
    after = tuple(None if x is None or x >= n else x for x in after)
    if hand and n > 0:
        checked.add(line)
        if keep is None:
            findings.add((line, text, "hand-written vmcnt wait without a kvb-keep annotation"))
        elif after[ages + 1] is not None:
            findings.add((line, text, "reached with LDS-DMA loads issued before any DMA group mark"))
        elif after[min(keep, ages)] is not None and keep <= ages:
            findings.add((line, text, f"leaves a load of a DMA group older than the {keep} newest in flight"))
    return seen, after


def scan_function(lines):
    """(findings, number of hand-counted waits checked, DMA group sizes) for
    one function's assembly lines."""
    blocks = parse(lines)
    index = {b["label"]: k for k, b in enumerate(blocks) if b["label"] is not None}

    def succ(k):
        out = [index[x] for x in blocks[k]["succ"] if x in index]
        if blocks[k]["falls"] and k + 1 < len(blocks):
            out.append(k + 1)
        return out

    keeps = [ins[3][2] for b in blocks for ins in b["ins"] if ins[1] == "wait" and ins[3][2] is not None]
    ages = max(keeps, default=1)
    start = (False, (None,) * (ages + 2))
    entry = {0: {start}} if blocks else {}
    work = [(0, start)] if blocks else []
    findings, checked = set(), set()
    while work:  # one (block, entry state) at a time: states are never merged
        k, st = work.pop()
        for ins in blocks[k]["ins"]:
            st = _step(st, ins, findings, checked, ages)
        for j in succ(k):
            cur = entry.setdefault(j, set())
            if st not in cur:
                cur.add(st)
                work.append((j, st))
    # DMA instructions per group: from each mark, every path to the next
    # mark, counting LDS-DMA loads.
    sizes = set()
    for k, b in enumerate(blocks):
        for pos, ins in enumerate(b["ins"]):
            if ins[1] != "mark":
                continue
            stack, seen_states = [(k, pos + 1, 0)], set()
            while stack:
                bk, p, cnt = stack.pop()
                if (bk, p, cnt) in seen_states or cnt > 4 * MAX_PENDING:
                    continue
                seen_states.add((bk, p, cnt))
                ended = False
                for q in range(p, len(blocks[bk]["ins"])):
                    kind = blocks[bk]["ins"][q][1]
                    if kind == "mark":
                        sizes.add(cnt)
                        ended = True
                        break
                    if kind == "dma":
                        cnt += 1
                if ended:
                    continue
                for j in succ(bk):  # a path that ends without another mark gives no size
                    stack.append((j, 0, cnt))
    return sorted(findings), len(checked), sizes


def _hand_vmcnt(chunk):
    """Whether an inline-asm region of the function waits on vmcnt(N > 0)."""
    for m in re.finditer(r";;#ASMSTART\n(.*?);;#ASMEND", chunk, re.S):
        if any(int(w) > 0 for w in _VMCNT.findall(m.group(1))):
            return True
    return False


def scan_asm(text):
    """{function name: (findings, waits checked, DMA group sizes)} for every
    function with a hand-counted wait or a DMA group mark."""
    out = {}
    starts = [(m.start(), m.group(1)) for m in re.finditer(r"^(_Z\w+):", text, re.M)]
    for pos, name in starts:
        end = text.find(".Lfunc_end", pos)
        chunk = text[pos:end if end >= 0 else len(text)]
        if _MARK not in chunk and "kvb-keep" not in chunk and not _hand_vmcnt(chunk):
            continue  # nothing hand-counted in this function
        f, n, sizes = scan_function(chunk.split("\n")[1:])
        if f or n or sizes:
            out[name] = (f, n, sizes)
    return out


def main(paths):
    bad = 0
    for p in paths:
        for name, (f, n, sizes) in scan_asm(open(p).read()).items():
            print(f"{p}: {name}: {n} hand-counted wait(s), DMA group sizes {sorted(sizes)}, {len(f)} finding(s)")
            for line, text, why in f[:4]:
                print(f"    line {line + 1}: {text}: {why}")
            bad += len(f)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
