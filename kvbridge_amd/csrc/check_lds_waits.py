"""Static check of the kernels' device assembly: no instruction may read or
overwrite the destination register of an LDS read (ds_read*) before an
s_waitcnt that covers that read.

The kernels issue some LDS reads from inline asm (the reads are invisible to
the compiler's own wait insertion).  Were such a read's wait emitted later
than the read, the compiler could copy or reuse its destination before the
data lands -- silent garbage.  LDS-counter (lgkmcnt) operations complete in
issue order for this purpose, so s_waitcnt lgkmcnt(N) retires all but the N
most recent pending operations; every DS operation (LDS writes included),
scalar memory loads and messages count too.

Usage: python check_lds_waits.py FILE.s ...   (exit status 1 on findings)
The assembly comes from `make -C kvbridge_amd/csrc asm` (the build's flags).
"""
import re
import sys

_LGKM = re.compile(r"^(ds_\w+|s_load\w*|s_buffer_load\w*|s_sendmsg\w*)\s")  # every op the LDS counter counts
_VDST = re.compile(r"^\S+\s+(?:v\[(\d+):(\d+)\]|v(\d+))")
_VREG = re.compile(r"v\[(\d+):(\d+)\]|(?<![a-z_])v(\d+)")
_WAIT = re.compile(r"lgkmcnt\((\d+)\)")


def _regs(m):
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


_LABEL = re.compile(r"^(\.LBB\w+):")
_TARGET = re.compile(r"^s_c?branch\w*\s+(\.LBB\w+)")
_MAX_PENDING = 15  # the LDS counter's range: the wave cannot have more in flight


def _merge(a, b):
    """Pending lists of two paths, aligned at the youngest entry: a register
    counts as pending at a position if it is on either path."""
    n = max(len(a), len(b))
    a = [frozenset()] * (n - len(a)) + a
    b = [frozenset()] * (n - len(b)) + b
    return [x | y for x, y in zip(a, b)]


def scan_function(lines):
    """Findings (line index, instruction) in one function's assembly lines.

    Follows the control-flow graph (labels, branches, fall-through): each
    block starts from the merge of the pending LDS operations its
    predecessors end with, so code that a branch skips or that runs out of
    line is checked against the paths that actually reach it."""
    # basic blocks: (first line, [(line index, instruction)], successor labels, falls through)
    blocks, cur, labels = [], None, {}
    for i, raw in enumerate(lines):
        t = raw.split(";")[0].strip()
        m = _LABEL.match(t)
        if m:
            if cur is not None:
                blocks.append(cur)
            cur = {"label": m.group(1), "ins": [], "succ": [], "falls": True}
            labels[m.group(1)] = len(blocks)
            continue
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        if cur is None:
            cur = {"label": None, "ins": [], "succ": [], "falls": True}
        cur["ins"].append((i, t))
        tm = _TARGET.match(t)
        if tm:
            cur["succ"].append(tm.group(1))
            if t.startswith("s_branch"):
                cur["falls"] = False
        if t.startswith(("s_endpgm", "s_setpc")):
            cur["falls"] = False
        if tm or t.startswith(("s_endpgm", "s_setpc")):
            blocks.append(cur)
            cur = {"label": None, "ins": [], "succ": [], "falls": True}
    if cur is not None:
        blocks.append(cur)
    for k, b in enumerate(blocks):  # labels of blocks split at a branch
        if b["label"] is not None:
            labels[b["label"]] = k

    def run(block, pending, found):
        for i, t in block["ins"]:
            if t.startswith("s_waitcnt"):
                w = _WAIT.search(t)
                if w is not None:
                    keep = int(w.group(1))
                    pending = pending[len(pending) - keep:] if 0 < keep < len(pending) else ([] if keep == 0 else pending)
                continue
            live = frozenset().union(*pending) if pending else frozenset()
            if live:
                ops = t.split(None, 1)
                if len(ops) == 2 and any(_regs(m) & live for m in _VREG.finditer(ops[1])):
                    found.append((i, t))
            if _LGKM.match(t):
                d = _VDST.match(t) if t.startswith("ds_read") else None
                pending = (pending + [frozenset(_regs(d)) if d else frozenset()])[-_MAX_PENDING:]
        return pending

    entry = {0: []}
    work = [0] if blocks else []
    while work:  # fixed point of the block entry states
        k = work.pop()
        out = run(blocks[k], entry[k], [])
        succ = [labels[x] for x in blocks[k]["succ"] if x in labels]
        if blocks[k]["falls"] and k + 1 < len(blocks):
            succ.append(k + 1)
        for j in succ:
            new = out if j not in entry else _merge(entry[j], out)
            if j not in entry or new != entry[j]:
                entry[j] = new
                work.append(j)
    found = []
    for k in sorted(entry):
        run(blocks[k], entry[k], found)
    return sorted(set(found))


def scan_asm(text):
    """{function name: findings} for every function in an assembly file."""
    out = {}
    starts = [(m.start(), m.group(1)) for m in re.finditer(r"^(_Z\w+):", text, re.M)]
    for k, (pos, name) in enumerate(starts):
        end = text.find(".Lfunc_end", pos)
        body = text[pos:end if end >= 0 else len(text)].split("\n")[1:]
        f = scan_function(body)
        if f:
            out[name] = f
    return out


def main(paths):
    bad = 0
    for p in paths:
        for name, f in scan_asm(open(p).read()).items():
            bad += len(f)
            print(f"{p}: {name}: {len(f)} use(s) of an LDS read's register before its wait, e.g. {f[0][1]}")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
