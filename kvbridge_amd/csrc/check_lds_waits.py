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


def scan_function(lines):
    """Findings (line index, instruction) in one function's assembly lines."""
    pending = []  # (dest registers of an LDS read, or empty for other lgkm ops), oldest first
    found = []
    for i, raw in enumerate(lines):
        t = raw.split(";")[0].strip()
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        if t.startswith("s_waitcnt"):
            w = _WAIT.search(t)
            if w is not None:
                keep = int(w.group(1))
                pending = pending[len(pending) - keep:] if keep < len(pending) else pending
                if keep == 0:
                    pending = []
            continue
        if t.startswith(("s_endpgm", "s_branch", "s_cbranch", "s_setpc", "s_barrier")) and not pending:
            continue
        live = set().union(*[p for p in pending]) if pending else set()
        if live:
            ops = t.split(None, 1)
            if len(ops) == 2 and any(_regs(m) & live for m in _VREG.finditer(ops[1])):
                found.append((i, t))
        if _LGKM.match(t):
            d = _VDST.match(t) if t.startswith("ds_read") else None
            pending.append(_regs(d) if d else set())
    return found


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
