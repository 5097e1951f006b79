"""Checks compiled gfx950 assembly for LDS loads whose results are used
before they have arrived.

The pipelined prefill GEMM issues some LDS reads as inline asm (the
compiler cannot tell its DMA ring slots apart and would otherwise wait for
every DMA in flight before each read).  The compiler does not know such an
asm result is still in flight, so it must not copy, read or overwrite the
destination registers before the s_waitcnt lgkmcnt that retires the load.
This scans every function whose name matches a pattern and reports any
instruction that touches the VGPRs of a pending ds_read (LDS operations
retire in issue order, so lgkmcnt(n) retires all but the newest n).

usage: python tests/lds_wait_check.py file.s [name-substring]
"""
import re
import sys


def _regs(tok):
    m = re.fullmatch(r"[va]\[(\d+):(\d+)\]", tok)
    if m:
        pre = tok[0]
        return {(pre, i) for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


def check_function(lines):
    """Returns the list of (line number, text) hazards in one function."""
    pend = []
    bad = []
    for ln, raw in lines:
        t = raw.split(";")[0].strip()
        if not t or t.endswith(":") or t.startswith("."):
            continue
        op, _, rest = t.partition(" ")
        ops = [o.strip().split()[0] for o in rest.split(",") if o.strip()] if rest else []
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", rest)
            if m:
                n = int(m.group(1))
                pend = pend[len(pend) - n:] if 0 < n < len(pend) else ([] if n == 0 else pend)
            continue
        if op.startswith("s_load") or op.startswith("s_buffer_load"):
            pend.append(set())
            continue
        if op.startswith("s_"):
            continue
        live = set().union(*pend) if pend else set()
        touched = set().union(*[_regs(o) for o in ops]) if ops else set()
        if touched & live:
            bad.append((ln, t))
        if op.startswith("ds_read"):
            pend.append(_regs(ops[0]) if ops else set())
        elif op.startswith("ds_"):
            pend.append(set())
    return bad


def check_file(path, pattern=""):
    """{function name: hazards} for the functions whose name contains pattern."""
    funcs, cur = {}, None
    for i, line in enumerate(open(path).read().splitlines(), 1):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is not None:
            funcs[cur].append((i, line))
            if "s_endpgm" in line:
                cur = None
    return {f: check_function(ls) for f, ls in funcs.items() if pattern in f}


if __name__ == "__main__":
    res = check_file(sys.argv[1], sys.argv[2] if len(sys.argv) > 2 else "")
    n = 0
    for f, bad in res.items():
        for ln, t in bad:
            print(f"{f}:{ln}: {t}")
        n += len(bad)
        print(f"{f}: {'ok' if not bad else str(len(bad)) + ' hazards'}")
    sys.exit(1 if n else 0)
