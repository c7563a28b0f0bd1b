"""Static check of the library's gfx950 ISA: no instruction may touch a VGPR
that an LDS read (ds_read*) or a vector memory load is still filling.

Several kernels issue LDS reads from inline asm and wait for them with their
own `s_waitcnt lgkmcnt(N)`, so the compiler does not know when a read's
destination registers hold the data.  It may then copy such a register
(`v_mov`), or reuse it, between the read and its wait, and the copy takes
whatever the register held before.  Whether the data has landed by then is a
matter of timing, so tests can pass while the code is wrong.  This check
follows the control-flow graph of every kernel and models `lgkmcnt` as LDS
reads completing in issue order (a wait for at most N outstanding retires
all but the newest N reads), and `vmcnt` the same way for vector memory
loads (global_load*, buffer_load*).  Every LDS read and vector load takes a
place in its counter's order, but only those issued by inline asm have their
destinations tracked: the compiler waits for its own loads itself (the
LDS-DMA forms have no destination registers).  A read whose
destination or address registers are in flight, or any other instruction
that reads or writes them, is a violation.  Scalar-memory loads and LDS
writes also count against lgkmcnt, and vector stores against vmcnt; leaving
them out of the model only keeps more loads in flight, so the check stays
conservative.

Used by build.py on every .hip source; `python -m jules_amd.isa_check file.s`
checks an assembly file by hand.
"""
import re
import sys

_RANGE = re.compile(r"\b([va])\[(\d+):(\d+)\]")
_ONE = re.compile(r"\b([va])(\d+)\b")
_WAIT = re.compile(r"lgkmcnt\((\d+)\)")
_VMWAIT = re.compile(r"vmcnt\((\d+)\)")
_VMEM_LOAD = ("global_load", "buffer_load", "flat_load")
_KERNEL = re.compile(r"^(_Z\S+):")
_MAX_TRACKED = 64


def _regs(operands):
    """The vector and accumulation registers an operand list names."""
    out = set()
    for m in _RANGE.finditer(operands):
        out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    for m in _ONE.finditer(_RANGE.sub("", operands)):
        out.add(f"{m.group(1)}{m.group(2)}")
    return out


def _blocks(lines):
    """Split one function's lines into basic blocks:
    [(label, [(line_no, mnemonic, operands, issued_by_asm)], falls_through)]."""
    blocks = []
    label, body = "__entry__", []
    in_asm = False
    for ln, raw in lines:
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        t = raw.split(";")[0].strip()
        if not t or (t.startswith(".") and not t.endswith(":")):
            continue
        if t.endswith(":"):
            blocks.append((label, body, True))
            label, body = t[:-1], []
            continue
        parts = t.split(None, 1)
        mn, ops = parts[0], (parts[1] if len(parts) > 1 else "")
        body.append((ln, mn, ops, in_asm))
        if mn.startswith(("s_branch", "s_cbranch", "s_setpc")) or mn == "s_endpgm":
            ends = mn.startswith(("s_branch", "s_setpc")) or mn == "s_endpgm"
            blocks.append((label, body, not ends))
            label, body = f"__after_{ln}", []
    blocks.append((label, body, False))
    return blocks


def _merge1(a, b):
    """Join two in-flight queues (oldest first) aligned at the newest read."""
    n = max(len(a), len(b))
    a = [frozenset()] * (n - len(a)) + a
    b = [frozenset()] * (n - len(b)) + b
    return [x | y for x, y in zip(a, b)][-_MAX_TRACKED:]


def _merge(a, b):
    """Join two (LDS queue, vector memory queue) states."""
    return (_merge1(a[0], b[0]), _merge1(a[1], b[1]))


def _retire(q, n):
    """A wait for at most n outstanding: all but the newest n have completed."""
    return q[len(q) - n:] if len(q) > n else q


def check_function(lines):
    """[(line_no, text)] of the violations in one function's assembly lines."""
    blocks = _blocks(lines)
    index = {b[0]: i for i, b in enumerate(blocks)}
    succ = []
    for i, (_, body, falls) in enumerate(blocks):
        s = []
        if body and body[-1][1].startswith(("s_branch", "s_cbranch")):
            target = body[-1][2].split()[0] if body[-1][2].split() else ""
            if target in index:
                s.append(index[target])
        if falls and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)
    state = {0: ([], [])}
    work = [0]
    bad = set()
    while work:
        i = work.pop()
        q, v = list(state[i][0]), list(state[i][1])
        for ln, mn, ops, asm in blocks[i][1]:
            if mn.startswith("s_waitcnt"):
                m = _WAIT.search(ops)
                if m:
                    q = _retire(q, int(m.group(1)))
                m = _VMWAIT.search(ops)
                if m:
                    v = _retire(v, int(m.group(1)))
                continue
            lds = mn.startswith(("ds_read", "ds_load"))
            vmem = mn.startswith(_VMEM_LOAD)
            if lds or vmem:
                fields = [f.strip() for f in ops.split(",")]
                to_lds = vmem and ("_lds_" in mn or re.search(r"\blds\b", ops) is not None)
                dst = _regs(fields[0]) if asm and not to_lds else set()
                src = set()
                for f in (fields if to_lds else fields[1:]):
                    src |= _regs(f)
                if any((src | dst) & r for r in q + v):
                    bad.add((ln, f"{mn} {ops}".strip()))
                if lds or mn.startswith("flat_load"):
                    q = (q + [frozenset(dst)])[-_MAX_TRACKED:]
                if vmem:
                    v = (v + [frozenset(dst)])[-_MAX_TRACKED:]
                continue
            if any(_regs(ops) & r for r in q + v):
                bad.add((ln, f"{mn} {ops}".strip()))
        q = (q, v)
        for j in succ[i]:
            new = _merge(state[j], q) if j in state else q
            if j not in state or new != state[j]:
                state[j] = new
                work.append(j)
    return sorted(bad)


def check_asm(text):
    """{kernel symbol: [(line_no, text)]} for every function with violations."""
    found = {}
    name, body = None, []
    for ln, line in enumerate(text.splitlines(), 1):
        m = _KERNEL.match(line)
        if m:
            name, body = m.group(1), []
            continue
        if name is None:
            continue
        body.append((ln, line))
        if line.strip().startswith(".Lfunc_end"):
            bad = check_function(body)
            if bad:
                found[name] = bad
            name = None
    return found


if __name__ == "__main__":
    total = 0
    for path in sys.argv[1:]:
        with open(path) as f:
            res = check_asm(f.read())
        for k, v in res.items():
            for ln, t in v[:5]:
                print(f"{path}:{ln}: {k[:60]}: {t}")
            total += len(v)
    print("violations:", total)
    sys.exit(1 if total else 0)
