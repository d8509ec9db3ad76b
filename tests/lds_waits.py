"""A check of generated AMDGPU assembly: no instruction touches the
destination registers of a ds_read before an s_waitcnt lgkmcnt has retired
that read, on any path through the function.

The product kernels issue their LDS fragment reads as inline asm and wait for
them with explicit lgkmcnt waits, so that the reads overlap the MFMAs. The
compiler treats an asm's outputs as ready when the asm ends: if register
pressure makes it copy or reuse a destination before the wait, the copy holds
whatever the register held before the LDS data arrived. This module finds such
accesses by dataflow over the function's control-flow graph: for every read
still in flight it tracks the fewest LGKM operations issued after it on any
path; s_waitcnt lgkmcnt(k) retires the reads with at least k younger ones.
"""
import re

_CAP = 16        # lgkmcnt is four bits: a read with 16 younger ops is retired by any wait


def _regs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _blocks(body):
    ins = []
    for line in body:
        t = line.split(";")[0].strip()
        if not t:
            continue
        if t.startswith(".") and not re.match(r"^\.LBB\d+_\d+:", t):
            continue
        ins.append(t)
    blocks, cur = [], []
    for t in ins:
        if re.match(r"^\.LBB\d+_\d+:", t):
            if cur:
                blocks.append(cur)
            cur = [t]
            continue
        cur.append(t)
        op = t.split()[0]
        if op.startswith("s_cbranch") or op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            blocks.append(cur)
            cur = []
    if cur:
        blocks.append(cur)
    labels = {b[0][:-1]: i for i, b in enumerate(blocks) if b and b[0].endswith(":")}
    succ = []
    for i, b in enumerate(blocks):
        last = b[-1] if b else ""
        op = last.split()[0] if last else ""
        s = []
        if op.startswith("s_cbranch") or op == "s_branch":
            m = re.search(r"(\.LBB\d+_\d+)", last)
            if m and m.group(1) in labels:
                s.append(labels[m.group(1)])
        if op not in ("s_branch", "s_endpgm", "s_setpc_b64") and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)
    return blocks, succ


def _run(block, bi, state, report=None):
    st = dict(state)             # read id -> (younger LGKM ops, destination registers)
    for k, t in enumerate(block):
        if t.endswith(":"):
            continue
        op = t.split()[0]
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", t)
            if m:
                n = int(m.group(1))
                st = {i: v for i, v in st.items() if v[0] < n}
            continue
        operands = t[len(op):]
        if op.startswith("ds_read"):
            # LDS returns in issue order: a later read may target a pending
            # read's registers; only its address must not be one of them
            used = _regs(operands.split(",", 1)[1] if "," in operands else "")
        else:
            used = _regs(operands)
        if report is not None:
            for i, (_, dest) in st.items():
                if dest and used & dest:
                    report.append((t, i))
        if op.startswith("ds_") or op.startswith("s_load") or op.startswith("s_buffer_load"):
            st = {i: (min(y + 1, _CAP), d) for i, (y, d) in st.items()}
            dest = _regs(t[len(op):].split(",")[0]) if op.startswith("ds_read") else None
            st[(bi, k)] = (0, dest)
    return st


def violations(body):
    """The (instruction, read) pairs of one function's assembly lines where an
    instruction touches a read's destination before a wait retires it."""
    blocks, succ = _blocks(body)
    if not blocks:
        return []
    entry = [None] * len(blocks)
    entry[0] = {}
    work = [0]
    while work:
        bi = work.pop()
        st = _run(blocks[bi], bi, entry[bi])
        for s in succ[bi]:
            if entry[s] is None:
                new = st
            else:
                new = dict(entry[s])
                for i, (y, d) in st.items():
                    new[i] = (min(y, new[i][0]), d) if i in new else (y, d)
            if entry[s] is None or new != entry[s]:
                entry[s] = new
                work.append(s)
    report = []
    for bi, b in enumerate(blocks):
        if entry[bi] is not None:
            _run(b, bi, entry[bi], report)
    return report


def functions(asm_text, name_pattern):
    """{symbol: body lines} for the functions whose symbol matches name_pattern."""
    lines = asm_text.split("\n")
    out = {}
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S+):", line)
        if m and re.search(name_pattern, m.group(1)):
            end = next(j for j in range(i + 1, len(lines)) if lines[j].startswith(".Lfunc_end"))
            out[m.group(1)] = lines[i + 1:end]
    return out
