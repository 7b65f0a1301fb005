"""Static checks of the generated gfx950 assembly.

In-flight register hazards: kernels that issue their loads as inline assembly
and wait with explicit ``s_waitcnt vmcnt(N)`` rely on nothing touching a load's
destination registers until a wait has retired it. ``check`` runs a forward
dataflow over each kernel's control-flow graph (basic blocks split at labels and
branches): the state maps every possibly outstanding load to the smallest number
of vector-memory instructions issued after it on any path, a wait ``vmcnt(N)``
retires the loads with at least N younger instructions (completion is in order),
paths merge by union with the minimum count, and a load with 63 younger
instructions has necessarily completed. Any instruction that reads, or writes
other than as a later load's destination, a destination register of a possibly
outstanding load is reported (loads return in issue order, so a later load into
the same register lands after it).

    python -m sglang_restomod_amd.isa_check file.s   (exit status 1 on any hazard)
"""
import re
import sys

VMEM = ('global_load', 'global_store', 'global_atomic', 'buffer_', 'flat_', 'scratch_')
LOADS = ('global_load', 'buffer_load', 'flat_load', 'scratch_load')


def regs(tok):
    tok = tok.strip().rstrip(',')
    m = re.match(r'([va])\[(\d+):(\d+)\]', tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r'([va])(\d+)$', tok)
    if m:
        return {tok}
    return set()


def _parse(body):
    """Instructions (text) and label -> instruction index."""
    insts, labels = [], {}
    for line in body:
        t = line.split(';')[0].strip()
        if not t:
            continue
        if t.endswith(':'):
            labels[t[:-1]] = len(insts)
            continue
        if t.startswith('.'):
            continue
        insts.append(t)
    return insts, labels


def _blocks(insts, labels):
    """Basic blocks as (start, end) index pairs and their successor block indices."""
    leaders = {0} | set(labels.values())
    for i, t in enumerate(insts):
        if t.startswith(('s_branch', 's_cbranch', 's_endpgm', 's_setpc')):
            leaders.add(i + 1)
    starts = sorted(x for x in leaders if x < len(insts))
    index = {s: k for k, s in enumerate(starts)}
    blocks, succ = [], []
    for k, s0 in enumerate(starts):
        e = starts[k + 1] if k + 1 < len(starts) else len(insts)
        blocks.append((s0, e))
        last = insts[e - 1]
        op = last.split()[0]
        nxt = [index[e]] if e in index else []
        if op == 's_branch':
            succ.append([index[labels[last.split()[1]]]])
        elif op.startswith('s_cbranch'):
            succ.append([index[labels[last.split()[1]]]] + nxt)
        elif op.startswith(('s_endpgm', 's_setpc')):
            succ.append([])
        else:
            succ.append(nxt)
    return blocks, succ


def _step(state, t, hazards, idx):
    """Apply instruction `t` (index idx) to `state` {load_idx: (younger, dst, text)}."""
    m = re.search(r'vmcnt\((\d+)\)', t) if t.startswith('s_waitcnt') else None
    if m:
        n = int(m.group(1))
        return {k: v for k, v in state.items() if v[0] < n}
    op = t.split()[0]
    args = t[len(op):].split(',')
    used = set()
    is_load = op.startswith(LOADS) and 'lds' not in op
    for n, a in enumerate(args):
        if is_load and n == 0:
            continue  # a later load's destination: loads return in issue order, so its write lands last
        used |= regs(a.split()[0] if a.split() else a)
    for k, (younger, dst, txt) in state.items():
        if dst & used:
            hazards.add((idx, k, f"'{t}' touches {sorted(dst & used)} of in-flight '{txt}'"))
    if op.startswith(VMEM):
        state = {k: (v[0] + 1, v[1], v[2]) for k, v in state.items() if v[0] + 1 < 63}
        if op.startswith(LOADS) and 'lds' not in op:
            state[idx] = (0, regs(args[0]), t)
    return state


def _merge(a, b):
    out = dict(a)
    for k, v in b.items():
        out[k] = v if k not in out else (min(out[k][0], v[0]), v[1], v[2])
    return out


def check(body, name, verbose=True):
    """Dataflow over the kernel's blocks; return the number of distinct hazards."""
    insts, labels = _parse(body)
    if not insts:
        return 0
    blocks, succ = _blocks(insts, labels)
    ins = [None] * len(blocks)
    ins[0] = {}
    work = [0]
    hazards = set()
    while work:
        b = work.pop()
        state = ins[b]
        s0, e = blocks[b]
        for i in range(s0, e):
            state = _step(state, insts[i], hazards, i)
        for nb in succ[b]:
            merged = state if ins[nb] is None else _merge(ins[nb], state)
            if ins[nb] is None or merged != ins[nb]:
                ins[nb] = merged
                if nb not in work:
                    work.append(nb)
    if verbose:
        for i, (idx, k, msg) in enumerate(sorted(hazards)):
            if i >= 10:
                break
            print(f"{name}: instruction {idx}: {msg}")
    return len(hazards)

# Writes through the scalar data cache (scalar stores and atomics, and that cache's
# write-back / discard) must never appear in this library's kernels.
SCALAR_CACHE_WRITES = re.compile(r"^\s*(s_store|s_buffer_store|s_scratch_store|s_atomic|s_buffer_atomic|"
                                 r"s_dcache_wb|s_dcache_discard)\w*", re.M)


def scalar_cache_writes(path):
    """Lines of an assembly listing that write through the scalar data cache."""
    return [m.group(0).strip() for m in SCALAR_CACHE_WRITES.finditer(open(path).read())]


def check_file(path, verbose=False):
    """Return the number of hazards over all kernels of an assembly listing."""
    s = open(path).read()
    total = 0
    for name in re.findall(r"^(_ZN2ma\w*):", s, re.M):
        start = s.index(name + ":")
        end = s.index(".Lfunc_end", start)
        lines = s[start:end].splitlines()[1:]
        p = check(lines, name[:50])
        if verbose:
            print(f"{name[:60]}: {p} hazards")
        total += p
    return total


if __name__ == "__main__":
    sys.exit(1 if check_file(sys.argv[1], verbose=True) else 0)
