"""Static check of the generated gfx950 assembly for in-flight register hazards.

Kernels that issue their loads as inline assembly and wait with explicit
``s_waitcnt vmcnt(N)`` rely on nothing touching a load's destination registers
until a wait has retired it. This script simulates the in-order vector-memory
counter over each kernel's instruction list (twice back to back, so that loads
pending at the end of a loop body meet the loop top) and reports every read or
write of a destination register whose load is still outstanding.

    python -m sglang_restomod_amd.isa_check file.s   (exit status 1 on any hazard)
"""
import re, sys

def regs(tok):
    tok = tok.strip().rstrip(',')
    m = re.match(r'([va])\[(\d+):(\d+)\]', tok)
    if m: return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r'([va])(\d+)$', tok)
    if m: return {tok}
    return set()

def check(body, name):
    """Simulate the vector-memory counter over `body`; return the hazard count."""
    pending = []  # list of (seq, dst_regs, text)
    issued = 0
    problems = 0
    for ln, line in enumerate(body):
        t = line.strip()
        if not t or t.startswith(('.', ';')) or t.endswith(':'): continue
        op = t.split()[0]
        m = re.match(r's_waitcnt\s+vmcnt\((\d+)\)', t)
        if m:
            n = int(m.group(1))
            # in-order: all but the last n outstanding ops retire
            if len(pending) > n: pending = pending[len(pending) - n:] if n else []
            continue
        if op.startswith(('s_endpgm', 's_branch', 's_cbranch', 's_setpc')):
            continue
        args = t[len(op):].split(',')
        is_vm = op.startswith(('global_load', 'global_store', 'buffer_', 'flat_', 'scratch_', 'global_atomic'))
        # uses: all register operands of this instruction
        used = set()
        for a in args: used |= regs(a.split()[0] if a.split() else a)
        for (seq, dst, txt) in pending:
            if dst & used:
                problems += 1
                if problems <= 10:
                    print(f"{name}: line {ln}: '{t}' touches {sorted(dst & used)} of in-flight '{txt}'")
        if is_vm:
            dst = set()
            if op.startswith(('global_load', 'buffer_load', 'flat_load', 'scratch_load')) and 'lds' not in op:
                dst = regs(args[0])
            pending.append((issued, dst, t))
            issued += 1
    return problems

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
    for name in re.findall(r"^(_ZN2ma\w*(?:partial|extend)\w*):", s, re.M):
        start = s.index(name + ":")
        end = s.index(".Lfunc_end", start)
        lines = s[start:end].splitlines()
        p = check(lines + lines, name[:50])
        if verbose:
            print(f"{name[:60]}: {p} hazards")
        total += p
    return total


if __name__ == "__main__":
    sys.exit(1 if check_file(sys.argv[1], verbose=True) else 0)
