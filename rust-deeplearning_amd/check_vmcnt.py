"""Build check of the fused GEMV kernels' hand-counted load wait.

The activation prep of the fused GEMV kernels (csrc/gemv_fused.hip) loads x
with inline-asm `global_load_dwordx4 ..., off` instructions issued ahead of
the weight stream, then waits for them alone with an inline-asm
`s_waitcnt vmcnt(N)` (wait_prep_x): vector-memory loads complete in issue
order, so the x loads are done once at most N loads are outstanding -- if at
least N load instructions were issued after them.  The compiler does not
track inline-asm loads, so nothing else guards that count.

This script reads the device assembly the compiler emits for
csrc/gemv_fused.hip (`hipcc -S --offload-device-only`, inline asm between
`;;#ASMSTART` / `;;#ASMEND` markers) and checks, in every function, each
inline-asm `s_waitcnt vmcnt(N)` that follows asm x loads: at least N
vector-memory load instructions lie on every path from the last of those
loads to the wait.  Between them the compiler emits only forward branches
around divergent blocks (`s_cbranch_execz` to a label before the wait); a
load counts only outside every such skippable range, and a branch backwards,
out of the range, or into it from elsewhere fails the check.  It exits
non-zero, naming the function, when a wait does not hold.

Usage: python check_vmcnt.py build/gemv_fused.s
"""
import re
import sys

FUNC = re.compile(r"^([A-Za-z_][\w.$]*):\s*(;.*)?$")
LOAD = re.compile(r"^(buffer|global|flat|scratch)_load")
XLOAD = re.compile(r"^global_load_dwordx4\s+v\[\d+:\d+\],\s*v\[\d+:\d+\],\s*off$")
WAIT = re.compile(r"^s_waitcnt\s+vmcnt\((\d+)\)$")
CF = re.compile(r"^(s_cbranch|s_branch|s_setpc|s_swappc|s_endpgm)")
BLOCK = re.compile(r"^\.LBB\w*:")


def functions(lines):
    """(name, [lines]) of each function body (from its label to .Lfunc_end)."""
    name, body = None, []
    for line in lines:
        s = line.strip()
        m = FUNC.match(s)
        if m and not s.startswith(".") and m.group(1).startswith("_Z"):
            if name:
                yield name, body
            name, body = m.group(1), []
            continue
        if name is not None:
            if s.startswith(".Lfunc_end"):
                yield name, body
                name, body = None, []
            else:
                body.append(s)
    if name:
        yield name, body


BRANCH = re.compile(r"^(s_cbranch_\w+|s_branch)\s+(\.LBB\w+)")


def window_loads(body, lo, hi, targets_from):
    """Loads on every path through body[lo:hi] (or None: control flow the
    check does not accept).  targets_from: label -> positions of branches to it."""
    labels = {}
    for i in range(lo, hi):
        m = BLOCK.match(body[i])
        if m:
            labels[body[i][:-1]] = i
    skipped = []
    for i in range(lo, hi):
        s = body[i]
        m = BRANCH.match(s)
        if m:
            t = labels.get(m.group(2))
            if t is None or t <= i:
                return None  # out of the range, or backwards
            skipped.append((i, t))
        elif CF.match(s):
            return None  # s_endpgm / s_setpc / an indirect branch
    for lab, pos in labels.items():
        if any(not (lo <= src < hi) for src in targets_from.get(lab, [])):
            return None  # entered from outside the range
    n = 0
    for i in range(lo, hi):
        if LOAD.match(body[i]) and not any(a < i < t for a, t in skipped):
            n += 1
    return n


def check_function(name, body):
    """Problems found in one function, and the number of waits checked."""
    problems, checked = [], 0
    targets_from = {}
    for i, s in enumerate(body):
        m = BRANCH.match(s)
        if m:
            targets_from.setdefault(m.group(2), []).append(i)
    in_asm = False
    last_x = None  # index of the last asm x load seen
    for i, s in enumerate(body):
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not in_asm:
            continue
        if XLOAD.match(s):
            last_x = i
            continue
        m = WAIT.match(s)
        if m and last_x is not None:
            n = int(m.group(1))
            checked += 1
            got = window_loads(body, last_x + 1, i, targets_from)
            if got is None:
                problems.append(f"{name}: control flow the check does not accept before s_waitcnt vmcnt({n})")
            elif got < n:
                problems.append(f"{name}: s_waitcnt vmcnt({n}) after only {got} loads on some path")
            last_x = None
    return problems, checked


def check(text):
    problems, checked = [], 0
    for name, body in functions(text.splitlines()):
        p, c = check_function(name, body)
        problems += p
        checked += c
    return problems, checked


def main(argv):
    if len(argv) != 2:
        print(__doc__.strip().splitlines()[-1])
        return 2
    problems, checked = check(open(argv[1]).read())
    for p in problems:
        print("check_vmcnt:", p)
    if checked == 0:
        print("check_vmcnt: no hand-counted waits found (assembly of csrc/gemv_fused.hip expected)")
        return 1
    if problems:
        return 1
    print(f"check_vmcnt: {checked} hand-counted waits hold")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
