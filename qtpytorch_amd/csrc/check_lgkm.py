"""Static check of the hand-counted LDS waits in the gfx950 assembly.

The pipelined GEMM issues its LDS fragment reads (ds_read_b128,
ds_read_b64_tr_b8) and stage stores (ds_write_b128) as inline assembly and
waits for them with explicit ``s_waitcnt lgkmcnt(N)``, so the compiler does
not insert waits of its own for those reads.  A read whose result is used,
or whose destination registers are rewritten, before a wait that retires it
is a silent error: the data lands in the registers later and overwrites
whatever the compiler has put there since.

This script compiles a source file to gfx950 assembly (device code only) and
runs a dataflow over the basic blocks of every GEMM kernel.  The state is
the ordered queue of outstanding LGKM operations:

  * each LDS instruction (``ds_*``) enters the queue with the vector
    registers it writes (none for stores), marked when it was issued from
    inline assembly (between the compiler's ``;;#ASMSTART`` / ``;;#ASMEND``
    markers);
  * ``s_waitcnt lgkmcnt(N)`` retires the oldest LDS entries until at most N
    LDS entries remain (LDS operations of one wave complete in issue
    order).  Scalar memory operations (``s_load*``, ``s_memtime``) count
    toward the same counter but may complete before older LDS operations,
    so they are taken as already complete: a wait then retires no more LDS
    entries than it would without them;
  * an instruction that reads or writes a vector register still owed by an
    outstanding inline-asm LDS read is reported.  Reads the compiler issued
    itself get compiler-placed waits and only count toward the queue.

States flow along branch edges; where two predecessors of a block disagree
(a join or a loop head reached with different outstanding reads), that is
reported too.  build.py runs the check after compiling the GEMM; run it
directly (optionally with a source path) to print the report.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
from typing import Dict, Iterable, List, Set, Tuple

_REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")
_WAIT = re.compile(r"lgkmcnt\((\d+)\)")
# LDS instructions without a vector destination
_DS_NODEST = re.compile(r"^ds_(write|store|add|sub|rsub|inc|dec|min|max|and|or|xor|cmpst|mskor|nop)")

Entry = Tuple[str, frozenset, bool]  # ("lds", registers it writes, issued by inline asm)
State = Tuple[Entry, ...]


def _regs(text: str) -> Set[Tuple[str, int]]:
    out: Set[Tuple[str, int]] = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add((m.group(1), int(m.group(2))))
        else:
            k, lo, hi = m.group(3), int(m.group(4)), int(m.group(5))
            out.update((k, r) for r in range(lo, hi + 1))
    return out


def _owed(state: State) -> Set[Tuple[str, int]]:
    out: Set[Tuple[str, int]] = set()
    for kind, dest, manual in state:
        if kind == "lds" and manual:
            out |= dest
    return out


def _step(state: State, op: str, rest: str, manual: bool, where: str, problems: List[str]) -> State:
    """Apply one instruction to the queue; report touches of owed registers."""
    q = list(state)
    if op == "s_waitcnt":
        w = _WAIT.search(rest)
        if w:
            n = int(w.group(1))
            if n == 0:
                return ()
            while len(q) > n:
                q.pop(0)
        return tuple(q)
    operands = [p.strip() for p in rest.split(",") if p.strip()]
    touched: Set[Tuple[str, int]] = set()
    for o in operands:
        touched |= _regs(o)
    bad = touched & _owed(state)
    if bad:
        problems.append(f"{where}: {op} touches {sorted(bad)} before the inline-asm LDS read into them was waited for")
    if op.startswith("ds_"):
        dest = frozenset() if _DS_NODEST.match(op) else frozenset(_regs(operands[0]) if operands else set())
        q.append(("lds", dest, manual))
    return tuple(q)


def _functions(asm: str) -> List[Tuple[str, List[Tuple[int, str]]]]:
    funcs: List[Tuple[str, List[Tuple[int, str]]]] = []
    cur = None
    for i, ln in enumerate(asm.splitlines(), 1):
        fm = re.match(r"^([A-Za-z_][\w.$]*):", ln)
        if fm and not fm.group(1).startswith(".L"):
            cur = (fm.group(1), [])
            funcs.append(cur)
            continue
        if cur is not None:
            if re.match(r"^\.Lfunc_end", ln):
                cur = None
                continue
            cur[1].append((i, ln))
    return funcs


def check_function(name: str, lines: List[Tuple[int, str]]) -> List[str]:
    # split into basic blocks: (label, [(line, op, rest, manual)], successors)
    blocks: List[Tuple[str, List[Tuple[int, str, str, bool]]]] = [("<entry>", [])]
    in_asm = False
    for i, ln in lines:
        if ";;#ASMSTART" in ln:
            in_asm = True
            continue
        if ";;#ASMEND" in ln:
            in_asm = False
            continue
        lm = re.match(r"^(\.LBB[\w.]+):", ln)
        if lm:
            blocks.append((lm.group(1), []))
            continue
        s = ln.split(";", 1)[0].strip()
        if not s or s.startswith("."):
            continue
        parts = s.split(None, 1)
        blocks[-1][1].append((i, parts[0], parts[1] if len(parts) > 1 else "", in_asm))
        if parts[0] in ("s_branch", "s_endpgm", "s_setpc_b64") or parts[0].startswith("s_cbranch"):
            blocks.append((f"<after line {i}>", []))  # a branch ends its block
    index = {lab: k for k, (lab, _) in enumerate(blocks)}
    succ: Dict[int, List[int]] = {}
    for k, (lab, ins) in enumerate(blocks):
        nxt = [k + 1] if k + 1 < len(blocks) else []
        out: List[int] = []
        ends = False
        for _, op, rest, _m in ins:
            if op in ("s_branch",):
                out.append(index[rest.split()[0]])
                ends = True
            elif op.startswith("s_cbranch"):
                out.append(index[rest.split()[0]])
            elif op in ("s_endpgm", "s_setpc_b64"):
                ends = True
        if not ends:
            out += nxt
        succ[k] = out
    problems: List[str] = []
    states: Dict[int, State] = {0: ()}
    work = [0]
    done_mismatch: Set[int] = set()
    visits: Dict[int, int] = {}
    while work:
        k = work.pop()
        visits[k] = visits.get(k, 0) + 1
        if visits[k] > 64:
            problems.append(f"{name}: no fixed point at {blocks[k][0]}")
            break
        st = states[k]
        for line, op, rest, manual in blocks[k][1]:
            st = _step(st, op, rest, manual, f"{name}: line {line}", problems)
        for t in succ[k]:
            if t not in states:
                states[t] = st
                work.append(t)
            elif states[t] != st and t not in done_mismatch:
                if _owed(states[t]) or _owed(st):
                    problems.append(f"{name}: {blocks[t][0]} is reached with different outstanding inline-asm LDS reads")
                    done_mismatch.add(t)
    return sorted(set(problems))


def check_asm(asm: str, only: Iterable[str] = ()) -> Tuple[int, List[str]]:
    """(functions checked, problems) for the functions of `asm` whose names
    contain one of `only` (all when empty)."""
    only = list(only)
    problems: List[str] = []
    n = 0
    for name, lines in _functions(asm):
        if only and not any(o in name for o in only):
            continue
        n += 1
        problems += check_function(name, lines)
    return n, problems


def compile_asm(src: str, hipcc: str, flags: List[str]) -> str:
    """Device-only gfx950 assembly of `src` (flags as for the library build)."""
    cmd = [hipcc, *[f for f in flags if f not in ("-fPIC",)], "--cuda-device-only", "-S", src, "-o", "-"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"assembly of {src} failed:\n{r.stderr[-4000:]}")
    return r.stdout


def check_source(src: str, hipcc: str, flags: List[str]) -> Tuple[int, List[str]]:
    return check_asm(compile_asm(src, hipcc, flags), only=("k_qgemm",))


def main() -> int:
    here = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, os.path.dirname(os.path.dirname(here)))
    from qtpytorch_amd.csrc import build as b

    src = sys.argv[1] if len(sys.argv) > 1 else os.path.join(here, "mxk_gemm.hip")
    n, problems = check_source(src, b.hipcc(), b.HIPCC_FLAGS)
    for p in problems:
        print(p)
    print(f"{os.path.basename(src)}: {n} GEMM kernels checked, {len(problems)} problems")
    return 1 if problems else 0


if __name__ == "__main__":
    sys.exit(main())
