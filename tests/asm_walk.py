"""Reading gfx950 assembly built here (hipcc -S): kernels, instructions,
registers and a walk over every control-flow path from an instruction.
Used by the build-level checks of inline-asm code (CPU only)."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

_VREG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_AREG = re.compile(r"\ba\[(\d+):(\d+)\]|\ba(\d+)\b")
_BRANCH = re.compile(r"^s_(c)?branch\w*\s+(\.LBB\w+)")


def compile_asm(build, src: Path, out: Path) -> str:
    """gfx950 assembly of one source, with the flags the library build uses for it."""
    flags = [f for f in build.common_flags() if f != "-fPIC"] + build.source_flags(src)
    proc = subprocess.run([build.hipcc(), *flags, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                          capture_output=True, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def kernels(asm: str) -> dict[str, list[str]]:
    out, cur, name = {}, None, None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name, cur = m.group(1), []
            continue
        if cur is not None:
            cur.append(line)
            if "s_endpgm" in line:
                out[name] = cur
                cur = None
    return out


def instrs(lines: list[str]):
    """(kind, text) per line: 'label', 'instr' or None for comments/directives."""
    res = []
    for raw in lines:
        t = raw.split(";")[0].rstrip()
        s = t.strip()
        if not s or s.startswith(".") and not re.match(r"^\.LBB\w+:", s) or s.startswith("//"):
            res.append((None, s))
        elif re.match(r"^\.LBB\w+:", s):
            res.append(("label", s[:-1]))
        else:
            res.append(("instr", s))
    return res


def asm_origin(lines: list[str]) -> set[int]:
    """Indices (as in instrs(lines)) of instructions written as inline asm
    in the source, which the compiler brackets with ;;#ASMSTART / ;;#ASMEND:
    the compiler inserts no wait states for their hazards."""
    out, inside = set(), False
    for i, raw in enumerate(lines):
        s = raw.strip()
        if s.startswith(";;#ASMSTART"):
            inside = True
        elif s.startswith(";;#ASMEND"):
            inside = False
        elif inside:
            out.add(i)
    return out


def _regs(pattern: re.Pattern, text: str) -> set[int]:
    regs = set()
    for a, b, one in pattern.findall(text):
        if one:
            regs.add(int(one))
        else:
            regs.update(range(int(a), int(b) + 1))
    return regs


def vregs(text: str) -> set[int]:
    return _regs(_VREG, text)


def aregs(text: str) -> set[int]:
    return _regs(_AREG, text)


def walk(ins, start: int, step):
    """Run step(i, text, state) -> (stop, new_state) over every path from
    instruction index `start` (the loop's back edges included), each path
    ending where step says stop or at s_endpgm.  `state` starts as 0 and must
    be hashable; a (position, state) pair is visited once."""
    labels = {t: i for i, (k, t) in enumerate(ins) if k == "label"}
    seen = set()
    stack = [(start, 0)]
    while stack:
        i, st = stack.pop()
        while i < len(ins):
            if (i, st) in seen:
                break
            seen.add((i, st))
            k, t = ins[i]
            if k != "instr":
                i += 1
                continue
            stop, st = step(i, t, st)
            if stop or t.startswith("s_endpgm"):
                break
            bm = _BRANCH.match(t)
            if bm:
                target = labels[bm.group(2)]
                if bm.group(1):  # conditional: both ways
                    stack.append((target, st))
                    i += 1
                    continue
                i = target
                continue
            i += 1


def _successors(ins) -> dict[int, list[int]]:
    """Instruction-level control flow: index -> indices of the instructions
    that can run next."""
    order = [i for i, (k, _) in enumerate(ins) if k == "instr"]
    first_after = {}
    pending = []
    for i, (k, t) in enumerate(ins):
        if k == "label":
            pending.append(t)
        elif k == "instr":
            for lab in pending:
                first_after[lab] = i
            pending = []
    nxt = {a: b for a, b in zip(order, order[1:])}
    succ = {}
    for i in order:
        t = ins[i][1]
        bm = _BRANCH.match(t)
        if t.startswith("s_endpgm"):
            succ[i] = []
        elif bm and not bm.group(1):
            succ[i] = [first_after[bm.group(2)]]
        elif bm:
            succ[i] = [j for j in (nxt.get(i), first_after.get(bm.group(2))) if j is not None]
        else:
            succ[i] = [nxt[i]] if i in nxt else []
    return succ


def predecessors(ins) -> dict[int, list[int]]:
    pred = {}
    for i, js in _successors(ins).items():
        pred.setdefault(i, [])
        for j in js:
            pred.setdefault(j, []).append(i)
    return pred


def walk_back(ins, pred, start: int, step):
    """As walk(), backwards along every path that reaches instruction `start`
    (its predecessors first)."""
    seen = set()
    stack = [(p, 0) for p in pred.get(start, [])]
    while stack:
        i, st = stack.pop()
        if (i, st) in seen:
            continue
        seen.add((i, st))
        stop, st = step(i, ins[i][1], st)
        if not stop:
            stack.extend((p, st) for p in pred.get(i, []))


def valu_dsts(text: str) -> tuple[set[int], set[int]]:
    """(VGPRs, AGPRs) a VALU instruction writes: its first operand (both
    operands of a permlane swap).  Empty for anything that is not VALU."""
    if not text.startswith("v_") or text.startswith("v_mfma"):
        return set(), set()
    ops = [o.strip() for o in text.split(None, 1)[1].split(",")] if " " in text else []
    dst = ops[:2] if "permlane" in text and "swap" in text else ops[:1]
    return vregs(" ".join(dst)), aregs(" ".join(dst))
