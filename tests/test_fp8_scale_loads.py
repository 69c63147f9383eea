"""Build check of the fp8 block-scaled GEMM's untracked scale loads, on the
gfx950 assembly built here (CPU only).

gemm_fp8_bs_kernel reads its block scales with `global_load_dword`
issued as inline asm, which the compiler does not track, and makes them
safe with an asm `s_waitcnt vmcnt(N)` that names the scale registers.
Between such a load and the wait that lands it the register holds a value
still in flight: a copy or a spill the register allocator placed there
(for instance to coalesce the scales carried around the block loop) would
read it too early, and any write to it would be overwritten when the load
lands.  This test walks the assembly from every scale load, along every
control-flow path (into the loop's next iteration too), to the first vmcnt
wait, and asserts that no instruction on the way names the register and
that the wait's count is at most the number of vector-memory instructions
issued after the load on that path, so that the wait lands it.
"""
from __future__ import annotations

import re
import subprocess

import pytest

from conftest import REPO_ROOT, import_submodule

SRC = REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / "gemm_fp8_bs.hip"
KERNEL = "_ZN2mx5gemm818gemm_fp8_bs_kernel"

_VREG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_VMEM = re.compile(r"^\s*(global_|buffer_|flat_|scratch_)")


def _kernels(asm: str) -> dict[str, list[str]]:
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


def _instrs(lines: list[str]):
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


def _regs(text: str) -> set[int]:
    regs = set()
    for a, b, one in _VREG.findall(text):
        if one:
            regs.add(int(one))
        else:
            regs.update(range(int(a), int(b) + 1))
    return regs


def _check_kernel(lines: list[str]) -> tuple[int, list[str]]:
    ins = _instrs(lines)
    labels = {t: i for i, (k, t) in enumerate(ins) if k == "label"}
    loads = [i for i, (k, t) in enumerate(ins)
             if k == "instr" and re.match(r"^global_load_dword\s+v\d+,\s*v\d+,\s*s\[", t)]
    problems = []
    for li in loads:
        reg = int(re.match(r"^global_load_dword\s+v(\d+)", ins[li][1]).group(1))
        seen = set()
        stack = [(li + 1, 0)]  # (instruction index, vector-memory ops issued since the load)
        while stack:
            i, nv = stack.pop()
            while i < len(ins):
                if (i, nv) in seen:
                    break
                seen.add((i, nv))
                k, t = ins[i]
                if k != "instr":
                    i += 1
                    continue
                m = re.match(r"^s_waitcnt\b.*vmcnt\((\d+)\)", t)
                if m:
                    if int(m.group(1)) > nv:
                        problems.append(f"{ins[li][1]!r}: {t!r} does not land it ({nv} loads after it on this path)")
                    break
                if reg in _regs(t):
                    problems.append(f"{ins[li][1]!r}: {t!r} names v{reg} before the load is waited for")
                    break
                if t.startswith("s_endpgm"):
                    problems.append(f"{ins[li][1]!r}: kernel ends before a vmcnt wait")
                    break
                if _VMEM.match(t):
                    nv += 1
                bm = re.match(r"^s_(c)?branch\w*\s+(\.LBB\w+)", t)
                if bm:
                    target = labels[bm.group(2)]
                    if bm.group(1):  # conditional: both ways
                        stack.append((target, nv))
                        i += 1
                        continue
                    i = target
                    continue
                i += 1
    return len(loads), problems


@pytest.fixture(scope="module")
def fp8_asm(tmp_path_factory):
    build = import_submodule("build")
    try:
        hipcc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("fp8asm") / "gemm_fp8_bs.s"
    flags = [f for f in build.common_flags() if f != "-fPIC"]
    proc = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", str(SRC), "-o", str(out)],
                          capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def test_scale_registers_untouched_until_their_wait(fp8_asm):
    kernels = {n: body for n, body in _kernels(fp8_asm).items() if n.startswith(KERNEL)}
    assert len(kernels) >= 2, "both tile shapes of gemm_fp8_bs_kernel are in the code object"
    for name, body in kernels.items():
        nloads, problems = _check_kernel(body)
        assert nloads >= 3, f"{name}: expected the block-scale loads, found {nloads}"
        assert not problems, f"{name}:\n" + "\n".join(problems[:10])


def test_checker_sees_a_planted_copy():
    """The walk flags a register copy placed between a scale load and its
    wait, a wait that would not land the load, and follows a loop back-edge."""
    good = ["global_load_dword v7, v1, s[2:3]", "global_load_lds_dwordx4 v2, s[4:5]", "s_waitcnt vmcnt(1)",
            "v_mov_b32_e32 v8, v7", "s_endpgm"]
    assert _check_kernel(good) == (1, [])
    copied = good[:2] + ["v_mov_b32_e32 v9, v7"] + good[2:]
    assert "names v7" in _check_kernel(copied)[1][0]
    early = good[:2] + ["s_waitcnt vmcnt(2)"] + good[3:]
    assert "does not land" in _check_kernel(early)[1][0]
    loop = [".LBB0_1:", "s_waitcnt vmcnt(1)", "v_add_f32_e32 v3, v7, v3", "global_load_dword v7, v1, s[2:3]",
            "v_add_u32_e32 v7, 1, v7", "s_cbranch_scc0 .LBB0_1", "s_waitcnt vmcnt(0)", "s_endpgm"]
    assert "names v7" in _check_kernel(loop)[1][0]
    back = [".LBB0_1:", "s_waitcnt vmcnt(0)", "v_add_f32_e32 v3, v7, v3", "global_load_dword v7, v1, s[2:3]",
            "s_cbranch_scc0 .LBB0_1", "v_mov_b32_e32 v4, v7", "s_endpgm"]
    assert "names v7" in _check_kernel(back)[1][0]  # the fall-through path reads it unwaited
