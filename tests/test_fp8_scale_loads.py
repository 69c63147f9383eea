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

import pytest

import asm_walk
from conftest import REPO_ROOT, import_submodule

SRC = REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / "gemm_fp8_bs.hip"
KERNEL = "_ZN2mx5gemm818gemm_fp8_bs_kernel"

_VMEM = re.compile(r"^\s*(global_|buffer_|flat_|scratch_)")
# the scale loads: one scale (global_load_dword), two or four (x2, x4) per lane
_SCALE_LOAD = re.compile(r"^global_load_dword(?:x2|x4)?\s+(v\d+|v\[\d+:\d+\]),\s*v\d+,\s*s\[")


def _check_kernel(lines: list[str]) -> tuple[int, list[str]]:
    ins = asm_walk.instrs(lines)
    loads = [i for i, (k, t) in enumerate(ins)
             if k == "instr" and _SCALE_LOAD.match(t)]
    problems = []
    for li in loads:
        load = ins[li][1]
        regs = asm_walk.vregs(_SCALE_LOAD.match(load).group(1))

        # state: vector-memory instructions issued since the load on this path
        def step(i, t, nv, load=load, regs=regs):
            m = re.match(r"^s_waitcnt\b.*vmcnt\((\d+)\)", t)
            if m:
                if int(m.group(1)) > nv:
                    problems.append(f"{load!r}: {t!r} does not land it ({nv} loads after it on this path)")
                return True, nv
            if regs & asm_walk.vregs(t):
                problems.append(f"{load!r}: {t!r} names {sorted(regs)} before the load is waited for")
                return True, nv
            if t.startswith("s_endpgm"):
                problems.append(f"{load!r}: kernel ends before a vmcnt wait")
                return True, nv
            return False, nv + (1 if _VMEM.match(t) else 0)

        asm_walk.walk(ins, li + 1, step)
    return len(loads), problems


@pytest.fixture(scope="module")
def fp8_asm(tmp_path_factory):
    build = import_submodule("build")
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    return asm_walk.compile_asm(build, SRC, tmp_path_factory.mktemp("fp8asm") / "gemm_fp8_bs.s")


def test_scale_registers_untouched_until_their_wait(fp8_asm):
    kernels = {n: body for n, body in asm_walk.kernels(fp8_asm).items() if n.startswith(KERNEL)}
    assert len(kernels) >= 4, "both tile shapes of gemm_fp8_bs_kernel, with and without grouped scale loads"
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
    assert "names [7]" in _check_kernel(copied)[1][0]
    early = good[:2] + ["s_waitcnt vmcnt(2)"] + good[3:]
    assert "does not land" in _check_kernel(early)[1][0]
    loop = [".LBB0_1:", "s_waitcnt vmcnt(1)", "v_add_f32_e32 v3, v7, v3", "global_load_dword v7, v1, s[2:3]",
            "v_add_u32_e32 v7, 1, v7", "s_cbranch_scc0 .LBB0_1", "s_waitcnt vmcnt(0)", "s_endpgm"]
    assert "names [7]" in _check_kernel(loop)[1][0]
    # a paired load: a read of its second register is caught too
    pair = ["global_load_dwordx2 v[8:9], v1, s[2:3]", "v_mov_b32_e32 v10, v9", "s_waitcnt vmcnt(0)", "s_endpgm"]
    assert _check_kernel(pair)[0] == 1 and "names [8, 9]" in _check_kernel(pair)[1][0]
    back = [".LBB0_1:", "s_waitcnt vmcnt(0)", "v_add_f32_e32 v3, v7, v3", "global_load_dword v7, v1, s[2:3]",
            "s_cbranch_scc0 .LBB0_1", "v_mov_b32_e32 v4, v7", "s_endpgm"]
    assert "names [7]" in _check_kernel(back)[1][0]  # the fall-through path reads it unwaited
