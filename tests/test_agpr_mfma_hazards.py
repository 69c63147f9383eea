"""Build check of the inline-asm MFMAs with AGPR accumulators, on the
gfx950 assembly built here (CPU only).

The GQA forward's one-wave-per-SIMD kernels (64 queries per wave) issue
their P.V MFMAs as inline asm (`mfma32_agpr`), so the O accumulators stay in
AGPRs while the score MFMAs write VGPRs.  The compiler does not know that
asm is an MFMA and inserts none of the wait states the hardware needs
around one; the code provides them instead: `agpr_settle` (21 wait states) before any
other access to the accumulator, and `operand_settle` (2 wait states)
between the VALU writes of an A or B operand and the MFMAs that read it.
This test checks the result in the built code: from every MFMA that writes
AGPRs, along every control-flow path (the loop's back edges included), no
instruction touches those AGPRs within 19 wait states (the most a 32x32
MFMA result needs before a VALU or v_accvgpr access), except the next MFMA
accumulating into the same registers, which the hardware forwards; and
no VALU instruction writes any source register of an MFMA (A, B or
accumulator) within the 2 wait states before it, which the hardware needs
and which the asm does not add (an `s_nop` in front of every MFMA would
cost ~7 cycles each in a stream of MFMAs).  The second check covers every
MFMA of the GQA and MLA decode kernels, whose rare rescale writes
accumulators through asm the compiler cannot see into; a third asserts
that no inline-asm instruction (such as that rescale's reads) touches an
MFMA's result within 19 wait states, since the compiler guards only its
own instructions.  A register copy
the allocator placed next to one of them, or a settle the scheduler
moved, fails it.
"""
from __future__ import annotations

import re

import pytest

import asm_walk
from conftest import REPO_ROOT, import_submodule

SRC = REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / "gqa_fwd.hip"
MLA_SRC = REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / "mla_decode.hip"
KERNEL = "_ZN2mx3gqa14gqa_fwd_kernel"
NEED = 19      # MFMA result -> other access
NEED_SRC = 2   # VALU write -> MFMA source read

_MFMA_A = re.compile(r"^v_mfma\S*\s+(a\[\d+:\d+\]),")
_ACCUM = re.compile(r"^v_mfma\S*\s+(a\[\d+:\d+\]),\s*\S+,\s*\S+,\s*(a\[\d+:\d+\])$")


def _check_kernel(lines: list[str]) -> tuple[int, list[str]]:
    ins = asm_walk.instrs(lines)
    mfmas = [i for i, (k, t) in enumerate(ins) if k == "instr" and _MFMA_A.match(t)]
    problems = []
    for li in mfmas:
        mf = ins[li][1]
        dst = _MFMA_A.match(mf).group(1)
        regs = asm_walk.aregs(dst)

        # state: wait states since the MFMA on this path (capped at NEED)
        def step(i, t, ws, mf=mf, dst=dst, regs=regs):
            if regs & asm_walk.aregs(t):
                m = _ACCUM.match(t)
                if not (m and m.group(1) == dst and m.group(2) == dst) and ws < NEED:
                    problems.append(f"{mf!r}: {t!r} touches {dst} {ws} wait states after it")
                return True, ws
            m = re.match(r"^s_nop (\d+)$", t)
            ws = min(NEED, ws + (int(m.group(1)) + 1 if m else 1))
            return ws >= NEED, ws

        asm_walk.walk(ins, li + 1, step)
    return len(mfmas), problems


def _check_asm_readers(lines: list[str]) -> tuple[int, list[str]]:
    """Every MFMA: no inline-asm instruction touches its result registers
    within NEED wait states after it (the compiler guards only its own
    instructions; an asm reader such as scale_acc after a builtin MFMA is
    the code's to guard)."""
    ins = asm_walk.instrs(lines)
    origin = asm_walk.asm_origin(lines)
    mfmas = [i for i, (k, t) in enumerate(ins) if k == "instr" and t.startswith("v_mfma")]
    problems = []
    for li in mfmas:
        mf = ins[li][1]
        dst = mf.split(None, 1)[1].split(",")[0]
        dv, da = asm_walk.vregs(dst), asm_walk.aregs(dst)

        # the walk goes on past the compiler's own accesses to the registers
        # (it guards those), so an asm access behind one is still seen
        def step(i, t, ws, mf=mf, dst=dst, dv=dv, da=da):
            if i in origin and (dv & asm_walk.vregs(t) or da & asm_walk.aregs(t)):
                m = _ACCUM.match(t)
                if not (m and m.group(1) == dst and m.group(2) == dst) and ws < NEED:
                    problems.append(f"{mf!r}: asm {t!r} touches {dst} {ws} wait states after it")
                    return True, ws
            ws = min(NEED, ws + _waits(t))
            return ws >= NEED, ws

        asm_walk.walk(ins, li + 1, step)
    return len(mfmas), problems


def _waits(t: str) -> int:
    m = re.match(r"^s_nop (\d+)$", t)
    return int(m.group(1)) + 1 if m else 1


def _check_sources(lines: list[str]) -> tuple[int, list[str]]:
    """Every MFMA: no VALU write to one of its sources within NEED_SRC wait
    states before it, on any path that reaches it."""
    ins = asm_walk.instrs(lines)
    pred = asm_walk.predecessors(ins)
    mfmas = [i for i, (k, t) in enumerate(ins) if k == "instr" and t.startswith("v_mfma")]
    problems = []
    for li in mfmas:
        mf = ins[li][1]
        srcs = mf.split(None, 1)[1].split(",")[1:4]
        sv, sa = asm_walk.vregs(",".join(srcs)), asm_walk.aregs(",".join(srcs))

        def step(i, t, ws, mf=mf, sv=sv, sa=sa):
            dv, da = asm_walk.valu_dsts(t)
            if (dv & sv or da & sa) and ws < NEED_SRC:
                problems.append(f"{mf!r}: source written by {t!r} {ws} wait states before it")
                return True, ws
            ws += _waits(t)
            return ws >= NEED_SRC, ws

        asm_walk.walk_back(ins, pred, li, step)
    return len(mfmas), problems


@pytest.fixture(scope="module")
def gqa_asm(tmp_path_factory):
    build = import_submodule("build")
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    return asm_walk.compile_asm(build, SRC, tmp_path_factory.mktemp("gqaasm") / "gqa_fwd.s")


@pytest.fixture(scope="module")
def mla_asm(tmp_path_factory):
    build = import_submodule("build")
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    return asm_walk.compile_asm(build, MLA_SRC, tmp_path_factory.mktemp("mlaasm") / "mla_decode.s")


def test_agpr_accumulators_wait_for_their_mfmas(gqa_asm):
    ks = asm_walk.kernels(gqa_asm)
    qt2 = {n: b for n, b in ks.items() if n.startswith(KERNEL) and "ELi2ELi4E" in n}
    assert len(qt2) == 8, "QT=2 kernels: D 64 and 128, bf16 and f16, causal and not"
    for name, body in ks.items():
        n, problems = _check_kernel(body)
        if name in qt2:
            assert n >= 16, f"{name}: expected the P.V MFMAs in AGPR form, found {n}"
        else:
            assert n == 0, f"{name}: unexpected AGPR-form MFMAs"
        assert not problems, f"{name}:\n" + "\n".join(problems[:10])


@pytest.mark.parametrize("which", ["gqa", "mla"])
def test_mfma_sources_wait_for_valu_writes(which, request):
    asm = request.getfixturevalue(f"{which}_asm")
    total = 0
    for name, body in asm_walk.kernels(asm).items():
        n, problems = _check_sources(body)
        total += n
        assert not problems, f"{name}:\n" + "\n".join(problems[:10])
    assert total > 0


@pytest.mark.parametrize("which", ["gqa", "mla"])
def test_asm_readers_wait_for_mfma_results(which, request):
    asm = request.getfixturevalue(f"{which}_asm")
    for name, body in asm_walk.kernels(asm).items():
        _, problems = _check_asm_readers(body)
        assert not problems, f"{name}:\n" + "\n".join(problems[:10])


def test_checker_sees_planted_hazards():
    """The walks flag an accumulator read too soon (also across a branch) and
    a source written too soon (also along a loop's back edge), and accept a
    settled read, back-to-back accumulation and unrelated writes."""
    mf = "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]"
    settle = ["s_nop 7", "s_nop 7", "s_nop 4"]
    good = [mf, mf, *settle, "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    assert _check_kernel(good) == (2, [])
    early = [mf, "s_nop 7", "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    assert "touches a[0:15] 8 wait states" in _check_kernel(early)[1][0]
    no_nop = ["v_mov_b32_e32 v4, 0", mf, *settle, "s_endpgm"]
    assert "source written by 'v_mov_b32_e32 v4, 0' 0 wait states" in _check_sources(no_nop)[1][0]
    one = ["v_cvt_pk_bf16_f32 v5, v8, v9", "s_nop 0", mf, *settle, "s_endpgm"]
    assert "1 wait states" in _check_sources(one)[1][0]
    assert _check_sources(["v_cvt_pk_bf16_f32 v5, v8, v9", "s_nop 1", mf, *settle, "s_endpgm"]) == (1, [])
    acc = ["v_accvgpr_write_b32 a3, v9", mf, "s_endpgm"]
    assert "v_accvgpr_write_b32 a3, v9" in _check_sources(acc)[1][0]
    other = ["v_mov_b32_e32 v20, 0", mf, "s_endpgm"]
    assert _check_sources(other) == (1, [])
    # an asm reader right after a builtin MFMA; the compiler's own reader is not the check's concern
    vmf = "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]"
    asm_read = [vmf, ";;#ASMSTART", "v_accvgpr_read_b32 v9, a2", ";;#ASMEND", "s_endpgm"]
    assert "asm 'v_accvgpr_read_b32 v9, a2' touches a[0:15] 0 wait states" in _check_asm_readers(asm_read)[1][0]
    assert _check_asm_readers([vmf, "s_nop 7", "v_accvgpr_read_b32 v9, a2", "s_endpgm"]) == (1, [])
    assert _check_asm_readers([vmf, *settle, ";;#ASMSTART", "v_accvgpr_read_b32 v9, a2", ";;#ASMEND",
                               "s_endpgm"]) == (1, [])
    # a write on the path that branches back to the MFMA
    loop = [".LBB0_1:", mf, "v_add_u32_e32 v1, 1, v1", "v_mov_b32_e32 v2, 0", "s_cbranch_scc0 .LBB0_1", "s_endpgm"]
    assert "v_mov_b32_e32 v2, 0" in _check_sources(loop)[1][0]
    other_acc = [mf, "s_nop 1", "v_mfma_f32_32x32x16_bf16 a[16:31], v[0:3], v[4:7], a[0:15]", "s_endpgm"]
    assert "touches" in _check_kernel(other_acc)[1][0]
    branch = [mf, "s_cbranch_scc0 .LBB0_2", *settle, "s_endpgm", ".LBB0_2:",
              "v_accvgpr_mov_b32 a16, a0", "s_endpgm"]
    assert "v_accvgpr_mov_b32 a16, a0" in _check_kernel(branch)[1][0]
