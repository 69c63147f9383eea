"""Build check of the inline-asm MFMAs with AGPR accumulators, on the
gfx950 assembly built here (CPU only).

The GQA forward's one-wave-per-SIMD kernels (64 queries per wave) issue
their P.V MFMAs as inline asm (`mfma32_agpr`), so the O accumulators stay in
AGPRs while the score MFMAs write VGPRs.  The compiler does not know that
asm is an MFMA and inserts none of the wait states the hardware needs
around one; the code provides them instead: an `s_nop` inside the asm ahead
of the MFMA (VALU-written A/B operands need two wait states), and
`agpr_settle` (21 wait states) before any other access to the accumulator.
This test checks the result in the built code: from every MFMA that writes
AGPRs, along every control-flow path (the loop's back edges included), no
instruction touches those AGPRs within 19 wait states (the most a 32x32
MFMA result needs before a VALU or v_accvgpr access), except the next MFMA
accumulating into the same registers, which the hardware forwards; and
every such MFMA comes right after its `s_nop`.  A register copy the
allocator placed after one of them, or a settle the scheduler moved, fails it.
"""
from __future__ import annotations

import re

import pytest

import asm_walk
from conftest import REPO_ROOT, import_submodule

SRC = REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / "gqa_fwd.hip"
KERNEL = "_ZN2mx3gqa14gqa_fwd_kernel"
NEED = 19

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
        prev = next(t for k, t in reversed(ins[:li]) if k == "instr")
        if not re.match(r"^s_nop [1-7]$", prev):
            problems.append(f"{mf!r}: preceded by {prev!r}, not its s_nop")

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


@pytest.fixture(scope="module")
def gqa_asm(tmp_path_factory):
    build = import_submodule("build")
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    return asm_walk.compile_asm(build, SRC, tmp_path_factory.mktemp("gqaasm") / "gqa_fwd.s")


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


def test_checker_sees_planted_hazards():
    """The walk flags an accumulator read too soon (also across a branch),
    a missing s_nop, and accepts a settled read and back-to-back accumulation."""
    mf = "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]"
    settle = ["s_nop 7", "s_nop 7", "s_nop 4"]
    good = ["s_nop 1", mf, "s_nop 1", mf, *settle, "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    assert _check_kernel(good) == (2, [])
    early = ["s_nop 1", mf, "s_nop 7", "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    assert "touches a[0:15] 8 wait states" in _check_kernel(early)[1][0]
    no_nop = ["v_mov_b32_e32 v4, 0", mf, *settle, "s_endpgm"]
    assert "not its s_nop" in _check_kernel(no_nop)[1][0]
    other = ["s_nop 1", mf, "s_nop 1", "v_mfma_f32_32x32x16_bf16 a[16:31], v[0:3], v[4:7], a[0:15]", "s_endpgm"]
    assert "touches" in _check_kernel(other)[1][0]
    branch = ["s_nop 1", mf, "s_cbranch_scc0 .LBB0_2", *settle, "s_endpgm", ".LBB0_2:",
              "v_accvgpr_mov_b32 a16, a0", "s_endpgm"]
    assert "v_accvgpr_mov_b32 a16, a0" in _check_kernel(branch)[1][0]
