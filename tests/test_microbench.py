"""The hardware characterisation probes (cuda-oxide-bench_amd/microbench):
the library builds with the package and exports its launchers, which
reject invalid arguments before launching (CPU); one short run of each
probe on the GPU returns finite, positive figures (gpu)."""
from __future__ import annotations

import ctypes
import importlib.util
import math

import pytest

from conftest import REPO_ROOT, announce

RUN_PY = REPO_ROOT / "cuda-oxide-bench_amd" / "microbench" / "run.py"
ALT_PY = REPO_ROOT / "cuda-oxide-bench_amd" / "microbench" / "alternatives.py"


@pytest.fixture(scope="module")
def runner():
    spec = importlib.util.spec_from_file_location("mx_microbench_run", RUN_PY)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_probe_library_exports_its_launchers(runner):
    lib = runner.load()
    for name in ("mxp_overlap_launch", "mxp_mfma_rate_launch", "mxp_contend_launch", "mxp_promote_launch",
                 "mxp_wg_read_launch", "mxp_stream_launch", "mxp_error_string"):
        assert hasattr(lib, name), name
    # invalid arguments are rejected before any HIP call
    assert lib.mxp_overlap_launch(0, 1, 0, 10, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert lib.mxp_overlap_launch(0, 1, 4, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert lib.mxp_overlap_launch(0, 1, 4, 10, None, ctypes.c_void_p(16), None) == -1
    assert lib.mxp_wg_read_launch(ctypes.c_void_p(16), 0, -1, 1, ctypes.c_void_p(16), None) == -1
    assert lib.mxp_wg_read_launch(None, 0, 8, 1, ctypes.c_void_p(16), None) == -1
    assert lib.mxp_mfma_rate_launch(8, 4, 10, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert lib.mxp_mfma_rate_launch(0, 4, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    p = ctypes.c_void_p(16)
    assert lib.mxp_contend_launch(5, 0, 1, 10, 0, p, p, p, p, p, None) == -1   # no such form
    assert lib.mxp_promote_launch(1, 4, 4, 1, 10, p, p, p, None) == -1   # lag 1..3
    assert lib.mxp_promote_launch(0, 1, 6, 1, 10, p, p, p, None) == -1   # 4 or 8 waves
    assert lib.mxp_promote_launch(4, 1, 4, 1, 10, p, p, p, None) == -1
    assert lib.mxp_contend_launch(0, 6, 1, 10, 0, p, p, p, p, p, None) == -1
    assert lib.mxp_contend_launch(0, 1, 1, 10, 10, p, p, p, p, None, None) == -1
    assert lib.mxp_stream_launch(0, 12, p, 0, 64, 1, p, None) == -1   # no such depth
    assert lib.mxp_stream_launch(2, 8, p, 0, 64, 1, p, None) == -1    # no such mode
    assert lib.mxp_stream_launch(1, 8, p, 0, 100, 1, p, None) == -1   # LDS copies take whole 1 KB chunks
    assert lib.mxp_stream_launch(1, 8, p, 0, 64, 0, p, None) == -1


def test_alternative_patches_apply():
    """Every alternative's text patches still match the kernel source exactly
    once (the tool refuses to build otherwise), each alternative changes the
    source, and every variant but the kernel as built is marked exact, so its
    output is compared bit for bit with the kernel as built's (CPU only; the
    build and the GPU run are the tool's)."""
    spec = importlib.util.spec_from_file_location("mx_microbench_alternatives", ALT_PY)
    alt = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(alt)
    for kernel, k in alt.KERNELS.items():
        base = (REPO_ROOT / "cuda-oxide-bench_amd" / "csrc" / k["source"]).read_text()
        for v, spec_v in k["variants"].items():
            text = alt.patched_source(kernel, v)
            assert (text == base) == (not spec_v[1]), f"{kernel}/{v}"
            assert (v == "as_built") != alt.variant_exact(kernel, v), f"{kernel}/{v}"


@pytest.mark.gpu
def test_probes_run(runner):
    lib = runner.load()
    announce("microbench overlap (MFMAs alone, v_dot2 alone and beside them)")
    mfma = runner.overlap_cycles(lib, 0, 1, 200, 1)
    dot2 = runner.overlap_cycles(lib, 3, 0, 200, 1)
    both = runner.overlap_cycles(lib, 3, 1, 200, 1)
    for v in (mfma, dot2, both):
        assert math.isfinite(v) and v > 0
    announce("microbench MFMA rate")
    lines = runner.mfma_rate(lib, target_ms=2.0, reps=1)
    assert len(lines) == 2 + 16
    announce("microbench MFMA beside VALU")
    lines = runner.contend(lib, iters=200, reps=1)
    # four partner modes per form, and the v_exp_f32 and v_dot2 streams beside the three bf16 forms
    assert len(lines) == 2 + sum(4 + (2 if form in (0, 1, 4) else 0) for form, _ in runner.CONTEND_FORMS)
    announce("microbench fp8 promotion")
    lines = runner.promote(lib, iters=100, reps=1)
    assert len(lines) == 2 + len(runner.PROMOTE_CASES)
    announce("microbench workgroup read")
    lines = runner.wg_read(lib, reps=2)
    assert len(lines) == 2 + 2 * (len(runner.WG_READ_CASES) + 1)
    announce("microbench read streams")
    lines = runner.stream(lib, reps=1)
    assert len(lines) == 2 + 2 * len(runner.STREAM_CASES) * len(runner.STREAM_DEPTHS)
