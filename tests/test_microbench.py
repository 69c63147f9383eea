"""The hardware characterisation probes (cuda-oxide-bench_amd/microbench):
the library builds with the package and exports its two launchers, which
reject invalid arguments before launching (CPU); one short run of each
probe on the GPU returns finite, positive figures (gpu)."""
from __future__ import annotations

import ctypes
import importlib.util
import math

import pytest

from conftest import REPO_ROOT, announce

RUN_PY = REPO_ROOT / "cuda-oxide-bench_amd" / "microbench" / "run.py"


@pytest.fixture(scope="module")
def runner():
    spec = importlib.util.spec_from_file_location("mx_microbench_run", RUN_PY)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_probe_library_exports_its_launchers(runner):
    lib = runner.load()
    for name in ("mxp_overlap_launch", "mxp_wg_read_launch"):
        assert hasattr(lib, name), name
    # invalid arguments are rejected before any HIP call
    assert lib.mxp_overlap_launch(0, 1, 0, 10, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert lib.mxp_overlap_launch(0, 1, 4, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert lib.mxp_overlap_launch(0, 1, 4, 10, None, ctypes.c_void_p(16), None) == -1
    assert lib.mxp_wg_read_launch(ctypes.c_void_p(16), 0, -1, 1, ctypes.c_void_p(16), None) == -1
    assert lib.mxp_wg_read_launch(None, 0, 8, 1, ctypes.c_void_p(16), None) == -1


@pytest.mark.gpu
def test_probes_run(runner):
    lib = runner.load()
    announce("microbench overlap (MFMAs alone, v_dot2 alone and beside them)")
    mfma = runner.overlap_cycles(lib, 0, 1, 200, 1)
    dot2 = runner.overlap_cycles(lib, 3, 0, 200, 1)
    both = runner.overlap_cycles(lib, 3, 1, 200, 1)
    for v in (mfma, dot2, both):
        assert math.isfinite(v) and v > 0
    announce("microbench workgroup read")
    lines = runner.wg_read(lib, reps=2)
    assert len(lines) == 2 + 2 * (len(runner.WG_READ_CASES) + 1)
