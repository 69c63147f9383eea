"""Host AddressSanitizer run of the C-ABI's argument validation (no GPU).

Builds the debug variant of the library with ASan on its host code
(`build.build_host_asan`, device code as usual) and runs the validation
driver tests/asan/capi_validation.cpp against it: every entry point is
called with arguments its checks must reject, and ASan watches those host
paths for invalid memory accesses.  The driver exits 0 only when every call
returns the expected status and ASan reports nothing."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import import_submodule


def test_capi_validation_under_asan(tmp_path):
    build = import_submodule("build")
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if not os.path.exists(build.clangxx()) and not shutil.which("clang++"):
        pytest.skip("clang++ not available")
    driver = build.build_host_asan(out_dir=tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=23")
    proc = subprocess.run([str(driver)], capture_output=True, text=True, timeout=120, env=env)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "capi_validation: 0 failure(s)" in proc.stdout
    assert "AddressSanitizer" not in proc.stderr
