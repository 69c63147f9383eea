"""The harness cells (drop-in replacements of the reference's main.py
harnesses) expose the reference's flags; checked via --help on the CPU."""
from __future__ import annotations

import subprocess
import sys

import pytest

from conftest import REPO_ROOT

CELLS = {
    "hip-matmul-tc-bf16": ["--smoke", "--bench", "--n", "--csv-out"],
    "hip-matmul-fp8": ["--smoke", "--bench", "--n", "--csv-out"],
    "hip-attn-gqa": ["--smoke", "--bench", "--export-cubin", "--csv-out", "--cubin-out", "--block-m", "--block-n",
                     "--iters"],
    "hip-attn-mla": ["--smoke", "--bench", "--export-cubin", "--csv-out", "--cubin-out"],
    "hip-attn-gdn": ["--smoke", "--bench", "--export-cubin", "--csv-out", "--cubin-out", "--shape"],
    "hip-attn-kda": ["--smoke", "--bench", "--export-cubin", "--csv-out", "--cubin-out", "--shape"],
}


@pytest.mark.parametrize("cell", sorted(CELLS))
def test_cell_cli(cell):
    main = REPO_ROOT / "cuda-oxide-bench_amd" / "cells" / cell / "main.py"
    out = subprocess.run([sys.executable, str(main), "--help"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    for flag in CELLS[cell]:
        assert flag in out.stdout, f"{cell}: {flag} missing"
