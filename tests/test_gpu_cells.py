"""Every harness cell's --bench path on the GPU, in-process, with 2 timed
iterations: exit code 0, and a results.csv whose header starts with the
reference harness's column order (extra columns may only follow), one row
per iteration, positive timings.  Reference headers:
  GEMM cells        cutile-matmul-tc-bf16/main.py:170, cutile-matmul-tiled-mixed/main.py:212
  GQA               cutile-attn-gqa/main.py:316-317
  MLA               cutile-attn-mla/main.py:320-323
  GDN               cutile-attn-gdn/main.py:366-369; sweep cuda-attn-gdn-tma/bench_sweep.cu:314-315
  KDA               cutile-attn-kda/main.py:448-451
"""
from __future__ import annotations

import csv
import importlib.util
import sys

import pytest

from conftest import REPO_ROOT, announce

pytestmark = pytest.mark.gpu

CELLS = REPO_ROOT / "cuda-oxide-bench_amd" / "cells"
GEMM = ["impl", "kernel", "n", "iter", "gpu_ms", "tflops"]
GQA = ["impl", "kernel", "batch", "seq", "n_q", "n_kv", "d_head", "block_m", "block_n", "iter", "gpu_ms", "tflops"]
MLA = ["impl", "kernel", "batch", "seq", "n_h", "qk_head_dim", "qk_pad", "d_v", "block_m", "block_n", "iter",
       "gpu_ms", "tflops"]
GDN = ["impl", "kernel", "batch", "n_heads", "d_k", "d_v", "block_v", "iter", "gpu_us", "gbps", "tflops"]
GDN_SWEEP = ["impl", "kernel", "shape", "batch", "n_heads", "d_k", "d_v", "block_v", "n_blocks", "iter", "gpu_ms",
             "gbps", "gflops"]
KDA = GDN


def run_cell(cell: str, argv: list[str]) -> int:
    path = CELLS / cell / "main.py"
    spec = importlib.util.spec_from_file_location(f"cell_{cell.replace('-', '_')}", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    old = sys.argv
    sys.argv = [str(path), *argv]
    try:
        return mod.main()
    finally:
        sys.argv = old


def read_csv(path):
    with open(path, newline="") as f:
        rows = list(csv.reader(f))
    return rows[0], rows[1:]


@pytest.mark.parametrize("cell,argv,header,time_col,nrows", [
    ("hip-matmul-tc-bf16", ["--bench", "--n", "2048"], GEMM, "gpu_ms", 2),
    ("hip-matmul-tiled-mixed", ["--bench"], GEMM, "gpu_ms", 2 * 3),
    ("hip-matmul-fp8", ["--bench", "--n", "2048"], GEMM, "gpu_ms", 2),
    ("hip-attn-gqa", ["--bench"], GQA, "gpu_ms", 2),
    ("hip-attn-gqa", ["--bench", "--shape", "baseline", "--block-m", "64", "--block-n", "64"], GQA, "gpu_ms", 2),
    ("hip-attn-mla", ["--bench"], MLA, "gpu_ms", 2),
    ("hip-attn-mla", ["--bench", "--batch", "1", "--ctx", "32768"], MLA, "gpu_ms", 2),
    ("hip-attn-mla", ["--bench", "--mode", "prefill"], MLA, "gpu_ms", 2),
    ("hip-attn-gdn", ["--bench"], GDN, "gpu_us", 2),
    ("hip-attn-gdn", ["--bench", "--shape", "wide"], GDN, "gpu_us", 2),
    ("hip-attn-kda", ["--bench"], KDA, "gpu_us", 2),
])
def test_cell_bench_csv(tmp_path, cell, argv, header, time_col, nrows):
    announce(f"cell {cell} {' '.join(argv)}")
    out = tmp_path / "results.csv"
    rc = run_cell(cell, [*argv, "--iters", "2", "--csv-out", str(out)])
    assert rc == 0
    got, rows = read_csv(out)
    assert got[:len(header)] == header, f"{got} does not start with {header}"
    assert len(rows) == nrows
    k = got.index(time_col)
    assert all(float(r[k]) > 0 for r in rows)
    assert (tmp_path / "roofline.json").exists()


def test_gdn_sweep_csv(tmp_path):
    """--sweep over the reference sweep's five shapes, `wide` included."""
    announce("cell hip-attn-gdn --sweep")
    out = tmp_path / "results_sweep.csv"
    rc = run_cell("hip-attn-gdn", ["--sweep", "--iters", "2", "--warmup", "1", "--sweep-csv", str(out)])
    assert rc == 0
    got, rows = read_csv(out)
    assert got == GDN_SWEEP
    assert [r[2] for r in rows] == [s for s in ("qwen3_next_decode", "tiny", "small", "large", "wide") for _ in (0, 1)]
    for r in rows:
        d_v, bv, nblk = int(r[6]), int(r[7]), int(r[8])
        assert d_v % bv == 0 and nblk == int(r[3]) * int(r[4]) * (d_v // bv)


@pytest.mark.parametrize("argv", [["--block-m", "128"], ["--block-m", "256", "--block-n", "64"],
                                  ["--block-m", "128", "--wave-m", "64"]])
def test_gqa_tile_override_runs(tmp_path, argv):
    """--block-m / --block-n select the tile that runs (cutile-attn-gqa/main.py:202-230);
    results.csv reports it."""
    announce(f"cell hip-attn-gqa --bench {' '.join(argv)}")
    out = tmp_path / "results.csv"
    assert run_cell("hip-attn-gqa", ["--bench", *argv, "--iters", "2", "--csv-out", str(out)]) == 0
    got, rows = read_csv(out)
    bm = int(argv[argv.index("--block-m") + 1])
    wm = int(argv[argv.index("--wave-m") + 1]) if "--wave-m" in argv else 32
    assert all(int(r[got.index("block_m")]) == bm and int(r[got.index("block_n")]) == 64 for r in rows)
    assert all(int(r[got.index("wave_m")]) == wm for r in rows)


def test_gqa_tile_override_rejected(tmp_path):
    """A tile no kernel has (BLOCK_N other than the 64-key stage) fails like
    the reference's pick_blocks assertion (cutile-attn-gqa/main.py:213-219)."""
    announce("cell hip-attn-gqa --block-n 32 (rejected)")
    with pytest.raises(AssertionError):
        run_cell("hip-attn-gqa", ["--bench", "--block-m", "64", "--block-n", "32", "--iters", "2", "--csv-out",
                                  str(tmp_path / "r.csv")])


def test_gqa_block_m_sweep(tmp_path):
    """sweep_block_m.py: the reference's BLOCK_M sweep rows and CSV columns
    (cutile-attn-gqa/sweep_block_m.py, sweep_block_m_results.csv:1): 64 and
    128 pass the correctness shape, 256 is a compile-only SKIP there; every
    tile has a kernel at the bench shape.  wave_m is an appended column."""
    announce("cell hip-attn-gqa sweep_block_m.py")
    path = CELLS / "hip-attn-gqa" / "sweep_block_m.py"
    spec = importlib.util.spec_from_file_location("gqa_sweep", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = tmp_path / "sweep.csv"
    old = sys.argv
    sys.argv = [str(path), "--csv-out", str(out), "--wave-m", "32", "64"]
    try:
        assert mod.main() == 0
    finally:
        sys.argv = old
    got, rows = read_csv(out)
    assert got == ["block_m", "block_n", "correctness_status", "compile_status", "notes", "wave_m"]
    table = {(int(r[0]), int(r[5])): (r[2], r[3]) for r in rows}
    assert table[(64, 32)] == ("PASS", "OK") and table[(128, 32)] == ("PASS", "OK")
    assert table[(256, 32)] == ("SKIP", "OK") and table[(256, 64)] == ("SKIP", "OK")
    assert table[(128, 64)] == ("PASS", "OK")
    # 64-row blocks of 64-query waves would need 4 heads per workgroup: not at the correctness shape's G = 2
    assert table[(64, 64)][1] == "OK" and table[(64, 64)][0] == "ERROR"
    assert all(int(r[1]) == 64 for r in rows)
