"""Fixture interop on the CPU: the NPY contract of the reference's native
loader (cuda-attn-gqa/attn_gqa.cu:55-111), the reference's inputs/ file
names, and the master results table (results/scaling.csv:1)."""
from __future__ import annotations

import csv
import struct

import numpy as np
import pytest

from conftest import REPO_ROOT, import_submodule

npy = import_submodule("npy")
collect = import_submodule("collect_results")


def raw_npy(path, descr, shape, payload: bytes, version=(1, 0), fortran=False):
    hdr = f"{{'descr': '{descr}', 'fortran_order': {fortran}, 'shape': {shape!r}, }}".encode("latin1") + b"\n"
    ln = struct.pack("<H", len(hdr)) if version[0] == 1 else struct.pack("<I", len(hdr))
    path.write_bytes(b"\x93NUMPY" + bytes(version) + ln + hdr + payload)
    return path


@pytest.mark.parametrize("version", [(1, 0), (2, 0), (3, 0)])
@pytest.mark.parametrize("dt,descr", [(np.float16, "<f2"), (np.float32, "<f4")])
def test_reads_all_header_versions(tmp_path, version, dt, descr):
    a = (np.arange(24, dtype=np.float64).reshape(2, 3, 4) / 7 - 1).astype(dt)
    p = raw_npy(tmp_path / "a.npy", descr, (2, 3, 4), a.tobytes(), version)
    b = npy.read_npy(p)
    assert b.dtype == dt and b.shape == (2, 3, 4)
    assert np.array_equal(b, a)


def test_reads_numpy_written_files(tmp_path):
    for shape in [(5,), (1, 4, 128, 64), (0, 3), ()]:
        a = np.random.default_rng(1).standard_normal(shape).astype(np.float32)
        np.save(tmp_path / "n.npy", a)
        assert np.array_equal(npy.read_npy(tmp_path / "n.npy"), a)


def test_write_is_numpy_readable_and_aligned(tmp_path):
    for a in [np.float16([1.5, -2.0, 65504.0]), np.float32(np.arange(12).reshape(3, 4)), np.zeros((2, 0), np.float32)]:
        p = npy.write_npy(tmp_path / "w.npy", a)
        b = np.load(p, allow_pickle=False)
        assert b.dtype == a.dtype and np.array_equal(b, a)
        assert (p.stat().st_size - a.nbytes) % 64 == 0  # header padded to 64 bytes as numpy does
        assert np.array_equal(npy.read_npy(p), a)


@pytest.mark.parametrize("case", ["magic", "dtype", "fortran", "short", "truncated", "version"])
def test_rejections(tmp_path, case):
    p = tmp_path / "bad.npy"
    if case == "magic":
        p.write_bytes(b"\x93NUMPX\x01\x00\x00\x00")
    elif case == "dtype":
        raw_npy(p, "<f8", (2,), np.zeros(2).tobytes())
    elif case == "fortran":
        raw_npy(p, "<f4", (2, 2), np.zeros(4, np.float32).tobytes(), fortran=True)
    elif case == "short":
        raw_npy(p, "<f4", (4,), np.zeros(3, np.float32).tobytes())
    elif case == "truncated":
        p.write_bytes(b"\x93NUMPY\x01\x00\xff\x00{'descr'")
    else:
        p.write_bytes(b"\x93NUMPY\x04\x00\x00\x00")
    with pytest.raises(npy.NpyError):
        npy.read_npy(p)
    with pytest.raises(npy.NpyError):
        npy.read_npy(tmp_path / "absent.npy")


def test_write_rejects_other_dtypes(tmp_path):
    with pytest.raises(npy.NpyError):
        npy.write_npy(tmp_path / "x.npy", np.zeros(3, np.float64))


def test_fixture_set_names_and_roundtrip(tmp_path):
    """File names are the reference's (pytorch_reference_gdn.py:215-228);
    the 16-bit roles are stored as float16 and the state as float32."""
    rng = np.random.default_rng(0)
    arrays = {"q": rng.standard_normal((2, 4, 64)), "k": rng.standard_normal((2, 4, 64)),
              "v": rng.standard_normal((2, 4, 64)), "alpha": rng.random((2, 4)), "beta": rng.random((2, 4)),
              "S_in": rng.standard_normal((2, 4, 64, 64)), "o_expected": rng.standard_normal((2, 4, 64)),
              "S_out_expected": rng.standard_normal((2, 4, 64, 64))}
    paths = npy.save_fixture_set(tmp_path, "gdn", "correctness", arrays)
    names = sorted(p.name for p in paths)
    assert names == sorted(f"gdn_correctness_{s}.npy" for s in
                           ["q_f16", "k_f16", "v_f16", "alpha_f16", "beta_f16", "S_in_f32", "o_expected_f16",
                            "S_out_expected_f32"])
    fx = npy.load_fixture_set(tmp_path, "gdn", "correctness")
    assert fx["q"].dtype == np.float16 and fx["S_in"].dtype == np.float32
    assert np.array_equal(fx["alpha"], arrays["alpha"].astype(np.float16))
    assert np.array_equal(fx["S_out_expected"], arrays["S_out_expected"].astype(np.float32))


def test_missing_fixture_files_are_all_named(tmp_path):
    npy.write_npy(tmp_path / "gqa_tiny_q_f16.npy", np.zeros((1, 1, 2, 64), np.float16))
    with pytest.raises(npy.NpyError) as e:
        npy.load_fixture_set(tmp_path, "gqa", "tiny")
    msg = str(e.value)
    for s in ("k_f16", "v_f16", "expected_f32"):
        assert f"gqa_tiny_{s}.npy" in msg
    assert "gqa_tiny_q_f16.npy" not in msg
    with pytest.raises(npy.NpyError):
        npy.load_fixture_set(tmp_path, "nope", "tiny")


def write_csv(path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    return path


def test_master_table_from_cell_schemas(tmp_path):
    gemm = write_csv(tmp_path / "hip-matmul-tc-bf16" / "results.csv", ["impl", "kernel", "n", "iter", "gpu_ms", "tflops"],
                     [["hip", "gemm", 1024, i, ms, 2.147483648 / ms] for i, ms in enumerate([0.02, 0.01, 0.04, 0.03])])
    gqa = write_csv(tmp_path / "hip-attn-gqa" / "results.csv",
                    ["impl", "kernel", "batch", "seq", "n_q", "n_kv", "d_head", "block_m", "block_n", "iter", "gpu_ms",
                     "tflops", "causal", "dtype", "tflops_causal"],
                    [["hip", "gqa_fwd_fused", 1, 4096, 32, 8, 128, 32, 64, 0, 0.15, 1800.0, 1, "bf16", 900.0]])
    gdn = write_csv(tmp_path / "hip-attn-gdn" / "results.csv",
                    ["impl", "kernel", "batch", "n_heads", "d_k", "d_v", "block_v", "iter", "gpu_us", "gbps", "tflops"],
                    [["hip", "gdn_decode", 64, 32, 128, 128, 64, 0, 40.0, 6750.0, 5.0],
                     ["hip", "gdn_decode", 64, 32, 128, 128, 64, 1, 42.0, 6430.0, 4.8]])
    out = tmp_path / "master.csv"
    summ = tmp_path / "summary.md"
    assert collect.main(["--out", str(out), "--summary", str(summ), str(gemm), str(gqa), str(gdn)]) == 0
    rows = list(csv.DictReader(open(out)))
    assert list(rows[0].keys()) == collect.MASTER_HEADER
    assert len(rows) == 7
    g = [r for r in rows if r["cell"] == "hip-attn-gdn"]
    assert g[0]["unit"] == "GB/s" and float(g[0]["gpu_ms"]) == pytest.approx(0.040) and float(g[0]["rate"]) == 6750.0
    assert g[0]["config"] == "batch=64;n_heads=32;d_k=128;d_v=128;block_v=64"
    q = [r for r in rows if r["cell"] == "hip-attn-gqa"][0]
    assert q["unit"] == "TFLOPS" and "causal=1" in q["config"] and "dtype=bf16" in q["config"]
    st = {s["cell"]: s for s in collect.summarize(collect.read_cell_csv(gemm))}["hip-matmul-tc-bf16"]
    assert st["n"] == 4 and st["best_ms"] == pytest.approx(0.01) and st["median_ms"] == pytest.approx(0.025)
    assert st["iqr_ms"] == pytest.approx(0.0325 - 0.0175)  # inclusive quartiles of 0.01..0.04
    assert st["cv_pct"] == pytest.approx(np.std([0.01, 0.02, 0.03, 0.04], ddof=1) / 0.025 * 100)
    assert "| hip-attn-gdn | hip | gdn_decode |" in summ.read_text()


def test_master_table_rejects_foreign_csv(tmp_path):
    p = write_csv(tmp_path / "x" / "results.csv", ["a", "b"], [[1, 2]])
    with pytest.raises(ValueError):
        collect.read_cell_csv(p)


def test_cells_offer_fixture_replay():
    import subprocess
    import sys

    for cell in ("hip-attn-gqa", "hip-attn-gdn", "hip-attn-kda", "hip-attn-mla"):
        main = REPO_ROOT / "cuda-oxide-bench_amd" / "cells" / cell / "main.py"
        out = subprocess.run([sys.executable, str(main), "--help"], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0 and "--inputs-dir" in out.stdout and "--fixture" in out.stdout
