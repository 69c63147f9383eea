"""Pin the GEMM oracle (CPU): known answers, closed form, fp64 brute force."""
from __future__ import annotations

import numpy as np
import torch

from conftest import import_submodule
from oracle import gemm as ogemm

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_kat_constants():
    """oxide-gemm-sol/bench/cublas_correctness_test.py:8-11: A=1,B=1 -> K; A=2,B=3 -> 6K."""
    for k in (8, 512):
        a = torch.ones((16, k), dtype=torch.bfloat16)
        b = torch.ones((k, 24), dtype=torch.bfloat16)
        assert torch.all(ogemm.gemm_ref(a, b) == k)
        assert torch.all(ogemm.gemm_ref(2 * a, 3 * b) == 6 * k)


def test_kat_pattern():
    m, n, k = 40, 24, 64
    a = (torch.arange(m) % 8 + 1).float()[:, None].expand(m, k).to(torch.bfloat16)
    b = (torch.arange(n) % 8 + 1).float()[None, :].expand(k, n).to(torch.bfloat16)
    want = ((torch.arange(m) % 8 + 1)[:, None] * (torch.arange(n) % 8 + 1)[None, :] * k).float()
    assert torch.equal(ogemm.gemm_ref(a, b), want)


def test_closed_form_cell_matches_reference_log():
    """cuda-matmul-tc-bf16/matmul_tc_bf16.cu:228-233 inputs a[i]=(i%7)*0.01,
    b[i]=(i%11)*0.01 at N=4096.  The reference logs, at cell (746, 1839),
    want=6.1455 — its ref_elem (:201-207) over the fp32 inputs — and
    got=6.1520 from its bf16 GPU kernel (cuda-matmul-tc-bf16/ANALYSIS.md:17).
    The oracle reproduces both: the fp64 dot of the fp32 inputs, and the
    fp32-accumulated dot of the bf16 (round-to-nearest-even) inputs."""
    n = 4096
    row, col = 746, 1839
    idx_a = row * n + np.arange(n)
    idx_b = np.arange(n) * n + col
    af = ((idx_a % 7) * 0.01).astype(np.float32)
    bf = ((idx_b % 11) * 0.01).astype(np.float32)
    assert abs(ogemm.ref_elem(af[None, :], bf[:, None], 0, 0) - 6.1455) < 5e-5
    a = torch.from_numpy(af).to(torch.bfloat16)[None, :]
    b = torch.from_numpy(bf).to(torch.bfloat16)[:, None]
    # 4-decimal log value; the GPU's fp32 summation order over 4096 terms
    # moves the fourth decimal by a few 1e-5, so the pin is to 2e-4.
    assert abs(float(ogemm.gemm_ref(a, b)[0, 0]) - 6.1520) < 2e-4
    # ...and rounding the inputs to bf16 is what moves the value off 6.1455.
    assert abs(float(ogemm.gemm_ref(a, b)[0, 0]) - 6.1455) > 5e-3


def test_fp32_oracle_vs_fp64_bruteforce():
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", 7, 9, 13), seed=3)
    ref = ogemm.gemm_ref(a, b).double().numpy()
    a64, b64 = a.double().numpy(), b.double().numpy()
    brute = np.zeros((7, 9))
    for i in range(7):
        for j in range(9):
            s = 0.0
            for t in range(13):
                s += a64[i, t] * b64[t, j]
            brute[i, j] = s
    assert np.abs(ref - brute).max() <= 1e-5 * max(1.0, np.abs(brute).max())
    assert np.allclose(ogemm.gemm_ref_f64(a, b), brute, rtol=0, atol=1e-12)


def test_sampled_reference_matches_full():
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", 64, 48, 32), seed=5)
    full = ogemm.gemm_ref(a, b).numpy()
    rows, cols = [0, 5, 63], [0, 47, 11]
    assert np.allclose(ogemm.sample_reference(a, b, rows, cols), full[rows, cols], rtol=1e-6, atol=1e-6)
