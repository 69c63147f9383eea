"""GEMM oracle (test infrastructure only).

C = A @ B computed in fp32 from the bf16-rounded operands, as the
reference's CPU check does: cutile-matmul-tc-bf16/main.py:98-107 promotes
both operands to f32 before the product; cuda-matmul-tc-bf16/matmul_tc_bf16.cu:201-207
(ref_elem) accumulates a single cell in double.
"""
from __future__ import annotations

import numpy as np
import torch


def gemm_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Full fp32 product of (bf16) a [M,K] and b [K,N] on the CPU."""
    return a.detach().cpu().float() @ b.detach().cpu().float()


def gemm_ref_f64(a, b) -> np.ndarray:
    """Double-precision product (the accuracy anchor for the fp32 oracle)."""
    a64 = torch.as_tensor(a).detach().cpu().double().numpy()
    b64 = torch.as_tensor(b).detach().cpu().double().numpy()
    return a64 @ b64


def ref_elem(a32: np.ndarray, b32: np.ndarray, row: int, col: int) -> float:
    """One cell accumulated in double (cuda-matmul-tc-bf16/matmul_tc_bf16.cu:201-207)."""
    return float(np.dot(a32[row, :].astype(np.float64), b32[:, col].astype(np.float64)))


def sample_reference(a: torch.Tensor, b: torch.Tensor, rows, cols) -> np.ndarray:
    """fp32 dot products for the requested (row, col) cells
    (cutile-matmul-tc-bf16/main.py:98-107)."""
    a32 = a.detach().cpu().float().numpy()
    b32 = b.detach().cpu().float().numpy()
    return np.array([np.dot(a32[r, :], b32[:, c]) for r, c in zip(rows, cols)], dtype=np.float32)
