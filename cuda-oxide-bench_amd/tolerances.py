"""Correctness tolerances.

The per-dtype allclose table restates
analysis/wave15-attention-architecture/reference/tolerances.py:13-28.
The normwise bounds (max|got - ref| / max|ref|) are the acceptance
criteria of this path: 2e-2 for bf16 / fp8 outputs, 1e-3 for the fp32
GDN state.  The reference itself reports the same normwise quantity
(pytorch_reference.py:128-129, cutile-attn-gqa/main.py:259-262).
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Tolerance:
    atol: float
    rtol: float


TOLERANCES: dict[str, Tolerance] = {
    "f32": Tolerance(atol=1e-5, rtol=1e-5),
    "tf32": Tolerance(atol=1e-3, rtol=1e-3),
    "bf16": Tolerance(atol=1e-2, rtol=1e-2),
    "f16": Tolerance(atol=5e-3, rtol=5e-3),
}

NORMWISE_OUTPUT = 2e-2   # bf16 / fp8 outputs
NORMWISE_STATE = 1e-3    # fp32 GDN state


def get(dtype: str) -> Tolerance:
    return TOLERANCES[dtype]


def normwise_rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| over all elements (float64 arithmetic)."""
    import numpy as np

    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    denom = float(np.abs(r).max()) if r.size else 0.0
    return float(np.abs(g - r).max()) / (denom + 1e-30) if r.size else 0.0
