"""Error metrics used by the parity checks (test infrastructure only).

normwise_rel_err is the quantity the reference reports as `rel_err`
(analysis/wave15-attention-architecture/reference/pytorch_reference.py:128-129,
cutile-attn-gqa/main.py:259-262): max|got - ref| / max|ref|.
"""
from __future__ import annotations

import numpy as np


def to_f64(x) -> np.ndarray:
    try:
        import torch

        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", dtype=torch.float64).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(x, dtype=np.float64)


def normwise_rel_err(got, ref) -> float:
    g, r = to_f64(got), to_f64(ref)
    if r.size == 0:
        return 0.0
    return float(np.abs(g - r).max() / (np.abs(r).max() + 1e-30))


def max_abs_err(got, ref) -> float:
    g, r = to_f64(got), to_f64(ref)
    return float(np.abs(g - r).max()) if r.size else 0.0
