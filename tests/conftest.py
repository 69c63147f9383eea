"""Shared pytest setup: repo root on sys.path, the `gpu` marker, package handles."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))

PKG_NAME = "cuda-oxide-bench_amd"
GOLDEN_DIR = REPO_ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built kernel library")


def import_pkg():
    return importlib.import_module(PKG_NAME)


def import_submodule(name: str):
    return importlib.import_module(f"{PKG_NAME}.{name}")


@pytest.fixture(scope="session")
def pkg():
    return import_pkg()


@pytest.fixture(scope="session")
def ops():
    """The operator module; GPU tests only.  Fails (never skips) if the GPU or
    the native library is missing, so a GPU run cannot pass vacuously."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    p = import_pkg()
    return p.load_ops()


def load_golden(name: str) -> dict:
    import numpy as np

    with np.load(GOLDEN_DIR / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def from_bits(arr, dtype):
    """uint16 bit patterns -> torch bf16/f16 tensor (CPU)."""
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(dtype)


def announce(msg: str) -> None:
    """Print the case about to run on the GPU (flushed first, so a fault names it)."""
    print(f"[case] {msg}", flush=True)
