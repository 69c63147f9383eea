"""MI355X (gfx950) quant-inference kernel path: bf16 / fp8 block-scaled GEMM,
fused causal GQA forward, MLA absorbed decode and GDN decode.

The package directory name is not a Python identifier; import it with
``importlib.import_module("cuda-oxide-bench_amd")`` after putting the repo
root on ``sys.path`` (``__graft_entry__`` and the tests do this).

Operators live in ``.ops`` and call hand-written HIP kernels through the
C-ABI library ``libmxkernels.so`` (include/mx_kernels.h).
"""
from __future__ import annotations

from . import flops, inputs, quant, shapes, tolerances  # noqa: F401

__version__ = "0.1.0"


def load_ops():
    """Load the native library and return the operator module."""
    import importlib

    from . import _lib

    _lib.load()
    return importlib.import_module(__name__ + ".ops")
