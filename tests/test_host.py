"""Host-side logic on the CPU: operator argument validation (no GPU path and
no CPU fallback), the FLOP/byte model against the figures this path quotes,
and input generator determinism."""
from __future__ import annotations

import pytest
import torch

from conftest import import_submodule

shapes = import_submodule("shapes")
flops = import_submodule("flops")
inputs = import_submodule("inputs")
ops = import_submodule("ops")


def test_ops_refuse_cpu_tensors():
    a = torch.zeros((16, 16), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        ops.gemm_bf16(a, a)
    q = torch.zeros((1, 4, 16, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        ops.gqa_fwd(q, q[:, :2], q[:, :2], causal=True)


def test_ops_type_checks():
    with pytest.raises(TypeError):
        ops.gemm_bf16(torch.zeros((16, 16)), torch.zeros((16, 16)))


def test_flop_and_byte_model_matches_quoted_figures():
    assert flops.gemm_flops(shapes.GEMM_PARITY) == 2_147_483_648
    assert flops.gemm_bf16_bytes(shapes.GEMM_PARITY) == 6_291_456
    assert flops.gemm_flops(shapes.GEMM_TARGET) == 1_099_511_627_776
    assert flops.gemm_fp8_bytes(shapes.FP8_TARGET) == 270_548_992
    g = shapes.GQA_BASELINE
    assert flops.gqa_causal_flops(g) == 137_472_507_904
    assert flops.gqa_attention_flops(g) == 274_877_906_944
    assert flops.gqa_attention_bytes(g) == 83_886_080
    m = shapes.MLA_BASELINE
    assert flops.mla_decode_bytes(m) == 159_907_840
    assert flops.mla_decode_flops(m) == 36_507_222_016
    d = shapes.GDN_BASELINE
    assert flops.gdn_decode_bytes(d) == 270_024_704
    assert flops.gdn_decode_flops(d) == 201_326_592
    # reference convention (flops_gdn.py:59-70) at its own shape with f16 gates
    r = shapes.GDN_QWEN3_NEXT
    assert flops.gdn_decode_bytes(r, gate_bytes=2) == 16 * (2 * 256 * 256 * 4 + (2 * 256 + 2 * 256 + 2) * 2)


def test_causal_flops_closed_form():
    s = shapes.GQAShape("t", 1, 5, 1, 1, 2, True)
    # sum_{i<5} (i+1) = 15 keys; QK^T and PV each 2*D per key
    assert flops.gqa_causal_flops(s) == 15 * 2 * 2 * 2


def test_inputs_deterministic():
    a1, b1 = inputs.gemm_inputs(shapes.GemmShape("t", 8, 16, 8))
    a2, b2 = inputs.gemm_inputs(shapes.GemmShape("t", 8, 16, 8))
    assert torch.equal(a1, a2) and torch.equal(b1, b2)
    assert a1.float().abs().max() <= 1.0 and a1.float().min() < 0


def test_missing_library_fails_loudly(tmp_path):
    """With the kernel library absent the package raises at load time; there
    is no CPU fallback to route to."""
    import os
    import subprocess
    import sys

    from conftest import REPO_ROOT

    code = ("import importlib, sys; sys.path.insert(0, %r)\n"
            "pkg = importlib.import_module('cuda-oxide-bench_amd')\n"
            "try:\n    pkg.load_ops()\nexcept ImportError as e:\n    print('ImportError:', e); sys.exit(3)\n"
            "sys.exit(0)\n") % str(REPO_ROOT)
    env = dict(os.environ, MX_KERNELS_LIB=str(tmp_path / "libmxkernels.so"))
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert proc.returncode == 3, proc.stdout + proc.stderr
    assert "not found" in proc.stdout
