"""Pre-projected MLA prefill parity on the GPU (mx_mla_prefill_fwd) vs the
CPU oracle (mla_naive of pytorch_reference_mla.py:66-81).  Bounds: the
reference's f16 allclose gate (atol = rtol = 5e-3, cutile-attn-mla/
main.py:259-266) on its correctness shape; normwise <= 2e-2 elsewhere."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import mla as omla
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")
_lib = import_submodule("_lib")


def test_golden_reference_correctness_shape(ops):
    """Reference SHAPE_CORRECTNESS_MLA (1,128,4, qk 96, v 64), f16, reference recipe."""
    announce("mla prefill golden correctness f16")
    g = load_golden("mla_prefill_correctness_f16")
    q, k, v = (from_bits(g[x], torch.float16).cuda() for x in "qkv")
    o = ops.mla_prefill_fwd(q, k, v)
    torch.cuda.synchronize()
    o = o.float().cpu().numpy()
    assert np.allclose(o, g["o"], atol=5e-3, rtol=5e-3)


CASES = [
    # (B, S, H, d_qk, d_v, causal, dtype)
    (1, 2048, 128, 192, 128, False, torch.float16),   # reference bench shape (deepseek_v3)
    (1, 2048, 128, 192, 128, False, torch.bfloat16),
    (2, 300, 4, 192, 128, True, torch.bfloat16),      # ragged S, causal
    (1, 77, 3, 96, 64, False, torch.float16),
    (1, 190, 2, 96, 64, True, torch.bfloat16),
    (1, 129, 2, 128, 128, False, torch.bfloat16),
    (1, 1, 2, 192, 128, True, torch.float16),         # single token
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}S{c[1]}H{c[2]}qk{c[3]}v{c[4]}{'c' if c[5] else 'n'}")
def test_parity_vs_oracle(ops, case):
    B, S, H, dqk, dv, causal, dt = case
    announce(f"mla prefill B{B} S{S} H{H} qk{dqk} v{dv} causal={causal} {dt}")
    s = shapes.MLAShape("t", B, S, H, dqk - 64 if dqk > 64 else dqk // 2, 64 if dqk > 64 else dqk // 2, dv, 512,
                        causal)
    assert s.qk_head_dim == dqk
    q, k, v = inputs.mla_prefill_inputs(s, dtype=dt)
    o = ops.mla_prefill_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    heads = list(range(H)) if H * S <= 8192 else [0, 61, H - 1]
    ref = omla.mla_prefill_ref(q, k, v, causal=causal, heads=heads)
    err = normwise_rel_err(o.cpu()[:, heads], ref[:, heads])
    assert err <= TOL, f"normwise rel err {err:.3e}"


def test_unsupported_dims_rejected(ops):
    q = torch.zeros((1, 1, 64, 160), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros((1, 1, 64, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MXError) as e:
        ops.mla_prefill_fwd(q, q, v)
    assert e.value.code == _lib.MX_ERR_UNSUPPORTED
