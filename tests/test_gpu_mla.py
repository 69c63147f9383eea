"""MLA absorbed decode parity on the GPU vs the CPU oracle (mla_naive of
pytorch_reference_mla.py:66-81 with one shared latent KV head).  Bound:
normwise <= 2e-2 (bf16 output)."""
from __future__ import annotations

import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import mla as omla
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def run(ops, q, kv, scale):
    o = ops.mla_decode(q.cuda(), kv.cuda(), scale)
    torch.cuda.synchronize()
    return o.cpu()


def test_golden(ops):
    announce("mla golden H16 T40")
    g = load_golden("mla_decode_h16_t40")
    q, kv = from_bits(g["q"], torch.bfloat16), from_bits(g["kv"], torch.bfloat16)
    o = run(ops, q, kv, float(g["scale"][0]))
    assert normwise_rel_err(o, g["o"]) <= TOL


@pytest.mark.parametrize("bht", [(2, 16, 200), (1, 128, 1), (1, 128, 33), (3, 20, 500), (4, 128, 1024),
                                 (1, 128, 4096), (2, 64, 4100)])
def test_parity_vs_oracle(ops, bht):
    B, H, T = bht
    announce(f"mla B{B} H{H} T{T}")
    s = shapes.MLADecodeShape("t", B, H, T)
    q, kv = inputs.mla_inputs(s)
    o = run(ops, q, kv, s.scale)
    ref = omla.mla_decode_ref(q, kv, s.scale)
    err = normwise_rel_err(o, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"


def test_single_token_returns_its_latent(ops):
    announce("mla T=1 special case")
    s = shapes.MLADecodeShape("t", 2, 32, 1)
    q, kv = inputs.mla_inputs(s)
    o = run(ops, q, kv, s.scale).float()
    want = kv[:, 0, :512].float()[:, None, :].expand(2, 32, 512)
    assert torch.allclose(o, want, atol=1e-2, rtol=1e-2)


def test_baseline_config(ops):
    """BASELINE config B32 H128 T4096: four sequences against the oracle."""
    announce("mla BASELINE B32 H128 T4096")
    s = shapes.MLA_BASELINE
    q, kv = inputs.mla_inputs(s)
    o = run(ops, q, kv, s.scale)
    bs = [0, 7, 20, 31]
    ref = omla.mla_decode_ref(q, kv, s.scale, batches=bs)
    err = normwise_rel_err(o[bs], ref[bs])
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.isfinite(o.float()).all()
