"""GDN decode parity on the GPU vs the CPU oracle (fused form of
pytorch_reference_gdn.py:38-91).  Bounds: o normwise <= 2e-2 (bf16/f16
output), S_out normwise <= 1e-3 (fp32 state)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import gdn as ogdn
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL_O = 2e-2
TOL_S = 1e-3

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def to_dev(x):
    return {k: v.cuda() for k, v in x.items()}


def run(ops, x, inplace=False):
    d = to_dev(x)
    if inplace:
        o, s = ops.gdn_decode(d["q"], d["k"], d["v"], d["alpha"], d["beta"], d["S_in"], S_out=d["S_in"])
    else:
        o, s = ops.gdn_decode(d["q"], d["k"], d["v"], d["alpha"], d["beta"], d["S_in"])
    torch.cuda.synchronize()
    return o.cpu(), s.cpu()


@pytest.mark.parametrize("name,dt", [("gdn_correctness_f16", torch.float16), ("gdn_grouped_bf16", torch.bfloat16)])
def test_golden(ops, name, dt):
    announce(f"gdn golden {name}")
    g = load_golden(name)
    x = {"q": from_bits(g["q"], dt), "k": from_bits(g["k"], dt), "v": from_bits(g["v"], dt),
         "alpha": torch.from_numpy(g["alpha"]), "beta": torch.from_numpy(g["beta"]),
         "S_in": torch.from_numpy(g["S_in"])}
    o, s = run(ops, x)
    assert normwise_rel_err(o, g["o"]) <= TOL_O
    assert normwise_rel_err(s, g["S_out"]) <= TOL_S
    if dt == torch.float16:  # the reference's own gate: f16 allclose on o, 5e-3 on S (main.py:283-298)
        assert np.allclose(o.float().numpy(), g["o"], atol=5e-3, rtol=5e-3)
        assert np.abs(s.numpy() - g["S_out"]).max() < 5e-3


DIMS = [(64, 64), (64, 128), (128, 64), (128, 128), (128, 256), (256, 128), (256, 256), (64, 256), (256, 64),
        (512, 512), (512, 64), (64, 512), (512, 256)]


@pytest.mark.parametrize("dk,dv", DIMS)
def test_all_head_dims(ops, dk, dv):
    announce(f"gdn dk{dk} dv{dv}")
    s = shapes.GDNShape("t", batch=3, n_heads=4, d_k=dk, d_v=dv, n_k_heads=2)
    x = inputs.gdn_inputs(s)
    o, so = run(ops, x)
    ro, rs = ogdn.gdn_decode_ref(**x)
    assert normwise_rel_err(o, ro) <= TOL_O
    assert normwise_rel_err(so, rs) <= TOL_S


def test_wide_reference_shape(ops):
    """The reference registry's `wide` shape (B1 H16 d_k = d_v = 512,
    cutile-attn-gdn/main.py:65) on reference-distribution f16 inputs, with
    the column blocks the kernel picks reported by mx_gdn_decode_block_v."""
    announce("gdn wide B1 H16 d512 f16")
    s = shapes.GDN_REGISTRY["wide"]
    bv = ops.gdn_block_v(s.batch, s.n_heads, s.d_k, s.d_v)
    assert 16 <= bv <= 128 and s.d_v % bv == 0
    x = inputs.gdn_inputs(s, dtype=torch.float16, dist="reference")
    o, so = run(ops, x)
    ro, rs = ogdn.gdn_decode_ref(**x)
    assert normwise_rel_err(o, ro) <= TOL_O
    assert normwise_rel_err(so, rs) <= TOL_S
    assert np.abs(so.numpy() - rs.numpy()).max() < 5e-3  # the reference's S gate (main.py:298)


def test_baseline_config(ops):
    """BASELINE config: B64 Hk16 Hv32 d128, fp32 state, bf16 q/k/v."""
    announce("gdn BASELINE B64 Hk16 Hv32 d128")
    x = inputs.gdn_inputs(shapes.GDN_BASELINE)
    o, so = run(ops, x)
    ro, rs = ogdn.gdn_decode_ref(**x)
    eo, es = normwise_rel_err(o, ro), normwise_rel_err(so, rs)
    assert eo <= TOL_O, f"o err {eo:.3e}"
    assert es <= TOL_S, f"S err {es:.3e}"


def test_reference_shape_f16(ops):
    """Reference bench shape qwen3_next_decode (B1 H16 d256) with reference inputs."""
    announce("gdn reference qwen3_next_decode f16")
    x = inputs.gdn_inputs(shapes.GDN_QWEN3_NEXT, dtype=torch.float16, dist="reference")
    o, so = run(ops, x)
    ro, rs = ogdn.gdn_decode_ref(**x)
    assert normwise_rel_err(o, ro) <= TOL_O
    assert normwise_rel_err(so, rs) <= TOL_S


def test_in_place_update(ops):
    announce("gdn in-place")
    s = shapes.GDNShape("t", batch=4, n_heads=8, d_k=128, d_v=128, n_k_heads=4)
    x = inputs.gdn_inputs(s)
    ro, rs = ogdn.gdn_decode_ref(**x)
    o, so = run(ops, x, inplace=True)
    assert normwise_rel_err(so, rs) <= TOL_S
    assert normwise_rel_err(o, ro) <= TOL_O


def test_partial_overlap_rejected(ops):
    s = shapes.GDNShape("t", batch=2, n_heads=2, d_k=64, d_v=64)
    x = to_dev(inputs.gdn_inputs(s))
    buf = torch.zeros(2 * x["S_in"].numel(), dtype=torch.float32, device="cuda")
    S_in = buf[: x["S_in"].numel()].view_as(x["S_in"])
    S_out = buf[64: 64 + x["S_in"].numel()].view_as(x["S_in"])
    with pytest.raises(Exception, match="overlaps"):
        ops.gdn_decode(x["q"], x["k"], x["v"], x["alpha"], x["beta"], S_in, S_out=S_out)
