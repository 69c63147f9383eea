"""KDA decode parity on the GPU vs the CPU oracle (pytorch_reference_kda.py:42-73,
fp64).  Bounds: the reference's own acceptance gate, max_abs <= 1e-3 or
rel <= 1e-3 on o and on S (cutile-attn-kda/main.py:374-380), plus this
path's normwise bounds (o <= 2e-2 for the 16-bit output, S <= 1e-3)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import kda as okda
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL_O = 2e-2
TOL_S = 1e-3

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def run(ops, x, inplace=False):
    d = {k: v.cuda() for k, v in x.items()}
    o, s = ops.kda_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["S_in"],
                          S_out=d["S_in"] if inplace else None)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), s.cpu().numpy()


def reference_gate(got, want):
    err = float(np.abs(got - want).max())
    return err <= 1e-3 or err / (float(np.abs(want).max()) + 1e-30) <= 1e-3


def check(o, s, ro, rs):
    assert normwise_rel_err(torch.from_numpy(o), torch.from_numpy(ro)) <= TOL_O
    assert normwise_rel_err(torch.from_numpy(s), torch.from_numpy(rs)) <= TOL_S


def test_golden(ops):
    announce("kda golden correctness f16")
    g = load_golden("kda_correctness_f16")
    x = {n: from_bits(g[n], torch.float16) for n in ("q", "k", "v", "g", "beta")}
    x["S_in"] = torch.from_numpy(g["S_in"])
    o, s = run(ops, x)
    assert reference_gate(o, g["o"]) and reference_gate(s, g["S_out"])
    check(o, s, g["o"], g["S_out"])


@pytest.mark.parametrize("name", ["correctness", "kimi_linear_decode", "qwen3_next_gdn_parity", "large"])
def test_reference_shapes(ops, name):
    announce(f"kda {name} f16")
    x = inputs.kda_inputs(shapes.KDA_REGISTRY[name])
    o, s = run(ops, x)
    ro, rs = okda.kda_decode_ref(**x)
    assert reference_gate(o, ro) and reference_gate(s, rs)
    check(o, s, ro, rs)


DIMS = [(64, 64), (64, 256), (128, 128), (256, 64), (256, 256), (512, 512), (512, 128)]


@pytest.mark.parametrize("dk,dv", DIMS)
def test_head_dims_bf16(ops, dk, dv):
    announce(f"kda dk{dk} dv{dv} bf16")
    x = inputs.kda_inputs(shapes.KDAShape("t", batch=3, n_heads=5, d_k=dk, d_v=dv), dtype=torch.bfloat16)
    o, s = run(ops, x)
    ro, rs = okda.kda_decode_ref(**x)
    check(o, s, ro, rs)


def test_in_place_update(ops):
    announce("kda in-place")
    x = inputs.kda_inputs(shapes.KDA_KIMI_LINEAR)
    o, s = run(ops, x, inplace=True)
    ro, rs = okda.kda_decode_ref(**x)
    check(o, s, ro, rs)


def test_constant_gate_matches_gdn_kernel(ops):
    """g_i = log(alpha) on every channel: the KDA path equals the GDN path."""
    announce("kda == gdn at constant gate")
    s = shapes.KDAShape("t", batch=2, n_heads=8, d_k=128, d_v=128)
    x = inputs.kda_inputs(s, dtype=torch.bfloat16)
    x["g"] = torch.full((2, 8, 128), float(np.log(0.875)), dtype=torch.bfloat16)
    alpha = torch.exp(x["g"][..., 0].float())
    d = {k: v.cuda() for k, v in x.items()}
    o1, s1 = ops.kda_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["S_in"])
    o2, s2 = ops.gdn_decode(d["q"], d["k"], d["v"], alpha.cuda(), d["beta"].float(), d["S_in"])
    torch.cuda.synchronize()
    assert (s1 - s2).abs().max().item() <= 1e-6
    assert normwise_rel_err(o1.float().cpu(), o2.float().cpu()) <= 1e-2


def test_rejects_partial_overlap(ops):
    x = {k: v.cuda() for k, v in inputs.kda_inputs(shapes.KDAShape("t", 1, 4, 64, 64)).items()}
    flat = torch.empty(x["S_in"].numel() + 64, dtype=torch.float32, device="cuda")
    s_in = flat[:x["S_in"].numel()].view_as(x["S_in"])
    s_out = flat[64:].view_as(x["S_in"])
    with pytest.raises(Exception):
        ops.kda_decode(x["q"], x["k"], x["v"], x["g"], x["beta"], s_in, S_out=s_out)
