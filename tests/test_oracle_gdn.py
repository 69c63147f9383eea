"""Pin the GDN oracle (CPU): fused vs canonical form (pytorch_reference_gdn.py:201-213),
closed-form special cases, grouping equivalence, fp64 loops."""
from __future__ import annotations

import numpy as np
import torch

from conftest import import_submodule
from oracle import gdn as ogdn

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_fused_vs_canonical():
    for s, dist, dt in ((shapes.GDN_CORRECTNESS, "reference", torch.float16),
                        (shapes.GDNShape("t", 2, 4, 128, 128, 2), "baseline", torch.bfloat16)):
        x = inputs.gdn_inputs(s, dtype=dt, dist=dist)
        o1, s1 = ogdn.gdn_decode_ref(**x)
        o2, s2 = ogdn.gdn_decode_canonical(**x)
        assert (o1 - o2).abs().max().item() < 1e-3
        assert (s1 - s2).abs().max().item() < 1e-3


def test_beta_zero_is_pure_decay():
    x = inputs.gdn_inputs(shapes.GDNShape("t", 2, 2, 32, 48))
    x["beta"] = torch.zeros_like(x["beta"])
    _, s = ogdn.gdn_decode_ref(**x)
    assert torch.allclose(s, x["alpha"][..., None, None] * x["S_in"], atol=0, rtol=0)


def test_delta_rule_write():
    """With beta |k|^2 = 1 the updated state maps k exactly to v: k^T S' = v."""
    x = inputs.gdn_inputs(shapes.GDNShape("t", 2, 3, 64, 32), dtype=torch.bfloat16)
    kf = x["k"].float()
    x["beta"] = (1.0 / (kf * kf).sum(-1)).expand(2, 3).contiguous()
    _, s = ogdn.gdn_decode_ref(**x)
    ks = torch.einsum("bhk,bhkv->bhv", kf, s)
    assert torch.allclose(ks, x["v"].float(), atol=1e-4)


def test_alpha_one_beta_zero_reads_state():
    x = inputs.gdn_inputs(shapes.GDNShape("t", 1, 2, 16, 16))
    x["alpha"] = torch.ones_like(x["alpha"])
    x["beta"] = torch.zeros_like(x["beta"])
    o, _ = ogdn.gdn_decode_ref(**x)
    want = torch.einsum("bhk,bhkv->bhv", x["q"].float(), x["S_in"])
    assert torch.allclose(o, want, atol=1e-6)


def test_grouping_equals_duplicated_keys():
    x = inputs.gdn_inputs(shapes.GDNShape("t", 2, 4, 32, 32, n_k_heads=2))
    o, s = ogdn.gdn_decode_ref(**x)
    y = dict(x)
    y["q"] = x["q"].repeat_interleave(2, dim=1)
    y["k"] = x["k"].repeat_interleave(2, dim=1)
    o2, s2 = ogdn.gdn_decode_ref(**y)
    assert torch.equal(o, o2) and torch.equal(s, s2)


def test_fp64_loops():
    x = inputs.gdn_inputs(shapes.GDNShape("t", 1, 2, 4, 3, n_k_heads=1), dtype=torch.float16)
    o, s = ogdn.gdn_decode_ref(**x)
    q, k, v = (x[n].double().numpy() for n in "qkv")
    a, b, S = x["alpha"].double().numpy(), x["beta"].double().numpy(), x["S_in"].double().numpy()
    for h in range(2):
        Sh = S[0, h]
        u = [sum(k[0, 0, i] * a[0, h] * Sh[i, j] for i in range(4)) for j in range(3)]
        Sn = np.array([[a[0, h] * Sh[i, j] + b[0, h] * k[0, 0, i] * (v[0, h, j] - u[j]) for j in range(3)]
                       for i in range(4)])
        on = [sum(q[0, 0, i] * Sn[i, j] for i in range(4)) for j in range(3)]
        assert np.allclose(s[0, h].numpy(), Sn, atol=1e-6)
        assert np.allclose(o[0, h].numpy(), on, atol=1e-6)


def test_baseline_gate_distribution():
    x = inputs.gdn_inputs(shapes.GDNShape("t", 4, 8, 16, 16, 4))
    assert torch.all((x["alpha"] > 0) & (x["alpha"] < 1))
    assert torch.all((x["beta"] > 0) & (x["beta"] < 1))
    assert torch.allclose(x["k"].float().norm(dim=-1), torch.ones(4, 4), atol=1e-2)
