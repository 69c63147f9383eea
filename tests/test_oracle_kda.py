"""Pin the KDA oracle (CPU): the fused form against the literal recurrence of
pytorch_reference_kda.py:5-9, against the GDN oracle when the gate is
constant across channels (KDA with g_i = log alpha is GDN,
docs/adrs/0006-kda-as-gdn-extension.md:5-16), closed-form special cases
and fp64 loops."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import import_submodule
from oracle import gdn as ogdn
from oracle import kda as okda

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_fused_vs_canonical():
    for s in (shapes.KDA_CORRECTNESS, shapes.KDAShape("t", 2, 3, 128, 64)):
        x = inputs.kda_inputs(s)
        o1, s1 = okda.kda_decode_ref(**x)
        o2, s2 = okda.kda_decode_canonical(**x)
        assert np.abs(o1 - o2).max() < 1e-12 and np.abs(s1 - s2).max() < 1e-12


def test_constant_gate_is_gdn():
    """g_i = log(alpha) for every channel reduces KDA to GDN with that alpha."""
    s = shapes.KDAShape("t", 2, 4, 64, 32)
    x = inputs.kda_inputs(s, dtype=torch.float32)
    alpha = torch.tensor([[0.9, 0.7, 0.95, 0.5], [0.8, 0.99, 0.6, 0.75]])
    x["g"] = torch.log(alpha)[..., None].expand(2, 4, 64).contiguous()
    o, so = okda.kda_decode_ref(**x)
    og, sg = ogdn.gdn_decode_ref(x["q"], x["k"], x["v"], alpha, x["beta"].float(), x["S_in"])
    assert np.abs(o - og.numpy()).max() < 1e-5 and np.abs(so - sg.numpy()).max() < 1e-6


def test_beta_zero_is_pure_per_channel_decay():
    x = inputs.kda_inputs(shapes.KDAShape("t", 1, 2, 32, 48))
    x["beta"] = torch.zeros_like(x["beta"])
    o, so = okda.kda_decode_ref(**x)
    e = np.exp(x["g"].double().numpy())[..., None]
    assert np.array_equal(so, e * x["S_in"].double().numpy())
    assert np.allclose(o, np.einsum("bhk,bhkv->bhv", x["q"].double().numpy(), so), rtol=0, atol=1e-12)


def test_delta_rule_write():
    """beta |k|^2 = 1 makes the update write v exactly: k^T S' = v."""
    x = inputs.kda_inputs(shapes.KDAShape("t", 2, 3, 64, 32), dtype=torch.float32)
    kk = x["k"].double().numpy()
    x["beta"] = torch.from_numpy(1.0 / (kk * kk).sum(-1))
    _, so = okda.kda_decode_ref(**x)
    ks = np.einsum("bhk,bhkv->bhv", kk, so)
    assert np.allclose(ks, x["v"].double().numpy(), atol=1e-10)


def test_fp64_loops():
    s = shapes.KDAShape("t", 1, 2, 6, 5)
    x = inputs.kda_inputs(s, dtype=torch.float32)
    o, so = okda.kda_decode_ref(**x)
    q, k, v, g = (x[n].double().numpy() for n in ("q", "k", "v", "g"))
    beta, S = x["beta"].double().numpy(), x["S_in"].double().numpy()
    for h in range(2):
        D = [[math.exp(g[0, h, i]) * S[0, h, i, j] for j in range(5)] for i in range(6)]
        u = [sum(k[0, h, i] * D[i][j] for i in range(6)) for j in range(5)]
        Sn = [[D[i][j] + beta[0, h] * k[0, h, i] * (v[0, h, j] - u[j]) for j in range(5)] for i in range(6)]
        on = [sum(q[0, h, i] * Sn[i][j] for i in range(6)) for j in range(5)]
        assert np.allclose(so[0, h], np.array(Sn), rtol=0, atol=1e-14)
        assert np.allclose(o[0, h], np.array(on), rtol=0, atol=1e-14)


def test_reference_recipe():
    """The restated generator follows cutile-attn-kda/main.py:282-305: seed 17,
    decay exp(g) in (0, 1], beta in [0.1, 0.9], deterministic."""
    s = shapes.KDA_KIMI_LINEAR
    x = inputs.kda_inputs(s)
    y = inputs.kda_inputs(s)
    assert all(torch.equal(x[n], y[n]) for n in x)
    assert x["q"].dtype == torch.float16 and x["S_in"].dtype == torch.float32
    assert float(x["g"].max()) <= 0.0 and 0.1 <= float(x["beta"].min()) and float(x["beta"].max()) <= 0.9
    assert abs(float(x["q"].float().std()) * math.sqrt(s.d_k) - 1.0) < 0.05
    assert abs(float(x["S_in"].std()) - 0.1) < 0.005


@pytest.mark.parametrize("name", ["correctness", "kimi_linear_decode", "qwen3_next_gdn_parity", "large"])
def test_reference_recipe_bit_identical(name):
    """The f16 inputs are the reference's own values bit for bit: numpy draws
    in float64 cast once to float16 (cutile-attn-kda/main.py:287-292).  The
    same draws rounded through float32 first differ in a few values at the
    larger shapes, so this comparison would see a double rounding."""
    s = shapes.KDA_REGISTRY[name]
    x = inputs.kda_inputs(s)
    rng = np.random.default_rng(17)
    B, H, dk, dv = s.batch, s.n_heads, s.d_k, s.d_v
    sc = 1.0 / np.sqrt(dk)
    draws = {
        "q": rng.standard_normal((B, H, dk)) * sc,
        "k": rng.standard_normal((B, H, dk)) * sc,
        "v": rng.standard_normal((B, H, dv)),
        "g": -np.abs(rng.standard_normal((B, H, dk))) * 0.5,
        "beta": rng.uniform(0.1, 0.9, size=(B, H)),
    }
    S = (rng.standard_normal((B, H, dk, dv)) * 0.1).astype(np.float32)
    via32 = 0
    for n, d in draws.items():
        ref = d.astype(np.float16).view(np.uint16)
        got = x[n].numpy().view(np.uint16)
        assert np.array_equal(got, ref), n
        via32 += int((d.astype(np.float32).astype(np.float16).view(np.uint16) != ref).sum())
    assert np.array_equal(x["S_in"].numpy(), S)
    if name == "large":
        assert via32 > 0  # the float32 route is distinguishable at this shape
