"""Pin the GQA oracle (CPU): torch SDPA witness (as pytorch_reference.py:127-136
does), MHA/MQA reductions, invariants, fp64 brute force."""
from __future__ import annotations

import math

import numpy as np
import torch

from conftest import import_submodule
from oracle import gqa as ogqa

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_naive_vs_sdpa_reference_shape():
    q, k, v = inputs.gqa_inputs(shapes.GQA_CORRECTNESS, dtype=torch.float32, dist="reference")
    for causal in (False, True):
        a = ogqa.gqa_naive(q, k, v, causal=causal)
        b = ogqa.gqa_sdpa(q, k, v, causal=causal)
        assert (a - b).abs().max().item() < 1e-4  # the reference's own threshold (:130)


def test_reductions_mha_mqa():
    """n_kv = n_q is plain MHA; n_kv = 1 is MQA: both equal per-head softmax attention."""
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 4, 33, 16, generator=g)
    k = torch.randn(1, 1, 33, 16, generator=g)
    v = torch.randn(1, 1, 33, 16, generator=g)
    mqa = ogqa.gqa_naive(q, k, v, causal=True)
    mha = ogqa.gqa_naive(q, k.expand(1, 4, 33, 16).contiguous(), v.expand(1, 4, 33, 16).contiguous(), causal=True)
    assert torch.allclose(mqa, mha, atol=0, rtol=0)


def test_shift_invariance():
    """Adding the same constant to every score of a query leaves O unchanged.
    An extra coordinate (3.0 on every query, 1.0 on every key) shifts all
    scores by 3 * scale."""
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 2, 20, 8, generator=g)
    k = torch.randn(1, 1, 20, 8, generator=g)
    v = torch.randn(1, 1, 20, 8, generator=g)
    # append a coordinate: q gets 3.0, every key gets 1.0 -> every score + 3*scale
    q2 = torch.cat([q, torch.full((1, 2, 20, 1), 3.0)], -1)
    k2 = torch.cat([k, torch.ones(1, 1, 20, 1)], -1)
    a = ogqa.gqa_naive(q, k, v, scale=0.5)
    b = ogqa.gqa_naive(q2, k2, v, scale=0.5)
    assert torch.allclose(a, b, atol=1e-6)


def test_causal_row0_and_constant_v():
    q, k, v = inputs.gqa_inputs(shapes.GQAShape("t", 1, 40, 4, 2, 16, True), dtype=torch.float32)
    o = ogqa.gqa_naive(q, k, v, causal=True)
    for h in range(4):
        assert torch.allclose(o[0, h, 0], v[0, h // 2, 0])
    o1 = ogqa.gqa_naive(q, k, torch.ones_like(v), causal=True)
    assert torch.allclose(o1, torch.ones_like(o1), atol=1e-6)


def test_fp64_bruteforce():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 2, 6, 4, generator=g)
    k = torch.randn(1, 1, 6, 4, generator=g)
    v = torch.randn(1, 1, 6, 4, generator=g)
    o = ogqa.gqa_naive(q, k, v, causal=True).double().numpy()
    qd, kd, vd = q.double().numpy(), k.double().numpy(), v.double().numpy()
    for h in range(2):
        for s in range(6):
            sc = [sum(qd[0, h, s, d] * kd[0, 0, t, d] for d in range(4)) / math.sqrt(4) for t in range(s + 1)]
            mx = max(sc)
            w = [math.exp(x - mx) for x in sc]
            z = sum(w)
            want = [sum(w[t] * vd[0, 0, t, d] for t in range(s + 1)) / z for d in range(4)]
            assert np.allclose(o[0, h, s], want, atol=1e-6)


def test_heads_subset_equals_full():
    q, k, v = inputs.gqa_inputs(shapes.GQAShape("t", 1, 24, 8, 2, 16, True), dtype=torch.float32)
    full = ogqa.gqa_naive(q, k, v, causal=True)
    part = ogqa.gqa_naive(q, k, v, causal=True, heads=[1, 6])
    assert torch.equal(full[:, [1, 6]], part[:, [1, 6]])


def test_rows_subset_equals_full_and_sdpa():
    """Sampled query positions keep their own causal rows: equal to the same
    rows of the full computation and of the SDPA witness, and blind to keys
    past each row."""
    q, k, v = inputs.gqa_inputs(shapes.GQAShape("t", 2, 200, 8, 2, 32, True), dtype=torch.float32)
    rows = [0, 1, 63, 64, 127, 150, 199]
    for causal in (False, True):
        full = ogqa.gqa_naive(q, k, v, causal=causal)
        part = ogqa.gqa_naive(q, k, v, causal=causal, rows=rows)
        assert torch.allclose(part, full[:, :, rows], atol=1e-6, rtol=1e-6)
        sd = ogqa.gqa_sdpa(q, k, v, causal=causal)
        assert torch.allclose(part, sd[:, :, rows], atol=1e-5, rtol=1e-5)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 151:] += 3.0
    v2[:, :, 151:] -= 5.0
    a = ogqa.gqa_naive(q, k, v, causal=True, rows=[0, 64, 150])
    b = ogqa.gqa_naive(q, k2, v2, causal=True, rows=[0, 64, 150])
    assert torch.equal(a, b)
