"""The committed fixtures are reproducible: regenerating inputs with the
seeded generators and outputs with the oracle gives the stored arrays."""
from __future__ import annotations

import numpy as np
import torch

from conftest import from_bits, import_submodule, load_golden
from oracle import fp8 as ofp8
from oracle import gdn as ogdn
from oracle import gemm as ogemm
from oracle import gqa as ogqa
from oracle import kda as okda
from oracle import mla as omla

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_gemm_fixture():
    g = load_golden("gemm_bf16_72x136x96")
    a, b = inputs.gemm_inputs(shapes.GemmShape("golden", 72, 136, 96), seed=0x601D)
    assert torch.equal(from_bits(g["a"], torch.bfloat16), a)
    assert np.allclose(ogemm.gemm_ref(a, b).numpy(), g["c"], rtol=1e-6, atol=1e-6)


def test_fp8_fixture():
    g = load_golden("gemm_fp8_48x272x256")
    c = ofp8.gemm_fp8_bs_ref(g["a"], g["sa"], g["b"], g["sb"])
    assert np.allclose(c, g["c"], rtol=1e-6, atol=1e-5)


def test_gqa_fixtures():
    for name, dt, causal in (("gqa_correctness_f16", torch.float16, False), ("gqa_causal_bf16_s80", torch.bfloat16, True)):
        g = load_golden(name)
        q, k, v = (from_bits(g[x], dt) for x in "qkv")
        assert np.allclose(ogqa.gqa_naive(q, k, v, causal=causal).numpy(), g["o"], atol=1e-6)


def test_mla_prefill_fixture():
    g = load_golden("mla_prefill_correctness_f16")
    q, k, v = inputs.mla_prefill_inputs(shapes.MLA_PREFILL_CORRECTNESS, dtype=torch.float16)
    assert torch.equal(from_bits(g["q"], torch.float16), q) and torch.equal(from_bits(g["v"], torch.float16), v)
    assert np.allclose(omla.mla_prefill_ref(q, k, v).numpy(), g["o"], atol=1e-6)


def test_mla_fixture():
    g = load_golden("mla_decode_h16_t40")
    q, kv = from_bits(g["q"], torch.bfloat16), from_bits(g["kv"], torch.bfloat16)
    assert np.allclose(omla.mla_decode_ref(q, kv, float(g["scale"][0])).numpy(), g["o"], atol=1e-6)


def test_gdn_fixtures():
    for name, dt in (("gdn_correctness_f16", torch.float16), ("gdn_grouped_bf16", torch.bfloat16)):
        g = load_golden(name)
        x = {"q": from_bits(g["q"], dt), "k": from_bits(g["k"], dt), "v": from_bits(g["v"], dt),
             "alpha": torch.from_numpy(g["alpha"]), "beta": torch.from_numpy(g["beta"]),
             "S_in": torch.from_numpy(g["S_in"])}
        o, s = ogdn.gdn_decode_ref(**x)
        assert np.allclose(o.numpy(), g["o"], atol=1e-6) and np.allclose(s.numpy(), g["S_out"], atol=1e-7)


def test_kda_fixture():
    g = load_golden("kda_correctness_f16")
    x = inputs.kda_inputs(shapes.KDA_CORRECTNESS)
    for n in ("q", "k", "v", "g", "beta"):
        assert torch.equal(from_bits(g[n], torch.float16), x[n])
    assert np.array_equal(g["S_in"], x["S_in"].numpy())
    o, s = okda.kda_decode_ref(**x)
    assert np.array_equal(o, g["o"]) and np.array_equal(s, g["S_out"])
