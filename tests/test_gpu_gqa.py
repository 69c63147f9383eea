"""Fused GQA forward parity on the GPU vs the CPU oracle (gqa_naive of
pytorch_reference.py:51-74, plus the causal mask).  Bound: normwise
<= 2e-2 for bf16/f16 outputs; the reference's own f16 allclose gate
(atol = rtol = 5e-3, cutile-attn-gqa/main.py:258-265) on its correctness shape."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import gqa as ogqa
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def run(ops, q, k, v, causal):
    o = ops.gqa_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    return o.cpu()


def test_golden_reference_correctness_shape(ops):
    """Reference SHAPE_CORRECTNESS (1,128,4,2,64), f16, non-causal, reference inputs."""
    announce("gqa golden correctness f16")
    g = load_golden("gqa_correctness_f16")
    q, k, v = (from_bits(g[x], torch.float16) for x in "qkv")
    o = run(ops, q, k, v, causal=False).float().numpy()
    assert np.allclose(o, g["o"], atol=5e-3, rtol=5e-3)
    assert normwise_rel_err(o, g["o"]) <= 5e-3


def test_golden_causal_bf16(ops):
    announce("gqa golden causal bf16 S=80 D=128")
    g = load_golden("gqa_causal_bf16_s80")
    q, k, v = (from_bits(g[x], torch.bfloat16) for x in "qkv")
    o = run(ops, q, k, v, causal=True)
    assert normwise_rel_err(o, g["o"]) <= TOL


CASES = [
    # (B, S, Hq, Hkv, D, causal, dtype)
    (1, 128, 4, 2, 64, False, torch.bfloat16),
    (1, 128, 4, 2, 64, True, torch.float16),
    (2, 200, 8, 2, 128, True, torch.bfloat16),   # ragged S, G = 4
    (1, 257, 8, 8, 128, True, torch.bfloat16),   # MHA (G = 1), ragged
    (1, 190, 8, 1, 64, False, torch.bfloat16),   # MQA (G = 8)
    (1, 64, 6, 3, 128, True, torch.float16),     # G = 2
    (1, 1, 4, 1, 128, True, torch.bfloat16),     # single token
    (1, 1024, 32, 8, 128, True, torch.bfloat16),
    (1, 2048, 32, 8, 128, False, torch.float16),  # reference bench shape (llama3_8b)
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}S{c[1]}H{c[2]}/{c[3]}D{c[4]}{'c' if c[5] else 'n'}")
def test_parity_vs_oracle(ops, case):
    B, S, Hq, Hkv, D, causal, dt = case
    announce(f"gqa B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} causal={causal} {dt}")
    s = shapes.GQAShape("t", B, S, Hq, Hkv, D, causal)
    q, k, v = inputs.gqa_inputs(s, dtype=dt)
    o = run(ops, q, k, v, causal)
    heads = list(range(Hq)) if Hq * S <= 8192 else [0, Hq // 2 + 1, Hq - 1]
    ref = ogqa.gqa_naive(q, k, v, causal=causal, heads=heads)
    err = normwise_rel_err(o[:, heads], ref[:, heads])
    assert err <= TOL, f"normwise rel err {err:.3e}"


def test_baseline_config(ops):
    """BASELINE config: B1 Hq32 Hkv8 S4096 D128 bf16 causal, N(0,1) inputs;
    three heads (one per distinct position in its KV group) against the oracle."""
    announce("gqa BASELINE causal S4096")
    s = shapes.GQA_BASELINE
    q, k, v = inputs.gqa_inputs(s)
    o = run(ops, q, k, v, True)
    heads = [0, 13, 31]
    ref = ogqa.gqa_naive(q, k, v, causal=True, heads=heads)
    err = normwise_rel_err(o[:, heads], ref[:, heads])
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.isfinite(o.float()).all()


def test_constant_value_gives_constant_output(ops):
    announce("gqa V=1 -> O=1")
    s = shapes.GQAShape("t", 1, 300, 8, 2, 128, True)
    q, k, _ = inputs.gqa_inputs(s)
    v = torch.ones_like(k)
    o = run(ops, q, k, v, True).float()
    assert torch.all((o - 1.0).abs() <= 1e-2)


def test_causal_first_row_is_first_value(ops):
    """Causal query 0 sees only key 0: O[:, h, 0] = V[:, h // G, 0]."""
    announce("gqa causal row 0")
    s = shapes.GQAShape("t", 1, 128, 4, 2, 128, True)
    q, k, v = inputs.gqa_inputs(s)
    o = run(ops, q, k, v, True).float()
    for h in range(4):
        assert torch.allclose(o[0, h, 0], v[0, h // 2, 0].float(), atol=1e-2, rtol=1e-2)


# Every tile mx_gqa_fwd_tile accepts at these head groupings: (B, S, Hq, Hkv, D, BLOCK_M, wave_m).
# G = 4 covers the 8-wave kernel at 1, 2, 4 heads per workgroup, the 4-wave kernel at 32-row blocks and
# the one-wave-per-SIMD kernel (wave_m 64); G = 2 the 4-wave kernel at 64-row blocks; G = 1 whole-workgroup
# blocks; G = 8 eight heads per workgroup.  Ragged S everywhere.
TILES = [
    (1, 300, 8, 2, 128, 32, 32), (1, 300, 8, 2, 128, 64, 32), (1, 300, 8, 2, 128, 128, 32),
    (1, 300, 8, 2, 128, 256, 32), (1, 300, 8, 2, 128, 64, 64), (2, 300, 8, 2, 128, 128, 64),
    (1, 300, 8, 2, 128, 256, 64),
    (1, 200, 4, 2, 64, 64, 32), (1, 200, 4, 2, 64, 128, 32), (1, 200, 4, 2, 64, 256, 32),
    (1, 200, 4, 2, 64, 128, 64), (1, 200, 4, 2, 64, 256, 64),
    (1, 170, 4, 4, 64, 128, 32), (1, 170, 4, 4, 64, 256, 32), (1, 170, 4, 4, 128, 256, 64),
    (1, 130, 8, 1, 64, 32, 32), (1, 130, 8, 1, 128, 64, 64),
]


@pytest.mark.parametrize("causal", [True, False], ids=["c", "n"])
@pytest.mark.parametrize("case", TILES, ids=lambda c: f"B{c[0]}S{c[1]}H{c[2]}/{c[3]}D{c[4]}bm{c[5]}wm{c[6]}")
def test_tile_parity_vs_oracle(ops, case, causal):
    """Each explicit tile (the reference's --block-m override,
    cutile-attn-gqa/main.py:202-230) against gqa_naive, both dtypes."""
    B, S, Hq, Hkv, D, bm, wm = case
    for dt in (torch.bfloat16, torch.float16):
        announce(f"gqa tile BLOCK_M={bm} wave_m={wm} B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} causal={causal} {dt}")
        assert ops.gqa_tile_supported(Hq, Hkv, D, bm, 64, wm)
        s = shapes.GQAShape("t", B, S, Hq, Hkv, D, causal)
        q, k, v = inputs.gqa_inputs(s, dtype=dt, seed=inputs.SEED + bm + wm)
        o = ops.gqa_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal, block_m=bm, block_n=64, wave_m=wm)
        torch.cuda.synchronize()
        ref = ogqa.gqa_naive(q, k, v, causal=causal)
        err = normwise_rel_err(o.cpu(), ref)
        assert err <= TOL, f"normwise rel err {err:.3e}"


@pytest.mark.parametrize("bm,wm", [(64, 32), (128, 32), (256, 32), (64, 64), (128, 64), (256, 64)])
def test_tile_baseline_config(ops, bm, wm):
    """The BASELINE shape (B1 Hq32 Hkv8 S4096 D128 bf16 causal) on every
    tile of the reference's BLOCK_M sweep: three heads against the oracle,
    and the tile's output equal to the default tile's up to rounding."""
    announce(f"gqa BASELINE tile BLOCK_M={bm} wave_m={wm}")
    s = shapes.GQA_BASELINE
    q, k, v = (t.cuda() for t in inputs.gqa_inputs(s))
    o = ops.gqa_fwd(q, k, v, causal=True, block_m=bm, block_n=64, wave_m=wm)
    torch.cuda.synchronize()
    heads = [0, 13, 31]
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    ref = ogqa.gqa_naive(qc, kc, vc, causal=True, heads=heads)
    err = normwise_rel_err(o.cpu()[:, heads], ref[:, heads])
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.isfinite(o.float()).all()


def test_tile_rejections_enqueue_nothing(ops):
    """A tile no kernel has raises before any launch, and leaves out untouched."""
    import importlib

    _lib = importlib.import_module("cuda-oxide-bench_amd._lib")
    s = shapes.GQAShape("t", 1, 128, 8, 2, 128, True)
    q, k, v = (t.cuda() for t in inputs.gqa_inputs(s))
    out = torch.full_like(q, float("nan"))
    for bm, bn, wm in ((64, 32, 32), (16, 64, 32), (32, 64, 64)):
        with pytest.raises(_lib.MXError):
            ops.gqa_fwd(q, k, v, causal=True, out=out, block_m=bm, block_n=bn, wave_m=wm)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
