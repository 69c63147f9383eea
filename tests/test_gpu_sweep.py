"""Seeded random-shape sweep: every kernel family against its CPU oracle on
shapes drawn at random (fixed seeds), so that ragged edges and dispatch
paths beyond the hand-picked cases of the per-kernel tests are exercised.
The bounds are those of the per-kernel tests: normwise <= 2e-2 for bf16/f16
outputs, <= 1e-3 for fp32 recurrent state, bit-exact for the quantiser."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import announce, import_submodule
from oracle import fp8 as ofp8
from oracle import gdn as ogdn
from oracle import gemm as ogemm
from oracle import gqa as ogqa
from oracle import kda as okda
from oracle import mla as omla
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2
TOL_S = 1e-3

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def _draws(seed: int, n: int, draw):
    rng = np.random.default_rng(seed)
    return [draw(rng) for _ in range(n)]


# ---- bf16 GEMM: half free shapes (M any, N and K multiples of 8), half whole
# 64x64 tiles with 128-deep K chunks (the direct-load small-grid path) ----
def _gemm_shape(rng):
    if rng.random() < 0.5:
        return int(rng.integers(1, 1100)), 8 * int(rng.integers(1, 140)), 8 * int(rng.integers(1, 150))
    return 64 * int(rng.integers(1, 17)), 64 * int(rng.integers(1, 17)), 128 * int(rng.integers(4, 11))


@pytest.mark.parametrize("mnk", _draws(101, 16, _gemm_shape), ids=lambda s: "x".join(map(str, s)))
def test_gemm_bf16_random(ops, mnk):
    m, n, k = mnk
    announce(f"sweep gemm_bf16 {m}x{n}x{k}")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k), seed=m * 7 + n * 13 + k)
    c = ops.gemm_bf16(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    ref = ogemm.gemm_ref(a, b)
    assert normwise_rel_err(c.cpu(), ref) <= TOL


# ---- batched bf16 GEMM: small-M items (M <= 32, K whole 64-deep chunks:
# weight-streaming kernel and its split-K variant) and larger items ----
def _batched_shape(rng):
    nb = int(rng.integers(1, 13))
    m = int(rng.integers(1, 33)) if rng.random() < 0.7 else int(rng.integers(33, 200))
    return nb, m, 8 * int(rng.integers(1, 41)), 64 * int(rng.integers(1, 13))


@pytest.mark.parametrize("bmnk", _draws(102, 8, _batched_shape), ids=lambda s: "x".join(map(str, s)))
def test_gemm_bf16_batched_random(ops, bmnk):
    nb, m, n, k = bmnk
    announce(f"sweep gemm_bf16_batched {nb}x{m}x{n}x{k}")
    g = torch.Generator().manual_seed(nb * 1009 + m * 31 + n + k)
    a = (torch.rand((nb, m, k), generator=g) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand((nb, k, n), generator=g) * 2 - 1).to(torch.bfloat16)
    c = ops.gemm_bf16_batched(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    c = c.cpu()
    for i in range(nb):
        assert normwise_rel_err(c[i], ogemm.gemm_ref(a[i], b[i])) <= TOL


# ---- GQA forward: batch, heads, grouping, ragged S, D, mask and dtype ----
def _gqa_case(rng):
    return (int(rng.integers(1, 3)), int(rng.choice([1, 2, 4])), int(rng.choice([1, 2, 4, 8])),
            int(rng.integers(1, 600)), int(rng.choice([64, 128])), bool(rng.integers(0, 2)),
            bool(rng.integers(0, 2)))


@pytest.mark.parametrize("case", _draws(103, 10, _gqa_case),
                         ids=lambda c: f"B{c[0]}kv{c[1]}G{c[2]}S{c[3]}D{c[4]}{'c' if c[5] else 'n'}{'h' if c[6] else 'b'}")
def test_gqa_random(ops, case):
    B, hkv, G, S, D, causal, half = case
    dt = torch.float16 if half else torch.bfloat16
    announce(f"sweep gqa B{B} Hkv{hkv} G{G} S{S} D{D} causal={causal} {dt}")
    g = torch.Generator().manual_seed(B * 7 + hkv * 11 + G * 13 + S + D)
    q = torch.randn((B, hkv * G, S, D), generator=g).to(dt)
    k = torch.randn((B, hkv, S, D), generator=g).to(dt)
    v = torch.randn((B, hkv, S, D), generator=g).to(dt)
    o = ops.gqa_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    ref = ogqa.gqa_naive(q, k, v, causal=causal, scale=1.0 / math.sqrt(D))
    assert normwise_rel_err(o.cpu(), ref) <= TOL


def _gqa_tile_case(rng):
    """A random shape and a random tile among those mx_gqa_fwd_tile has at its head grouping."""
    G = int(rng.choice([1, 2, 4, 8]))
    wm = int(rng.choice([32, 64]))
    waves = 8 if wm == 32 else 4
    bms = sorted({waves * wm // h for h in (1, 2, 4, 8) if h <= waves and waves % h == 0 and G % h == 0}
                 | ({128 // h for h in (1, 2, 4) if G % h == 0} if wm == 32 else set()))
    return (int(rng.integers(1, 3)), int(rng.choice([1, 2])), G, int(rng.integers(1, 500)),
            int(rng.choice([64, 128])), bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
            int(rng.choice(bms)), wm)


@pytest.mark.parametrize("case", _draws(211, 12, _gqa_tile_case),
                         ids=lambda c: f"B{c[0]}kv{c[1]}G{c[2]}S{c[3]}D{c[4]}{'c' if c[5] else 'n'}"
                                       f"{'h' if c[6] else 'b'}bm{c[7]}wm{c[8]}")
def test_gqa_tile_random(ops, case):
    """Seeded random shapes on random explicit tiles (mx_gqa_fwd_tile)."""
    B, hkv, G, S, D, causal, half, bm, wm = case
    dt = torch.float16 if half else torch.bfloat16
    announce(f"sweep gqa tile BLOCK_M={bm} wave_m={wm} B{B} Hkv{hkv} G{G} S{S} D{D} causal={causal} {dt}")
    assert ops.gqa_tile_supported(hkv * G, hkv, D, bm, 64, wm)
    g = torch.Generator().manual_seed(B * 5 + hkv * 3 + G * 17 + S + D + bm + wm)
    q = torch.randn((B, hkv * G, S, D), generator=g).to(dt)
    k = torch.randn((B, hkv, S, D), generator=g).to(dt)
    v = torch.randn((B, hkv, S, D), generator=g).to(dt)
    o = ops.gqa_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal, block_m=bm, block_n=64, wave_m=wm)
    torch.cuda.synchronize()
    ref = ogqa.gqa_naive(q, k, v, causal=causal, scale=1.0 / math.sqrt(D))
    assert normwise_rel_err(o.cpu(), ref) <= TOL


# ---- MLA prefill pairs (qk 192 / v 128 and qk 96 / v 64) ----
def _prefill_case(rng):
    dqk, dv = [(192, 128), (96, 64)][int(rng.integers(0, 2))]
    return int(rng.integers(1, 7)), int(rng.integers(1, 400)), dqk, dv, bool(rng.integers(0, 2))


@pytest.mark.parametrize("case", _draws(104, 4, _prefill_case),
                         ids=lambda c: f"H{c[0]}S{c[1]}qk{c[2]}v{c[3]}{'c' if c[4] else 'n'}")
def test_mla_prefill_random(ops, case):
    H, S, dqk, dv, causal = case
    announce(f"sweep mla_prefill H{H} S{S} qk{dqk} v{dv} causal={causal}")
    s = shapes.MLAShape("t", 1, S, H, dqk - 64 if dqk > 64 else dqk // 2, 64 if dqk > 64 else dqk // 2, dv, 512,
                        causal)
    q, k, v = inputs.mla_prefill_inputs(s, dtype=torch.bfloat16)
    o = ops.mla_prefill_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    ref = omla.mla_prefill_ref(q, k, v, causal=causal)
    assert normwise_rel_err(o.cpu(), ref) <= TOL


# ---- MLA absorbed decode: batch, heads and ragged T (split and unsplit) ----
def _mla_case(rng):
    return int(rng.integers(1, 6)), int(rng.integers(1, 141)), int(rng.integers(1, 1300))


@pytest.mark.parametrize("bht", _draws(105, 6, _mla_case), ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}")
def test_mla_decode_random(ops, bht):
    B, H, T = bht
    announce(f"sweep mla_decode B{B} H{H} T{T}")
    s = shapes.MLADecodeShape("t", B, H, T)
    q, kv = inputs.mla_inputs(s, seed=B * 101 + H * 7 + T)
    ws = torch.empty(max(1, ops.mla_decode_workspace_bytes(B, H, T)), dtype=torch.uint8, device="cuda")
    o = ops.mla_decode(q.cuda(), kv.cuda(), s.scale, workspace=ws)
    torch.cuda.synchronize()
    assert normwise_rel_err(o.cpu(), omla.mla_decode_ref(q, kv, s.scale)) <= TOL


# ---- fp8 block-scaled GEMM: M any, N multiples of 16, K of 128 ----
def _fp8_shape(rng):
    return int(rng.integers(1, 600)), 16 * int(rng.integers(1, 41)), 128 * int(rng.integers(1, 7))


@pytest.mark.parametrize("mnk", _draws(106, 6, _fp8_shape), ids=lambda s: "x".join(map(str, s)))
def test_gemm_fp8_random(ops, mnk):
    m, n, k = mnk
    announce(f"sweep gemm_fp8_bs {m}x{n}x{k}")
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k), seed=m + 3 * n + 5 * k)
    c = ops.gemm_fp8_bs(a8.cuda(), sa.cuda(), b8.cuda(), sb.cuda())
    torch.cuda.synchronize()
    ref = ofp8.gemm_fp8_bs_ref(ofp8.fp8_tensor_codes(a8), sa.numpy(), ofp8.fp8_tensor_codes(b8), sb.numpy())
    assert normwise_rel_err(c.cpu(), ref) <= TOL


# ---- GDN and KDA decode: batch, heads, grouping and head dims ----
_DIMS = [64, 128, 256, 512]


def _gdn_case(rng):
    return (int(rng.integers(1, 5)), int(rng.choice([1, 2, 4])), int(rng.choice([1, 2])),
            int(rng.choice(_DIMS)), int(rng.choice(_DIMS)))


@pytest.mark.parametrize("case", _draws(107, 4, _gdn_case), ids=lambda c: f"B{c[0]}Hk{c[1]}G{c[2]}k{c[3]}v{c[4]}")
def test_gdn_decode_random(ops, case):
    B, hk, G, dk, dv = case
    announce(f"sweep gdn_decode B{B} Hk{hk} G{G} dk{dk} dv{dv}")
    x = inputs.gdn_inputs(shapes.GDNShape("t", batch=B, n_heads=hk * G, d_k=dk, d_v=dv, n_k_heads=hk),
                          seed=B + hk * 3 + dk + dv)
    d = {key: val.cuda() for key, val in x.items()}
    o, so = ops.gdn_decode(d["q"], d["k"], d["v"], d["alpha"], d["beta"], d["S_in"])
    torch.cuda.synchronize()
    ro, rs = ogdn.gdn_decode_ref(**x)
    assert normwise_rel_err(o.cpu(), ro) <= TOL
    assert normwise_rel_err(so.cpu(), rs) <= TOL_S


def _kda_case(rng):
    return int(rng.integers(1, 5)), int(rng.integers(1, 9)), int(rng.choice(_DIMS[:3])), int(rng.choice(_DIMS[:3]))


@pytest.mark.parametrize("case", _draws(108, 3, _kda_case), ids=lambda c: f"B{c[0]}H{c[1]}k{c[2]}v{c[3]}")
def test_kda_decode_random(ops, case):
    B, H, dk, dv = case
    announce(f"sweep kda_decode B{B} H{H} dk{dk} dv{dv}")
    x = inputs.kda_inputs(shapes.KDAShape("t", batch=B, n_heads=H, d_k=dk, d_v=dv), dtype=torch.bfloat16)
    d = {key: val.cuda() for key, val in x.items()}
    o, so = ops.kda_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["S_in"])
    torch.cuda.synchronize()
    ro, rs = okda.kda_decode_ref(**x)
    assert normwise_rel_err(o.cpu(), ro) <= TOL
    assert normwise_rel_err(so.cpu(), rs) <= TOL_S


# ---- fp8 activation quantiser: bit-exact codes and scales ----
def _quant_shape(rng):
    return int(rng.integers(1, 700)), 128 * int(rng.integers(1, 17))


@pytest.mark.parametrize("mk", _draws(109, 4, _quant_shape), ids=lambda s: "x".join(map(str, s)))
def test_quant_fp8_random(ops, mk):
    m, k = mk
    announce(f"sweep quant_fp8 {m}x{k}")
    g = torch.Generator().manual_seed(m * 13 + k)
    x = (torch.randn((m, k), generator=g) * torch.exp(torch.randn((m, 1), generator=g) * 3)).to(torch.bfloat16)
    q, s = ops.quant_fp8_act(x.cuda())
    torch.cuda.synchronize()
    qe, se = ofp8.quantize_blockwise(x.float().numpy(), (1, 128))
    assert np.array_equal(s.cpu().numpy(), se)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qe)
