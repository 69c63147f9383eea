"""Long sequences and long contractions: index arithmetic, causal pairing
and split policies at sizes past the BASELINE configs, checked against the
CPU oracle on sampled query rows (attention) or in full (decode, GEMM).
Bounds as elsewhere: normwise <= 2e-2."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import announce, import_submodule
from oracle import gemm as ogemm
from oracle import gqa as ogqa
from oracle import mla as omla
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def _rows(S: int, n: int, seed: int) -> list[int]:
    """First and last rows, both sides of the 64-key tile and 128-query
    block edges, and random rows."""
    fixed = {0, 1, 63, 64, 127, 128, S // 2 - 1, S // 2, S - 65, S - 64, S - 2, S - 1}
    rng = np.random.default_rng(seed)
    extra = set(int(x) for x in rng.integers(0, S, n))
    return sorted(r for r in fixed | extra if 0 <= r < S)


@pytest.mark.parametrize("case", [
    # B, Hq, Hkv, S, D, causal, dtype
    (1, 8, 2, 16384, 128, True, torch.bfloat16),
    (1, 16, 2, 9000, 128, True, torch.float16),
    (2, 4, 4, 12345, 64, False, torch.bfloat16),
], ids=["S16384-G4-causal", "S9000-G8-causal-f16", "S12345-mha-d64"])
def test_gqa_long(ops, case):
    B, Hq, Hkv, S, D, causal, dt = case
    announce(f"long gqa B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} causal={causal} {dt}")
    g = torch.Generator().manual_seed(S + Hq)
    q = torch.randn((B, Hq, S, D), generator=g).to(dt)
    k = torch.randn((B, Hkv, S, D), generator=g).to(dt)
    v = torch.randn((B, Hkv, S, D), generator=g).to(dt)
    o = ops.gqa_fwd(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    heads = [0, Hq - 1]
    rows = _rows(S, 24, S)
    ref = ogqa.gqa_naive(q, k, v, causal=causal, scale=1.0 / math.sqrt(D), heads=heads, rows=rows)
    got = o.cpu()[:, heads][:, :, rows]
    assert normwise_rel_err(got, ref[:, heads]) <= TOL


def test_mla_prefill_long(ops):
    """Pre-projected MLA prefill (qk 192 / v 128), causal S = 8192."""
    H, S = 2, 8192
    announce(f"long mla_prefill H{H} S{S} qk192 v128 causal")
    s = shapes.MLAShape("t", 1, S, H, 128, 64, 128, 512, True)
    q, k, v = inputs.mla_prefill_inputs(s, dtype=torch.bfloat16)
    o = ops.mla_prefill_fwd(q.cuda(), k.cuda(), v.cuda(), causal=True)
    torch.cuda.synchronize()
    rows = _rows(S, 24, 7)
    ref = ogqa.gqa_naive(q, k, v, causal=True, scale=1.0 / math.sqrt(192), rows=rows)
    assert normwise_rel_err(o.cpu()[:, :, rows], ref) <= TOL


@pytest.mark.parametrize("bht", [(1, 128, 16384), (2, 16, 65536), (1, 128, 20000)])
def test_mla_decode_long(ops, bht):
    """More than 64 T splits (256, 128, 209): the merge gives each output
    element 4 or 8 threads, each summing one slice of the splits, whose sums
    meet in LDS; 209 splits make slices of unequal length."""
    B, H, T = bht
    announce(f"long mla_decode B{B} H{H} T{T}")
    nsplit = ops.mla_decode_splits(B, H, T)
    assert nsplit > 64, nsplit
    s = shapes.MLADecodeShape("t", B, H, T)
    q, kv = inputs.mla_inputs(s, seed=T + H)
    ws = torch.empty(ops.mla_decode_workspace_bytes(B, H, T), dtype=torch.uint8, device="cuda")
    o = ops.mla_decode(q.cuda(), kv.cuda(), s.scale, workspace=ws)
    torch.cuda.synchronize()
    assert normwise_rel_err(o.cpu(), omla.mla_decode_ref(q, kv, s.scale)) <= TOL


@pytest.mark.parametrize("mnk", [(256, 512, 65536), (64, 64, 131072), (300, 200, 40000)])
def test_gemm_bf16_long_k(ops, mnk):
    m, n, k = mnk
    announce(f"long gemm_bf16 {m}x{n}x{k}")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k), seed=k)
    c = ops.gemm_bf16(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    assert normwise_rel_err(c.cpu(), ogemm.gemm_ref(a, b)) <= TOL


def test_gemm_bf16_batched_many(ops):
    """A long batch: 1000 small-M items, each against its own weight."""
    nb, m, n, k = 1000, 16, 64, 128
    announce(f"long gemm_bf16_batched {nb}x{m}x{n}x{k}")
    g = torch.Generator().manual_seed(1000)
    a = (torch.rand((nb, m, k), generator=g) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand((nb, k, n), generator=g) * 2 - 1).to(torch.bfloat16)
    c = ops.gemm_bf16_batched(a.cuda(), b.cuda()).cpu()
    ref = torch.stack([torch.as_tensor(ogemm.gemm_ref(a[i], b[i])) for i in range(nb)])
    assert normwise_rel_err(c, ref) <= TOL
