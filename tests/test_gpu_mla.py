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


# (1, 20, 8000): 63 splits, merged by 2 thread slices per element, 20 of a
# 32-head tile; (2, 36, 12000): 125 splits, 4 slices, a second head tile of 4.
@pytest.mark.parametrize("bht", [(2, 16, 200), (1, 128, 1), (1, 128, 33), (3, 20, 500), (4, 128, 1024),
                                 (1, 128, 4096), (2, 64, 4100), (1, 20, 8000), (2, 36, 12000)])
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


def test_running_max_jumps(ops):
    """Tokens whose scores jump far above everything before them in their
    split (median jumps of 26-33 in log2 units for most heads, beyond the
    kernel's 16-unit headroom) force the value accumulators to be rescaled
    mid-split; spikes sit inside splits, on a split boundary and on the last
    token."""
    announce("mla running-max jumps B32 H128 T4096")
    s = shapes.MLA_BASELINE
    q, kv = inputs.mla_inputs(s)
    qsum = q.float().sum(dim=1)  # [B, 576]: a key aligned with every head's query
    spikes = {0: [100, 700, 1500], 7: [512, 3000, 3001], 20: [4095]}
    for b, pos in spikes.items():
        for j, t in enumerate(pos):
            kv[b, t] = (qsum[b] * (0.6 * (j + 1))).to(torch.bfloat16)
    bs = sorted(spikes)
    # The construction really does jump: first spike vs the preceding max.
    sc = torch.einsum("hd,td->ht", q[0].float(), kv[0].float()) * s.scale
    assert (sc[:, 100] - sc[:, :100].max(dim=1).values).median() * 1.4427 > 16
    o = run(ops, q, kv, s.scale)
    ref = omla.mla_decode_ref(q, kv, s.scale, batches=bs)
    err = normwise_rel_err(o[bs], ref[bs])
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.isfinite(o.float()).all()


def test_absorb_and_up_project(ops):
    """The per-head weight products around the decode (head-strided batched
    GEMM) against fp32 per-head matmuls, at the DeepSeek-V3 head shapes."""
    announce("mla absorb q / up-project B32 H128")
    s = shapes.MLA_BASELINE
    x = inputs.mla_projection_inputs(s)
    d = {k: v.cuda() for k, v in x.items()}
    q_lat = ops.mla_absorb_q(d["q_nope"], d["w_uk"])
    o_lat = torch.randn((s.batch, s.n_h, 512), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    o = ops.mla_up_project(o_lat.cuda(), d["w_uv"])
    torch.cuda.synchronize()
    ref_q = torch.einsum("bhn,hnc->bhc", x["q_nope"].float(), x["w_uk"].float())
    ref_o = torch.einsum("bhc,hcv->bhv", o_lat.float(), x["w_uv"].float())
    assert normwise_rel_err(q_lat.cpu(), ref_q) <= 2e-2
    assert normwise_rel_err(o.cpu(), ref_o) <= 2e-2


def test_absorbed_pipeline(ops):
    """q_nope, q_rope, latent cache, W_UK, W_UV -> o: the whole absorbed
    decode step (absorb, latent attention, up-projection) against the oracle."""
    announce("mla absorbed pipeline B4 H128 T1024")
    s = shapes.MLADecodeShape("t", batch=4, n_h=128, ctx=1024)
    _, kv = inputs.mla_inputs(s)
    x = inputs.mla_projection_inputs(s)
    d = {k: v.cuda() for k, v in x.items()}
    o = ops.mla_decode_absorbed(d["q_nope"], d["q_rope"], kv.cuda(), d["w_uk"], d["w_uv"], s.scale)
    torch.cuda.synchronize()
    ref = omla.mla_absorbed_ref(x["q_nope"], x["q_rope"], kv, x["w_uk"], x["w_uv"], s.scale)
    assert normwise_rel_err(o.cpu(), ref) <= 2e-2


@pytest.mark.parametrize("b,h,t,dv", [(32, 128, 4096, 128), (40, 16, 300, 64), (1, 128, 64, 128)])
def test_absorbed_step_shapes(ops, b, h, t, dv):
    """The one-call absorbed step at the BASELINE shape (split decode,
    small-M projections), a batch above 32 (register-staged projections)
    and a single sequence (unsplit decode)."""
    announce(f"mla absorbed step B{b} H{h} T{t} dv{dv}")
    s = shapes.MLADecodeShape("t", batch=b, n_h=h, ctx=t)
    _, kv = inputs.mla_inputs(s)
    x = inputs.mla_projection_inputs(s, d_v=dv)
    d = {k: v.cuda() for k, v in x.items()}
    o = ops.mla_decode_absorbed(d["q_nope"], d["q_rope"], kv.cuda(), d["w_uk"], d["w_uv"], s.scale)
    torch.cuda.synchronize()
    bs = list(range(min(b, 4)))
    ref = omla.mla_absorbed_ref(x["q_nope"][bs], x["q_rope"][bs], kv[bs], x["w_uk"], x["w_uv"], s.scale)
    assert normwise_rel_err(o.cpu()[bs], ref) <= 2e-2
