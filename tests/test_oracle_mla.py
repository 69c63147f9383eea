"""Pin the MLA decode oracle (CPU): reduction to the GQA oracle with one KV
head, special cases, and the split/merge rule the kernel's combine uses."""
from __future__ import annotations

import torch

from conftest import import_submodule
from oracle import gqa as ogqa
from oracle import mla as omla

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def test_reduces_to_gqa_with_one_kv_head():
    s = shapes.MLADecodeShape("t", 2, 8, 37)
    q, kv = inputs.mla_inputs(s)
    o = omla.mla_decode_ref(q, kv, s.scale)
    for b in range(2):
        # GQA oracle: 8 query heads over one KV head, one query position per head;
        # keys are the 576-wide latent rows, values their first 512 columns.
        # Pad V to 576 so K and V share a head dim, then crop the output.
        qq = q[b][None, :, None, :].float()
        kk = kv[b][None, None].float()
        vv = torch.nn.functional.pad(kv[b][:, :512].float(), (0, 64))[None, None]
        g = ogqa.gqa_naive(qq, kk, vv, causal=False, scale=s.scale)[0, :, 0, :512]
        assert torch.allclose(o[b], g, atol=1e-5, rtol=1e-5)


def test_single_token_and_identical_tokens():
    s = shapes.MLADecodeShape("t", 1, 4, 1)
    q, kv = inputs.mla_inputs(s)
    o = omla.mla_decode_ref(q, kv, s.scale)
    assert torch.allclose(o[0], kv[0, 0, :512].float().expand(4, 512))
    kv_same = kv[:, :1].expand(1, 9, 576).contiguous()
    o2 = omla.mla_decode_ref(q, kv_same, s.scale)
    assert torch.allclose(o2[0], kv[0, 0, :512].float().expand(4, 512), atol=1e-6)


def test_split_merge_equals_unsplit():
    s = shapes.MLADecodeShape("t", 2, 6, 100)
    q, kv = inputs.mla_inputs(s)
    full = omla.mla_decode_ref(q, kv, s.scale)
    parts = [omla.mla_partial(q, kv[:, a:b], s.scale) for a, b in ((0, 31), (31, 64), (64, 100))]
    assert torch.allclose(omla.mla_merge(parts), full, atol=1e-5, rtol=1e-5)


def test_absorption_identity():
    """Weight absorption changes nothing but roundings: the absorbed form
    (q_nope W_UK against the latent rows, then W_UV) equals attention over
    the materialised per-head keys and values (MECHANISMS.md:77-94)."""
    s = shapes.MLADecodeShape("t", 2, 4, 33)
    _, kv = inputs.mla_inputs(s)
    x = inputs.mla_projection_inputs(s)
    full = omla.mla_unabsorbed_ref(x["q_nope"], x["q_rope"], kv, x["w_uk"], x["w_uv"], s.scale)
    # absorbed, in float64 without the bf16 roundings
    qn, wk, wv = x["q_nope"].double(), x["w_uk"].double(), x["w_uv"].double()
    Q = torch.cat([torch.einsum("bhn,hnc->bhc", qn, wk), x["q_rope"].double()], dim=-1)
    sc = torch.einsum("bhd,btd->bht", Q, kv.double()) * s.scale
    o_lat = torch.einsum("bht,btc->bhc", torch.softmax(sc, -1), kv.double()[..., :512])
    absorbed = torch.einsum("bhc,hcv->bhv", o_lat, wv)
    assert torch.allclose(absorbed, full, rtol=1e-10, atol=1e-12)
    # and the rounded oracle stays within bf16 distance of it
    r = omla.mla_absorbed_ref(x["q_nope"], x["q_rope"], kv, x["w_uk"], x["w_uv"], s.scale).double()
    assert (r - full).abs().max() / full.abs().max() < 2e-2
