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


# ---- pre-projected prefill (mla_naive of pytorch_reference_mla.py:66-81) ----

def test_prefill_matches_sdpa_with_explicit_scale():
    """The reference cross-checks mla_naive against SDPA with scale
    1/sqrt(qk_head_dim) to < 1e-4 (pytorch_reference_mla.py:150-157)."""
    s = shapes.MLA_PREFILL_CORRECTNESS
    q, k, v = inputs.mla_prefill_inputs(s, dtype=torch.float32)
    o = omla.mla_prefill_ref(q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=s.scale)
    assert (o - ref).abs().max() < 1e-5
    oc = omla.mla_prefill_ref(q, k, v, causal=True)
    refc = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=s.scale)
    assert (oc - refc).abs().max() < 1e-5


def test_prefill_equals_the_references_zero_padded_form():
    """The reference's kernel pads qk_head_dim 192 to 256 with zero columns
    and keeps the scale at 1/sqrt(192) (cutile-attn-mla/main.py:89-106,
    179-206): the unpadded result must be the same attention."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn((1, 2, 33, 192), generator=g) / 192 ** 0.5
    k = torch.randn((1, 2, 33, 192), generator=g) / 192 ** 0.5
    v = torch.randn((1, 2, 33, 128), generator=g)
    pad = lambda t: torch.nn.functional.pad(t, (0, 64))  # noqa: E731
    padded = ogqa.gqa_naive(pad(q), pad(k), v, causal=False, scale=192 ** -0.5)
    assert torch.allclose(omla.mla_prefill_ref(q, k, v), padded, atol=1e-6)


def test_prefill_special_cases():
    g = torch.Generator().manual_seed(9)
    q = torch.randn((2, 3, 20, 96), generator=g)
    k = torch.randn((2, 3, 20, 96), generator=g)
    v = torch.randn((2, 3, 20, 64), generator=g)
    oc = omla.mla_prefill_ref(q, k, v, causal=True)
    assert torch.allclose(oc[:, :, 0], v[:, :, 0])                     # causal row 0 sees only key 0
    assert torch.allclose(omla.mla_prefill_ref(q, k, torch.ones_like(v)), torch.ones_like(v))
    # fp64 brute force, one (b, h, s) at a time
    b, h, i = 1, 2, 7
    sc = [sum(float(q[b, h, i, d]) * float(k[b, h, t, d]) for d in range(96)) / 96 ** 0.5 for t in range(20)]
    mx = max(sc)
    w = [pow(2.718281828459045, x - mx) for x in sc]
    ref = [sum(w[t] * float(v[b, h, t, c]) for t in range(20)) / sum(w) for c in range(64)]
    assert torch.allclose(omla.mla_prefill_ref(q, k, v)[b, h, i], torch.tensor(ref, dtype=torch.float32), atol=1e-5)
