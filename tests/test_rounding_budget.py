"""Error budget of the two roundings the device path adds to the reference's
semantics, measured on the CPU with the oracle (no GPU needed):

* GQA: the softmax scale times log2(e) is folded into Q, which is rounded to
  bf16 once (so the score MFMAs return log2-domain scores directly).  The
  reference scales the fp32 scores (cutile-attn-gqa/main.py:64-170).
* MLA decode: each T split stores its partial output normalised by its own
  row sum and rounded to bf16 before the log-sum-exp merge; the reference
  kernel does not split T (pytorch_reference_mla.py:66-81).

Each contribution is the normwise error of the oracle computed with only
that rounding added, against the oracle without it.  Both must stay far
inside the parity gate (2e-2) so that the device's other roundings (bf16 P,
bf16 output) keep their headroom.
"""
from __future__ import annotations

import math

import torch

from oracle.gqa import gqa_naive
from oracle.mla import mla_merge, mla_partial
from oracle.metrics import normwise_rel_err

BUDGET = 4e-3  # per added rounding, a fifth of the 2e-2 parity gate


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def test_gqa_folded_scale_rounding():
    g = torch.Generator().manual_seed(11)
    B, Hq, Hkv, S, D = 1, 4, 1, 1024, 128
    q = _bf16(torch.randn(B, Hq, S, D, generator=g))
    k = _bf16(torch.randn(B, Hkv, S, D, generator=g))
    v = _bf16(torch.randn(B, Hkv, S, D, generator=g))
    scale = 1.0 / math.sqrt(D)
    for causal in (False, True):
        ref = gqa_naive(q, k, v, causal=causal, scale=scale)
        # log2-domain scores from bf16(q * scale * log2 e); softmax base 2 ==
        # natural softmax of the scores times ln 2
        qf = _bf16(q * (scale * math.log2(math.e)))
        folded = gqa_naive(qf, k, v, causal=causal, scale=math.log(2.0))
        err = normwise_rel_err(folded, ref)
        print(f"GQA folded-scale bf16 Q, causal={causal}: normwise {err:.2e}")
        assert err <= BUDGET


def test_mla_bf16_split_partials_rounding():
    g = torch.Generator().manual_seed(12)
    B, H, T, nsplit = 2, 16, 2048, 8
    q = _bf16(torch.randn(B, H, 576, generator=g))
    kv = _bf16(torch.randn(B, T, 576, generator=g))
    scale = 1.0 / math.sqrt(192)
    parts = [mla_partial(q, kv[:, s * T // nsplit:(s + 1) * T // nsplit], scale) for s in range(nsplit)]
    exact = mla_merge(parts)
    # each split's output normalised by its own row sum and stored as bf16
    rounded = [(m, l, _bf16(o / l[..., None]) * l[..., None]) for m, l, o in parts]
    merged = mla_merge(rounded)
    err = normwise_rel_err(merged, exact)
    print(f"MLA bf16 normalised split partials ({nsplit} splits): normwise {err:.2e}")
    assert err <= BUDGET
    # the merge itself is exact in fp32 (split/merge = unsplit)
    from oracle.mla import mla_decode_ref
    assert normwise_rel_err(exact, mla_decode_ref(q, kv, scale)) <= 1e-5
