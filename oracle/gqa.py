"""GQA attention oracle (test infrastructure only).

Restates gqa_naive of
analysis/wave15-attention-architecture/reference/pytorch_reference.py:51-74
— repeat_interleave the KV heads over their query group, softmax(QK^T * scale) V
in fp32 — and adds the causal mask (key t visible to query s iff t <= s).
Computed one (batch, query head) at a time to bound memory at S = 4096.
"""
from __future__ import annotations

import math

import torch


def gqa_naive(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
              scale: float | None = None, heads: list[int] | None = None,
              rows: list[int] | None = None) -> torch.Tensor:
    """q [B,Hq,S,D], k/v [B,Hkv,S,D] (any float dtype) -> fp32 [B,Hq,S,D].

    `heads` restricts the computation to those query heads (others stay 0),
    for bounded CPU timing samples.  `rows` restricts it to those query
    positions (each keeps its own causal row): the result is then
    [B,Hq,len(rows),Dv], row i holding query position rows[i].  Long
    sequences are checked on such samples.
    """
    q = q.detach().cpu().float()
    k = k.detach().cpu().float()
    v = v.detach().cpu().float()
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    pos = torch.arange(S) if rows is None else torch.tensor(rows, dtype=torch.long)
    out = torch.zeros((B, Hq, pos.numel(), v.shape[-1]), dtype=torch.float32)
    mask = None
    if causal:
        mask = torch.arange(k.shape[2])[None, :] > pos[:, None]  # key t hidden from query s iff t > s
    for b in range(B):
        for h in (heads if heads is not None else range(Hq)):
            kv = h // G  # repeat_interleave(groups, dim=1) maps query head h to kv head h // G
            scores = (q[b, h, pos] @ k[b, kv].transpose(0, 1)) * scale
            if mask is not None:
                scores = scores.masked_fill(mask, float("-inf"))
            probs = torch.softmax(scores, dim=-1)
            out[b, h] = probs @ v[b, kv]
    return out


def gqa_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """torch SDPA with enable_gqa (pytorch_reference.py:31-48), fp32 CPU — the
    independent witness the reference cross-checks its naive oracle against."""
    return torch.nn.functional.scaled_dot_product_attention(
        q.detach().cpu().float(), k.detach().cpu().float(), v.detach().cpu().float(),
        is_causal=causal, enable_gqa=True)
