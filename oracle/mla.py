"""MLA oracles, pre-projected prefill and absorbed decode (test infrastructure only).

The reference's MLA oracle (analysis/wave15-attention-architecture/reference/
pytorch_reference_mla.py:66-81, mla_naive) is softmax attention with an
explicit scale 1/sqrt(qk_head_dim).  In weight-absorbed decode
(analysis/wave15-attention-research/MECHANISMS.md:91-94, 115-120) every
head attends over the same latent cache: K := KV[b] (576 = 512 latent +
64 rope), V := KV[b][:, :512], one query token per sequence.  This is
mla_naive with n_kv = 1, computed in fp32 per sequence.
"""
from __future__ import annotations

import torch


def mla_prefill_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    heads: list[int] | None = None) -> torch.Tensor:
    """Pre-projected MLA prefill: mla_naive of pytorch_reference_mla.py:66-81
    (softmax(q k^T / sqrt(qk_head_dim)) v per head, fp32), plus this path's
    causal mask.  q, k [B,H,S,d_qk], v [B,H,S,d_v] -> fp32 [B,H,S,d_v]."""
    q = q.detach().cpu().float()
    k = k.detach().cpu().float()
    v = v.detach().cpu().float()
    B, H, S, Dqk = q.shape
    scale = 1.0 / (Dqk ** 0.5)
    out = torch.zeros((B, H, S, v.shape[-1]), dtype=torch.float32)
    mask = torch.ones((S, S), dtype=torch.bool).triu(1) if causal else None
    for b in range(B):
        for h in (heads if heads is not None else range(H)):
            scores = (q[b, h] @ k[b, h].transpose(0, 1)) * scale
            if mask is not None:
                scores = scores.masked_fill(mask, float("-inf"))
            out[b, h] = torch.softmax(scores, dim=-1) @ v[b, h]
    return out


def mla_decode_ref(q: torch.Tensor, kv: torch.Tensor, scale: float, d_latent: int = 512,
                   batches: list[int] | None = None) -> torch.Tensor:
    """q [B,H,Dqk], kv [B,T,Dqk] -> fp32 [B,H,d_latent]."""
    q = q.detach().cpu().float()
    kv = kv.detach().cpu().float()
    B, H, _ = q.shape
    out = torch.zeros((B, H, d_latent), dtype=torch.float32)
    for b in (batches if batches is not None else range(B)):
        scores = (q[b] @ kv[b].transpose(0, 1)) * scale     # [H, T]
        probs = torch.softmax(scores, dim=-1)
        out[b] = probs @ kv[b][:, :d_latent]                 # [H, 512]
    return out


def mla_partial(q: torch.Tensor, kv: torch.Tensor, scale: float, d_latent: int = 512):
    """Unnormalised partial softmax state over a token slice:
    (m [B,H], l [B,H], o [B,H,d_latent]) with o = sum_t exp(s_t - m) v_t."""
    q = q.detach().cpu().float()
    kv = kv.detach().cpu().float()
    s = torch.einsum("bhd,btd->bht", q, kv) * scale
    m = s.amax(dim=-1)
    p = torch.exp(s - m[..., None])
    return m, p.sum(-1), torch.einsum("bht,btd->bhd", p, kv[..., :d_latent])


def mla_merge(parts) -> torch.Tensor:
    """Log-sum-exp merge of partial states (the split-KV combine rule)."""
    ms = torch.stack([p[0] for p in parts])
    M = ms.amax(0)
    ws = torch.exp(ms - M)
    l = sum(w * p[1] for w, p in zip(ws, parts))
    o = sum(w[..., None] * p[2] for w, p in zip(ws, parts))
    return o / l[..., None]


def mla_absorbed_ref(q_nope, q_rope, kv, w_uk, w_uv, scale: float) -> torch.Tensor:
    """The absorbed decode step with the device path's roundings
    (MECHANISMS.md:91-94, 115-120): q_lat = bf16(q_nope @ W_UK[h]) (fp32
    accumulate), Q = [q_lat, q_rope], o_lat = bf16(mla_decode_ref(Q, kv)),
    o = o_lat @ W_UV[h] in fp32.  Shapes: q_nope [B,H,dn], q_rope
    [B,H,dr], kv [B,T,dc+dr], w_uk [H,dn,dc], w_uv [H,dc,dv]."""
    qn, qr = q_nope.detach().cpu().float(), q_rope.detach().cpu().float()
    wk, wv = w_uk.detach().cpu().float(), w_uv.detach().cpu().float()
    q_lat = torch.einsum("bhn,hnc->bhc", qn, wk).to(torch.bfloat16).float()
    Q = torch.cat([q_lat, qr], dim=-1)
    o_lat = mla_decode_ref(Q, kv, scale, d_latent=wk.shape[2]).to(torch.bfloat16).float()
    return torch.einsum("bhc,hcv->bhv", o_lat, wv)


def mla_unabsorbed_ref(q_nope, q_rope, kv, w_uk, w_uv, scale: float, d_latent: int = 512) -> torch.Tensor:
    """The same step without absorption, float64: per-head keys
    k = [W_UK[h]^T c_t, k_rope_t] and values v = W_UV[h]^T c_t are
    materialised from the latent rows c_t = kv[b,t,:d_latent] and
    o = softmax(scale q.k) v with q = [q_nope, q_rope] (MECHANISMS.md:77-88).
    Equal to mla_absorbed_ref up to the bf16 roundings that one applies."""
    qn, qr = q_nope.detach().cpu().double(), q_rope.detach().cpu().double()
    wk, wv = w_uk.detach().cpu().double(), w_uv.detach().cpu().double()
    kvd = kv.detach().cpu().double()
    c, kr = kvd[..., :d_latent], kvd[..., d_latent:]
    k_nope = torch.einsum("btc,hnc->bhtn", c, wk)              # [B,H,T,dn]
    v = torch.einsum("btc,hcv->bhtv", c, wv)                   # [B,H,T,dv]
    s = (torch.einsum("bhn,bhtn->bht", qn, k_nope) + torch.einsum("bhr,btr->bht", qr, kr)) * scale
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bht,bhtv->bhv", p, v)
