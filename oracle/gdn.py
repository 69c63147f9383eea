"""Gated-DeltaNet decode oracle (test infrastructure only).

Restates gdn_decode_reference and gdn_decode_reference_canonical of
analysis/wave15-attention-architecture/reference/pytorch_reference_gdn.py:38-123
(fp32 einsums on upcast inputs), generalised to n_k_heads <= n_v_heads:
value head h reads key head h // (Hv / Hk) (q and k repeat-interleaved
over the value heads).
"""
from __future__ import annotations

import torch


def _expand(x: torch.Tensor, hv: int) -> torch.Tensor:
    hk = x.shape[1]
    assert hv % hk == 0
    return x.repeat_interleave(hv // hk, dim=1)


def gdn_decode_ref(q, k, v, alpha, beta, S_in):
    """Fused form (pytorch_reference_gdn.py:66-91).  Returns (o fp32 [B,Hv,dv], S_out fp32)."""
    vf = v.detach().cpu().float()
    Hv = vf.shape[1]
    qf = _expand(q.detach().cpu().float(), Hv)
    kf = _expand(k.detach().cpu().float(), Hv)
    af = alpha.detach().cpu().float()
    bf = beta.detach().cpu().float()
    S = S_in.detach().cpu().float()
    B = qf.shape[0]
    S_scaled = af.view(B, Hv, 1, 1) * S
    u = torch.einsum("bhk,bhkv->bhv", kf, S_scaled)
    residual = vf - u
    outer = torch.einsum("bhk,bhv->bhkv", kf, residual)
    S_out = S_scaled + bf.view(B, Hv, 1, 1) * outer
    o = torch.einsum("bhk,bhkv->bhv", qf, S_out)
    return o, S_out


def gdn_decode_canonical(q, k, v, alpha, beta, S_in):
    """Literal alpha (I - beta k k^T) S + beta k v^T (pytorch_reference_gdn.py:94-123)."""
    vf = v.detach().cpu().float()
    Hv = vf.shape[1]
    qf = _expand(q.detach().cpu().float(), Hv)
    kf = _expand(k.detach().cpu().float(), Hv)
    af = alpha.detach().cpu().float()
    bf = beta.detach().cpu().float()
    S = S_in.detach().cpu().float()
    B, _, dk = qf.shape
    kkT = torch.einsum("bhi,bhj->bhij", kf, kf)
    eye = torch.eye(dk, dtype=torch.float32).view(1, 1, dk, dk)
    M = eye - bf.view(B, Hv, 1, 1) * kkT
    aMS = af.view(B, Hv, 1, 1) * torch.einsum("bhij,bhjv->bhiv", M, S)
    S_out = aMS + bf.view(B, Hv, 1, 1) * torch.einsum("bhk,bhv->bhkv", kf, vf)
    o = torch.einsum("bhk,bhkv->bhv", qf, S_out)
    return o, S_out
