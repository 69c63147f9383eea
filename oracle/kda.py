"""Kimi-Delta-Attention (KDA) decode oracle (test infrastructure only).

KDA is GDN with a per-channel gate: the state row i decays by exp(g_i)
instead of a scalar alpha (docs/adrs/0006-kda-as-gdn-extension.md:5-16).

kda_decode_ref restates naive_recurrent_kda_step of
analysis/wave15-attention-architecture/reference/pytorch_reference_kda.py:42-73
(also cutile-attn-kda/main.py:147-179): float64 numpy, q used as given
(scale 1.0, the harness convention), order decay -> residual -> rank-1
update -> read-out.

kda_decode_canonical writes the recurrence literally as in the reference's
docstring (pytorch_reference_kda.py:5-9):
    S' = (I - beta k k^T) Diag(exp g) S + beta k v^T,   o = S'^T q
and is an independent check of the fused form.
"""
from __future__ import annotations

import numpy as np


def _np64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float64)


def kda_decode_ref(q, k, v, g, beta, S_in):
    """Fused form (pytorch_reference_kda.py:42-73).  Shapes q,k,g [B,H,dk];
    v [B,H,dv]; beta [B,H]; S_in [B,H,dk,dv].  Returns (o, S_out) float64."""
    q, k, v, g, beta, S = (_np64(x) for x in (q, k, v, g, beta, S_in))
    S = S * np.exp(g)[..., None]
    u = (k[..., None] * S).sum(axis=-2)
    residual = v - u
    S = S + (beta[..., None] * k)[..., None] * residual[..., None, :]
    o = np.einsum("bhk,bhkv->bhv", q, S)
    return o, S


def kda_decode_canonical(q, k, v, g, beta, S_in):
    """Literal (I - beta k k^T) Diag(exp g) S + beta k v^T (pytorch_reference_kda.py:5-9)."""
    q, k, v, g, beta, S = (_np64(x) for x in (q, k, v, g, beta, S_in))
    dk = q.shape[-1]
    kkT = np.einsum("bhi,bhj->bhij", k, k)
    M = np.eye(dk)[None, None] - beta[..., None, None] * kkT
    DS = np.exp(g)[..., None] * S
    S_out = np.einsum("bhij,bhjv->bhiv", M, DS) + beta[..., None, None] * np.einsum("bhk,bhv->bhkv", k, v)
    o = np.einsum("bhk,bhkv->bhv", q, S_out)
    return o, S_out
