"""Seeded synthetic inputs for every kernel (CPU torch.Generator, seed 0xC0FFEE).

Two distributions per kernel:
  * "baseline": the distributions this path is measured on (uniform[-1,1]
    GEMM operands, N(0,1) attention inputs, L2-normalised GDN keys with
    exp(-softplus)/sigmoid gates);
  * "reference": the reference's own generators, restated —
    cutile-matmul-tc-bf16/main.py:89-95 (numpy PCG64 U[0,1)),
    pytorch_reference.py:77-97 (make_qkv), pytorch_reference_mla.py:84-108,
    pytorch_reference_gdn.py:126-165 (make_inputs).
The draw order inside each function is fixed; changing it changes every
fixture.  Tensors are returned on the CPU; callers move them to the GPU.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .quant import quantize_fp8_blockwise
from .shapes import FP8GemmShape, GDNShape, GemmShape, GQAShape, KDAShape, MLADecodeShape, MLAShape

SEED = 0xC0FFEE
SAMPLE_SEED = 0xBEEF


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def gemm_inputs(s: GemmShape, seed: int = SEED, dist: str = "baseline") -> tuple[torch.Tensor, torch.Tensor]:
    """A[M,K], B[K,N] bf16 (round-to-nearest-even from fp32)."""
    if dist == "reference":
        rng = np.random.default_rng(seed)
        a = torch.from_numpy(rng.random((s.m, s.k), dtype=np.float32))
        b = torch.from_numpy(rng.random((s.k, s.n), dtype=np.float32))
    else:
        g = _gen(seed)
        a = torch.rand((s.m, s.k), generator=g, dtype=torch.float32) * 2.0 - 1.0
        b = torch.rand((s.k, s.n), generator=g, dtype=torch.float32) * 2.0 - 1.0
    return a.to(torch.bfloat16), b.to(torch.bfloat16)


def fp8_gemm_inputs(s: FP8GemmShape, seed: int = SEED):
    """A, B ~ N(0,1) quantised to e4m3 with 1x128 (A) / 128x128 (B) fp32 scales.

    Returns (a_fp8, sa, b_fp8, sb).
    """
    g = _gen(seed)
    a = torch.randn((s.m, s.k), generator=g, dtype=torch.float32)
    b = torch.randn((s.k, s.n), generator=g, dtype=torch.float32)
    a8, sa = quantize_fp8_blockwise(a, (1, 128))
    b8, sb = quantize_fp8_blockwise(b, (128, 128))
    return a8, sa, b8, sb


def gqa_inputs(s: GQAShape, dtype: torch.dtype = torch.bfloat16, seed: int = SEED, dist: str = "baseline"):
    """q [B,Hq,S,D], k, v [B,Hkv,S,D]."""
    g = _gen(seed)
    qs = (s.batch, s.n_q, s.seq, s.d_head)
    ks = (s.batch, s.n_kv, s.seq, s.d_head)
    if dist == "reference":
        sc = 1.0 / math.sqrt(s.d_head)
        q = torch.randn(qs, generator=g, dtype=torch.float32) * sc
        k = torch.randn(ks, generator=g, dtype=torch.float32) * sc
        v = torch.randn(ks, generator=g, dtype=torch.float32)
    else:
        q = torch.randn(qs, generator=g, dtype=torch.float32)
        k = torch.randn(ks, generator=g, dtype=torch.float32)
        v = torch.randn(ks, generator=g, dtype=torch.float32)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def mla_prefill_inputs(s: MLAShape, dtype: torch.dtype = torch.float16, seed: int = SEED):
    """q, k [B,n_h,S,qk_head_dim], v [B,n_h,S,d_v]: the draws of
    make_qkv_mla (pytorch_reference_mla.py:84-108) -- one CPU generator,
    q then k then v, q and k scaled by 1/sqrt(qk_head_dim), in fp32 -- cast
    to `dtype`."""
    g = _gen(seed)
    qk = s.qk_head_dim
    sc = 1.0 / math.sqrt(qk)
    q = torch.randn((s.batch, s.n_h, s.seq, qk), generator=g, dtype=torch.float32) * sc
    k = torch.randn((s.batch, s.n_h, s.seq, qk), generator=g, dtype=torch.float32) * sc
    v = torch.randn((s.batch, s.n_h, s.seq, s.d_v), generator=g, dtype=torch.float32)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def mla_inputs(s: MLADecodeShape, seed: int = SEED):
    """q [B,H,d_latent+d_rope], kv [B,T,d_latent+d_rope], both ~N(0,1) bf16."""
    g = _gen(seed)
    q = torch.randn((s.batch, s.n_h, s.d_qk), generator=g, dtype=torch.float32)
    kv = torch.randn((s.batch, s.ctx, s.d_qk), generator=g, dtype=torch.float32)
    return q.to(torch.bfloat16), kv.to(torch.bfloat16)


def gdn_inputs(s: GDNShape, dtype: torch.dtype = torch.bfloat16, seed: int = SEED, dist: str = "baseline"):
    """Returns dict q, k [B,Hk,dk]; v [B,Hv,dv]; alpha, beta [B,Hv] fp32; S_in fp32."""
    g = _gen(seed)
    B, Hv, Hk, dk, dv = s.batch, s.n_heads, s.hk, s.d_k, s.d_v
    if dist == "reference":
        sc = 1.0 / math.sqrt(dk)
        q = torch.randn((B, Hk, dk), generator=g, dtype=torch.float32) * sc
        k = torch.randn((B, Hk, dk), generator=g, dtype=torch.float32) * sc
        v = torch.randn((B, Hv, dv), generator=g, dtype=torch.float32)
        alpha = 0.85 + 0.13 * torch.rand((B, Hv), generator=g, dtype=torch.float32)
        beta = -0.5 + torch.rand((B, Hv), generator=g, dtype=torch.float32)
        S = torch.randn((B, Hv, dk, dv), generator=g, dtype=torch.float32) * 0.1
        # The reference stores its gates as f16; keep the f16-rounded values.
        alpha = alpha.to(torch.float16).float()
        beta = beta.to(torch.float16).float()
    else:
        q = torch.randn((B, Hk, dk), generator=g, dtype=torch.float32)
        k = torch.randn((B, Hk, dk), generator=g, dtype=torch.float32)
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn((B, Hv, dv), generator=g, dtype=torch.float32)
        S = torch.randn((B, Hv, dk, dv), generator=g, dtype=torch.float32) * 0.02
        xa = torch.randn((B, Hv), generator=g, dtype=torch.float32)
        xb = torch.randn((B, Hv), generator=g, dtype=torch.float32)
        alpha = torch.exp(-torch.nn.functional.softplus(xa))
        beta = torch.sigmoid(xb)
    return {
        "q": q.to(dtype), "k": k.to(dtype), "v": v.to(dtype),
        "alpha": alpha.contiguous(), "beta": beta.contiguous(), "S_in": S.contiguous(),
    }


KDA_SEED = 17


def kda_inputs(s: KDAShape, dtype: torch.dtype = torch.float16, seed: int = KDA_SEED):
    """The reference's KDA recipe (cutile-attn-kda/main.py:282-305), restated
    draw for draw on numpy's default_rng: q, k ~ N(0,1)/sqrt(d_k), v ~ N(0,1),
    g = -|N(0,1)|/2 (decay exp(g) in (~0.6, 1]), beta ~ U(0.1, 0.9),
    S_in ~ 0.1 N(0,1) fp32.  The draws stay float64 until the one cast to the
    input type, as the reference's astype(np.float16) does (numpy rounds
    float64 straight to half, round to nearest even); rounding through
    float32 first would change a few values per shape.
    Returns dict q, k, g [B,H,dk]; v [B,H,dv]; beta [B,H] in `dtype`; S_in fp32."""
    rng = np.random.default_rng(seed)
    B, Hh, dk, dv = s.batch, s.n_heads, s.d_k, s.d_v
    scale_k = 1.0 / np.sqrt(dk)
    q = rng.standard_normal((B, Hh, dk)) * scale_k
    k = rng.standard_normal((B, Hh, dk)) * scale_k
    v = rng.standard_normal((B, Hh, dv))
    gg = -np.abs(rng.standard_normal((B, Hh, dk))) * 0.5
    beta = rng.uniform(0.1, 0.9, size=(B, Hh))
    S = (rng.standard_normal((B, Hh, dk, dv)) * 0.1).astype(np.float32)

    def t(x):
        if dtype == torch.float16:
            return torch.from_numpy(x.astype(np.float16))
        if dtype == torch.float64:
            return torch.from_numpy(x)
        return torch.from_numpy(x.astype(np.float32)).to(dtype)

    return {"q": t(q), "k": t(k), "v": t(v), "g": t(gg), "beta": t(beta), "S_in": torch.from_numpy(S).contiguous()}


def mla_projection_inputs(s: MLADecodeShape, d_nope: int = 128, d_v: int = 128, seed: int = SEED + 1):
    """The tensors around the absorbed decode (DeepSeek-V3: d_nope = d_v = 128):
    q_nope [B,H,d_nope], q_rope [B,H,d_rope] ~ N(0,1); W_UK [H,d_nope,d_c],
    W_UV [H,d_c,d_v] ~ N(0,1)/sqrt(fan-in); all bf16."""
    g = _gen(seed)
    B, Hh, dc, dr = s.batch, s.n_h, s.d_latent, s.d_qk - s.d_latent
    q_nope = torch.randn((B, Hh, d_nope), generator=g, dtype=torch.float32)
    q_rope = torch.randn((B, Hh, dr), generator=g, dtype=torch.float32)
    w_uk = torch.randn((Hh, d_nope, dc), generator=g, dtype=torch.float32) / math.sqrt(d_nope)
    w_uv = torch.randn((Hh, dc, d_v), generator=g, dtype=torch.float32) / math.sqrt(dc)
    return {n: t.to(torch.bfloat16) for n, t in
            (("q_nope", q_nope), ("q_rope", q_rope), ("w_uk", w_uk), ("w_uv", w_uv))}
