"""Algorithmic work model: FLOPs and HBM bytes per call, and roofline peaks.

Follows the reference's single-source-of-truth FLOP modules
(analysis/wave15-attention-architecture/reference/flops.py:31-66,
flops_mla.py:32-64, flops_gdn.py:45-94) and adds the figures this path
reports: the causal algorithmic GQA count and the absorbed-decode MLA
traffic.  "Algorithmic" bytes count each tensor once (inputs read once,
outputs written once); "algorithmic" FLOPs count 2 per multiply-add of the
contractions only.
"""
from __future__ import annotations

from .shapes import FP8GemmShape, GDNShape, GemmShape, GQAShape, MLADecodeShape, MLAShape

# MI355X published peaks (dense).
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBPS = 8000.0


def gemm_flops(s: GemmShape | FP8GemmShape) -> int:
    return 2 * s.m * s.n * s.k


def gemm_bf16_bytes(s: GemmShape) -> int:
    return 2 * (s.m * s.k + s.k * s.n + s.m * s.n)


def gemm_fp8_bytes(s: FP8GemmShape) -> int:
    kb = s.k // 128
    nb = (s.n + 127) // 128
    return s.m * s.k + s.k * s.n + 2 * s.m * s.n + 4 * s.m * kb + 4 * kb * nb


def gqa_attention_flops(s: GQAShape) -> int:
    """Reference convention (flops.py:31-47): 4*B*Hq*S^2*D, causal not halved."""
    return 4 * s.batch * s.n_q * s.seq * s.seq * s.d_head


def gqa_causal_flops(s: GQAShape) -> int:
    """Work a causal kernel must do: query i attends to i+1 keys, so
    QK^T and PV each cost 2*D*sum_i(i+1) = D*S*(S+1) per head."""
    return 2 * s.batch * s.n_q * s.d_head * s.seq * (s.seq + 1)


def gqa_algorithmic_flops(s: GQAShape) -> int:
    return gqa_causal_flops(s) if s.causal else gqa_attention_flops(s)


def gqa_attention_bytes(s: GQAShape, dtype_bytes: int = 2) -> int:
    """Q, K, V read once, O written once (flops.py:54-66)."""
    return (2 * s.q_size + 2 * s.kv_size) * dtype_bytes


def mla_attention_flops(s: MLAShape) -> int:
    """2*B*n_h*S^2*(qk_head_dim + d_v) (flops_mla.py:32-45): full S x S,
    the reference's convention also for a causal run."""
    return 2 * s.batch * s.n_h * s.seq * s.seq * (s.qk_head_dim + s.d_v)


def mla_algorithmic_flops(s: MLAShape) -> int:
    """Work the kernel must do: full S x S, or S(S+1)/2 pairs when causal."""
    pairs = s.seq * (s.seq + 1) // 2 if s.causal else s.seq * s.seq
    return 2 * s.batch * s.n_h * pairs * (s.qk_head_dim + s.d_v)


def mla_attention_bytes(s: MLAShape, dtype_bytes: int = 2) -> int:
    """Q, K, V read once and O written once (flops_mla.py:52-64)."""
    return (2 * s.q_size + 2 * s.v_size) * dtype_bytes


def mla_decode_flops(s: MLADecodeShape) -> int:
    """2*B*H*T*(d_qk + d_latent): scores over 576 dims, values over 512."""
    return 2 * s.batch * s.n_h * s.ctx * (s.d_qk + s.d_latent)


def mla_decode_bytes(s: MLADecodeShape, dtype_bytes: int = 2) -> int:
    """Latent cache read once per sequence + Q read + O written."""
    kv = s.batch * s.ctx * s.d_qk
    q = s.batch * s.n_h * s.d_qk
    o = s.batch * s.n_h * s.d_latent
    return (kv + q + o) * dtype_bytes


def gdn_decode_flops(s: GDNShape) -> int:
    """6*B*H*d_k*d_v (flops_gdn.py:45-57)."""
    return 6 * s.batch * s.n_heads * s.d_k * s.d_v


def gdn_decode_bytes(s: GDNShape, io_bytes: int = 2, gate_bytes: int = 4) -> int:
    """fp32 state read + written, q/k per key head, v/o per value head,
    alpha/beta per value head (fp32 here; the reference's f16 gates are
    2 bytes each, flops_gdn.py:59-70)."""
    state = 2 * s.batch * s.n_heads * s.d_k * s.d_v * 4
    qk = 2 * s.batch * s.hk * s.d_k * io_bytes
    vo = 2 * s.batch * s.n_heads * s.d_v * io_bytes
    gates = 2 * s.batch * s.n_heads * gate_bytes
    return state + qk + vo + gates


def kda_decode_flops(s) -> int:
    """6*B*H*d_k*d_v (cutile-attn-kda/main.py:112-114)."""
    return 6 * s.batch * s.n_heads * s.d_k * s.d_v


def kda_decode_bytes(s, io_bytes: int = 2) -> int:
    """fp32 state read + written, plus q, k, g (d_k each), v, o (d_v each)
    and beta in the 16-bit I/O type per (b, h) (cutile-attn-kda/main.py:117-128)."""
    bh = s.batch * s.n_heads
    return bh * (2 * s.d_k * s.d_v * 4 + (3 * s.d_k + 2 * s.d_v + 1) * io_bytes)


def quant_fp8_act_bytes(m: int, k: int, io_bytes: int = 2) -> int:
    """16-bit activations read, e4m3 codes and 1x128 fp32 scales written."""
    return m * k * io_bytes + m * k + (m * k // 128) * 4


def tflops(flops: int, ms: float) -> float:
    return flops / (ms * 1e-3) / 1e12


def gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9
