"""Shape types and registries for the five kernels on the path.

Mirrors the reference's shape dataclasses
(analysis/wave15-attention-architecture/reference/shapes.py:20-54,
shapes_mla.py:26-67, shapes_gdn.py:27-80) and the GEMM harness constants
(cutile-matmul-tc-bf16/main.py:39-51), extended with what this path needs:
a causal flag for GQA, the absorbed-decode MLA shape (latent cache) and
separate key / value head counts for GDN.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class GemmShape:
    name: str
    m: int
    n: int
    k: int


@dataclass(frozen=True)
class GQAShape:
    """Grouped-query attention forward (reference shapes.py:20-54 + causal)."""

    name: str
    batch: int
    seq: int
    n_q: int
    n_kv: int
    d_head: int
    causal: bool = False

    @property
    def n_groups(self) -> int:
        return self.n_q // self.n_kv

    @property
    def q_size(self) -> int:
        return self.batch * self.seq * self.n_q * self.d_head

    @property
    def kv_size(self) -> int:
        return self.batch * self.seq * self.n_kv * self.d_head

    def assert_valid(self) -> None:
        assert self.n_q % self.n_kv == 0, f"{self.name}: n_q must be divisible by n_kv"


@dataclass(frozen=True)
class MLAShape:
    """Pre-projected MLA prefill (reference shapes_mla.py:26-67): every head
    has its own up-projected Q and K of qk_head_dim = d_h + d_rope and V of
    d_v; d_c (the latent rank) is carried but unused, as in the reference.
    `causal` is this path's addition (the reference cell is non-causal)."""

    name: str
    batch: int
    seq: int
    n_h: int
    d_h: int
    d_rope: int
    d_v: int
    d_c: int
    causal: bool = False

    @property
    def qk_head_dim(self) -> int:
        return self.d_h + self.d_rope

    @property
    def scale(self) -> float:
        return self.qk_head_dim ** -0.5

    @property
    def q_size(self) -> int:
        return self.batch * self.seq * self.n_h * self.qk_head_dim

    @property
    def v_size(self) -> int:
        return self.batch * self.seq * self.n_h * self.d_v

    def assert_valid(self) -> None:
        assert self.d_h > 0 and self.d_rope > 0 and self.d_v > 0
        assert self.n_h > 0 and self.seq > 0 and self.batch > 0
        assert self.d_c > 0


@dataclass(frozen=True)
class MLADecodeShape:
    """Weight-absorbed MLA decode: one query token per sequence, latent cache.

    Q [batch, n_h, d_latent + d_rope], KV [batch, ctx, d_latent + d_rope],
    O [batch, n_h, d_latent].  The softmax scale is 1/sqrt(qk_head_dim) with
    qk_head_dim = d_h + d_rope = 192 (reference shapes_mla.py:47-49 and
    pytorch_reference_mla.py:75), which absorption leaves unchanged.
    """

    name: str
    batch: int
    n_h: int
    ctx: int
    d_latent: int = 512
    d_rope: int = 64
    qk_head_dim: int = 192

    @property
    def d_qk(self) -> int:
        return self.d_latent + self.d_rope

    @property
    def scale(self) -> float:
        return self.qk_head_dim ** -0.5

    def assert_valid(self) -> None:
        assert self.batch > 0 and self.n_h > 0 and self.ctx > 0
        assert self.d_latent > 0 and self.d_rope >= 0


@dataclass(frozen=True)
class GDNShape:
    """GDN decode (reference shapes_gdn.py:27-80) with n_k_heads <= n_heads.

    n_heads is the number of value heads (one fp32 state tile each); the key
    head of value head h is h // (n_heads // n_k_heads).
    """

    name: str
    batch: int
    n_heads: int
    d_k: int
    d_v: int
    n_k_heads: int | None = field(default=None)

    @property
    def hk(self) -> int:
        return self.n_k_heads if self.n_k_heads is not None else self.n_heads

    @property
    def state_elems(self) -> int:
        return self.batch * self.n_heads * self.d_k * self.d_v

    def assert_valid(self) -> None:
        assert self.d_k > 0 and self.d_v > 0 and self.batch > 0 and self.n_heads > 0
        assert self.n_heads % self.hk == 0


@dataclass(frozen=True)
class KDAShape:
    """KDA decode (cutile-attn-kda/main.py:64-74): one key head per value head."""

    name: str
    batch: int
    n_heads: int
    d_k: int
    d_v: int

    @property
    def state_elems(self) -> int:
        return self.batch * self.n_heads * self.d_k * self.d_v

    def assert_valid(self) -> None:
        assert self.d_k > 0 and self.d_v > 0 and self.batch > 0 and self.n_heads > 0


@dataclass(frozen=True)
class FP8GemmShape:
    name: str
    m: int
    n: int
    k: int


# ---------------------------------------------------------------------------
# GEMM: reference smoke N=512 and bench sizes (cutile-matmul-tiled-mixed/main.py:55-60);
# BASELINE parity config 1024^3 and the 8192^3 roofline target.
GEMM_SMOKE = GemmShape("smoke", 512, 512, 512)
GEMM_PARITY = GemmShape("parity_1024", 1024, 1024, 1024)
GEMM_TARGET = GemmShape("target_8192", 8192, 8192, 8192)
GEMM_REGISTRY = {s.name: s for s in (GEMM_SMOKE, GEMM_PARITY, GEMM_TARGET,
                                       GemmShape("n2048", 2048, 2048, 2048),
                                       GemmShape("n4096", 4096, 4096, 4096))}

# fp8 block-scaled GEMM.
FP8_SMOKE = FP8GemmShape("smoke", 256, 256, 512)
FP8_TARGET = FP8GemmShape("target_8192", 8192, 8192, 8192)
FP8_REGISTRY = {s.name: s for s in (FP8_SMOKE, FP8_TARGET, FP8GemmShape("n4096", 4096, 4096, 4096))}

# GQA: reference correctness / llama3_8b shapes (shapes.py:57-74), plus the
# causal bf16 configuration this path is measured on.
GQA_CORRECTNESS = GQAShape("correctness", batch=1, seq=128, n_q=4, n_kv=2, d_head=64)
GQA_LLAMA3_8B = GQAShape("llama3_8b", batch=1, seq=2048, n_q=32, n_kv=8, d_head=128)
GQA_CORRECTNESS_CAUSAL = GQAShape("correctness_causal", batch=1, seq=128, n_q=4, n_kv=2, d_head=64, causal=True)
GQA_BASELINE = GQAShape("llama3_8b_causal_s4096", batch=1, seq=4096, n_q=32, n_kv=8, d_head=128, causal=True)
GQA_REGISTRY = {s.name: s for s in (GQA_CORRECTNESS, GQA_LLAMA3_8B, GQA_CORRECTNESS_CAUSAL, GQA_BASELINE)}

# MLA absorbed decode.
MLA_CORRECTNESS = MLADecodeShape("correctness_mla_decode", batch=2, n_h=16, ctx=200)
MLA_BASELINE = MLADecodeShape("deepseek_v3_decode", batch=32, n_h=128, ctx=4096)
MLA_REGISTRY = {s.name: s for s in (MLA_CORRECTNESS, MLA_BASELINE)}

# MLA prefill (pre-projected Q/K/V; shapes_mla.py:70-93).
MLA_PREFILL_CORRECTNESS = MLAShape("correctness_mla", batch=1, seq=128, n_h=4, d_h=64, d_rope=32, d_v=64, d_c=128)
MLA_PREFILL_BENCH = MLAShape("deepseek_v3", batch=1, seq=2048, n_h=128, d_h=128, d_rope=64, d_v=128, d_c=512)
MLA_PREFILL_REGISTRY = {s.name: s for s in (MLA_PREFILL_CORRECTNESS, MLA_PREFILL_BENCH)}

# GDN: reference registry (cutile-attn-gdn/main.py:62-72, shapes_gdn.py:85-104)
# and the Qwen3-Next-like batch-64 configuration this path is measured on.
GDN_CORRECTNESS = GDNShape("correctness", batch=2, n_heads=4, d_k=64, d_v=64)
GDN_QWEN3_NEXT = GDNShape("qwen3_next_decode", batch=1, n_heads=16, d_k=256, d_v=256)
GDN_BASELINE = GDNShape("qwen3_next_b64", batch=64, n_heads=32, d_k=128, d_v=128, n_k_heads=16)
GDN_REGISTRY = {s.name: s for s in (
    GDN_CORRECTNESS, GDN_QWEN3_NEXT, GDN_BASELINE,
    GDNShape("tiny", batch=1, n_heads=4, d_k=64, d_v=64),
    GDNShape("small", batch=1, n_heads=8, d_k=128, d_v=128),
    GDNShape("large", batch=4, n_heads=64, d_k=256, d_v=256),
    GDNShape("wide", batch=1, n_heads=16, d_k=512, d_v=512),
)}
# The reference sweep's shapes, in its order (cuda-attn-gdn-tma/bench_sweep.cu:302-309).
GDN_SWEEP = ("qwen3_next_decode", "tiny", "small", "large", "wide")

# KDA: reference registry (cutile-attn-kda/main.py:77-104).  "large" is the
# configuration this path is measured on (it fills the GPU).
KDA_CORRECTNESS = KDAShape("correctness", batch=1, n_heads=2, d_k=64, d_v=64)
KDA_KIMI_LINEAR = KDAShape("kimi_linear_decode", batch=1, n_heads=32, d_k=128, d_v=128)
KDA_QWEN3_PARITY = KDAShape("qwen3_next_gdn_parity", batch=1, n_heads=16, d_k=256, d_v=256)
KDA_LARGE = KDAShape("large", batch=4, n_heads=64, d_k=256, d_v=256)
KDA_REGISTRY = {s.name: s for s in (KDA_CORRECTNESS, KDA_KIMI_LINEAR, KDA_QWEN3_PARITY, KDA_LARGE)}
