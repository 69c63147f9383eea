"""Write the committed golden fixtures (inputs + oracle outputs) for small cases.

Run from the repo root:  python tests/golden/gen_golden.py
Each fixture stores its inputs bit-exactly (bf16 / f16 as uint16, e4m3 as
uint8) so parity never depends on RNG versions, plus the CPU oracle's fp32
expected outputs.  The reference commits no fixtures of its own (its
inputs/ directory is git-ignored), so these are generated from this
repository's oracle restatement and seeded generators.
"""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
pkg = importlib.import_module("cuda-oxide-bench_amd")
S = pkg.shapes
inputs = pkg.inputs

from oracle import fp8 as ofp8  # noqa: E402
from oracle import gdn as ogdn  # noqa: E402
from oracle import gemm as ogemm  # noqa: E402
from oracle import gqa as ogqa  # noqa: E402
from oracle import kda as okda  # noqa: E402
from oracle import mla as omla  # noqa: E402

OUT = Path(__file__).resolve().parent


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint16).numpy().copy() if t.dtype != torch.uint16 else t.numpy()


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def save(name: str, **arrays) -> None:
    path = OUT / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    print(f"wrote {path.relative_to(REPO)} ({path.stat().st_size} bytes)")


def main() -> int:
    # bf16 GEMM, ragged against every tile size.
    gs = S.GemmShape("golden", 72, 136, 96)
    a, b = inputs.gemm_inputs(gs, seed=0x601D)
    save("gemm_bf16_72x136x96", a=bits16(a), b=bits16(b), c=ogemm.gemm_ref(a, b).numpy())

    # fp8 block-scaled GEMM.
    fs = S.FP8GemmShape("golden", 48, 272, 256)
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(fs, seed=0xF8)
    ac, bc = ofp8.fp8_tensor_codes(a8), ofp8.fp8_tensor_codes(b8)
    save("gemm_fp8_48x272x256", a=ac, sa=sa.numpy(), b=bc, sb=sb.numpy(),
         c=ofp8.gemm_fp8_bs_ref(ac, sa.numpy(), bc, sb.numpy()))

    # GQA: the reference's correctness shape and distribution (f16, non-causal),
    # and a small causal bf16 case with BASELINE's distribution.
    g1 = S.GQA_CORRECTNESS
    q, k, v = inputs.gqa_inputs(g1, dtype=torch.float16, dist="reference")
    save("gqa_correctness_f16", q=bits16(q), k=bits16(k), v=bits16(v),
         o=ogqa.gqa_naive(q, k, v, causal=False).numpy(), shape=np.array([1, 128, 4, 2, 64, 0]))
    g2 = S.GQAShape("golden_causal", batch=1, seq=80, n_q=4, n_kv=2, d_head=128, causal=True)
    q, k, v = inputs.gqa_inputs(g2, dtype=torch.bfloat16, seed=0x6A)
    save("gqa_causal_bf16_s80", q=bits16(q), k=bits16(k), v=bits16(v),
         o=ogqa.gqa_naive(q, k, v, causal=True).numpy(), shape=np.array([1, 80, 4, 2, 128, 1]))

    # MLA absorbed decode.
    ms = S.MLADecodeShape("golden", batch=1, n_h=16, ctx=40)
    q, kv = inputs.mla_inputs(ms, seed=0x41A)
    save("mla_decode_h16_t40", q=bits16(q), kv=bits16(kv),
         o=omla.mla_decode_ref(q, kv, ms.scale).numpy(), scale=np.array([ms.scale], dtype=np.float64))

    # MLA prefill: the reference's correctness shape and recipe (f16, qk 96, v 64).
    mp = S.MLA_PREFILL_CORRECTNESS
    q, k, v = inputs.mla_prefill_inputs(mp, dtype=torch.float16)
    save("mla_prefill_correctness_f16", q=bits16(q), k=bits16(k), v=bits16(v),
         o=omla.mla_prefill_ref(q, k, v).numpy())

    # GDN: reference correctness shape/distribution (f16) and a grouped bf16 case.
    d1 = S.GDN_CORRECTNESS
    x = inputs.gdn_inputs(d1, dtype=torch.float16, dist="reference")
    o, so = ogdn.gdn_decode_ref(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"])
    save("gdn_correctness_f16", q=bits16(x["q"]), k=bits16(x["k"]), v=bits16(x["v"]),
         alpha=x["alpha"].numpy(), beta=x["beta"].numpy(), S_in=x["S_in"].numpy(),
         o=o.numpy(), S_out=so.numpy())
    d2 = S.GDNShape("golden_grouped", batch=2, n_heads=4, d_k=64, d_v=128, n_k_heads=2)
    x = inputs.gdn_inputs(d2, dtype=torch.bfloat16, seed=0x6D)
    o, so = ogdn.gdn_decode_ref(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"])
    save("gdn_grouped_bf16", q=bits16(x["q"]), k=bits16(x["k"]), v=bits16(x["v"]),
         alpha=x["alpha"].numpy(), beta=x["beta"].numpy(), S_in=x["S_in"].numpy(),
         o=o.numpy(), S_out=so.numpy())

    # KDA: the reference's correctness shape and recipe (f16, seed 17).
    x = inputs.kda_inputs(S.KDA_CORRECTNESS)
    o, so = okda.kda_decode_ref(**x)
    save("kda_correctness_f16", q=bits16(x["q"]), k=bits16(x["k"]), v=bits16(x["v"]), g=bits16(x["g"]),
         beta=bits16(x["beta"]), S_in=x["S_in"].numpy(), o=o, S_out=so)
    return 0


if __name__ == "__main__":
    sys.exit(main())
