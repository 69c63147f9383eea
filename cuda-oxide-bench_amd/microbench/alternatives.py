"""What a kernel's alternative designs cost, and what its operands do to the
clock: variants of one kernel source, each built as its own kernel library
and timed on the GPU.

    python cuda-oxide-bench_amd/microbench/alternatives.py build fp8   # CPU: patch, compile, check, link
    python cuda-oxide-bench_amd/microbench/alternatives.py run fp8     # GPU: time every variant, interleaved
    ... run gqa --variants as_built --inputs random,constant           # the same launches on constant operands

Every variant is an alternative design (alt_*): it computes what the kernel
as built computes, and run compares its output with the kernel as built's
bit for bit, by SHA-256.  No variant removes work; the input modes time the
kernel as built on random operands and on constant ones.

build: for each variant, a copy of the kernel source gets the variant's
text patches (each anchor must occur exactly the stated number of times,
once unless given, so a patch cannot drift onto other code), is compiled
with the library's own flags and linked with the package's other objects
(from its last build) into microbench/_alternatives/<kernel>/<variant>/
libmxkernels.so.  Before linking, an fp8 variant's gfx950 assembly goes
through the same check as tests/test_fp8_scale_loads.py: every untracked
scale load is landed by its wait before any instruction names its
register; a variant that fails is not built.

run: each variant's library is loaded in a process of its own
(MX_KERNELS_LIB) and timed like bench.py's graph-replayed cases (warm-up
calls, one graph of 20 launches, replayed after 300 ms of a device GEMM);
the variants (and input modes) take turn, --runs times.  Every variant
keeps every memory access in bounds and every wait count exact, as its
description says.
"""
from __future__ import annotations

import argparse
import os
import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG_DIR = HERE.parent
REPO_ROOT = PKG_DIR.parent
OUT_ROOT = HERE / "_alternatives"

# ---------------------------------------------------------------------------
# fp8 block-scaled GEMM (csrc/gemm_fp8_bs.hip), 8192^3.  Patches as
# (anchor, replacement); a variant is the concatenation of its parts.
# ---------------------------------------------------------------------------
FP8_PARTS = {
    # ---- alternative designs (each computes what the kernel as built does) ----
    # Order of a block's tile loads (the A block stays last, so the waits
    # stay exact).  As built: spread evenly over the four row blocks.
    "loads_b_first": [('    auto dma_share = [&](int mf) {\n#pragma unroll\n      for (int n = (NLD * mf) / FM; n < (NLD * (mf + 1)) / FM; ++n) {\n        if (n < 2 * CF::B_LPW)\n          issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n        else\n          issue_a(j + 2, n - 2 * CF::B_LPW);\n      }\n    };\n', '    auto dma_share = [&](int mf) {\n      if (mf == 0) {\n#pragma unroll\n        for (int n = 0; n < 2 * CF::B_LPW; ++n) issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n      } else {\n#pragma unroll\n        for (int n = (CF::A_LPW * (mf - 1)) / (FM - 1); n < (CF::A_LPW * mf) / (FM - 1); ++n) issue_a(j + 2, n);\n      }\n    };\n')],
    "loads_after_barrier": [('    auto dma_share = [&](int mf) {\n#pragma unroll\n      for (int n = (NLD * mf) / FM; n < (NLD * (mf + 1)) / FM; ++n) {\n        if (n < 2 * CF::B_LPW)\n          issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n        else\n          issue_a(j + 2, n - 2 * CF::B_LPW);\n      }\n    };\n', '    auto dma_share = [&](int mf) { (void)mf; };\n#pragma unroll\n    for (int n = 0; n < NLD; ++n) {\n      if (n < 2 * CF::B_LPW)\n        issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n      else\n        issue_a(j + 2, n - 2 * CF::B_LPW);\n    }\n')],
    "b_loads_after_barrier": [('    auto dma_share = [&](int mf) {\n#pragma unroll\n      for (int n = (NLD * mf) / FM; n < (NLD * (mf + 1)) / FM; ++n) {\n        if (n < 2 * CF::B_LPW)\n          issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n        else\n          issue_a(j + 2, n - 2 * CF::B_LPW);\n      }\n    };\n', '    auto dma_share = [&](int mf) {\n#pragma unroll\n      for (int n = (CF::A_LPW * mf) / FM; n < (CF::A_LPW * (mf + 1)) / FM; ++n) issue_a(j + 2, n);\n    };\n#pragma unroll\n    for (int n = 0; n < 2 * CF::B_LPW; ++n) issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);\n')],
    # Activation scales eight blocks per 16-byte load when K % 1024 == 0
    # and sA is 16-byte aligned (four per 8-byte load otherwise, as built).
    "act_scales_8": [
        ("__device__ __forceinline__ void ld_scales_if(u32x2 (&x)[2], const float* sbase, const uint32_t (&voff)[2],\n",
         "__device__ __forceinline__ void ld_scales_if(u32x4 (&x)[4], const float* sbase, const uint32_t (&voff)[4],\n"
         "                                             uint32_t go) {\n"
         "  asm volatile(\n"
         "      \"s_cmp_eq_u32 %[go], 0\\n\\t\"\n"
         "      \"s_cbranch_scc1 1f\\n\\t\"\n"
         "      \"global_load_dwordx4 %0, %4, %[b]\\n\\t\"\n"
         "      \"global_load_dwordx4 %1, %5, %[b]\\n\\t\"\n"
         "      \"global_load_dwordx4 %2, %6, %[b]\\n\\t\"\n"
         "      \"global_load_dwordx4 %3, %7, %[b]\\n\"\n"
         "      \"1:\"\n"
         "      : \"+v\"(x[0]), \"+v\"(x[1]), \"+v\"(x[2]), \"+v\"(x[3])\n"
         "      : \"v\"(voff[0]), \"v\"(voff[1]), \"v\"(voff[2]), \"v\"(voff[3]), [b] \"s\"(sbase), [go] \"s\"(go)\n"
         "      : \"memory\", \"scc\");\n"
         "}\n"
         "__device__ __forceinline__ void ld_scales_if(u32x4 (&x)[2], const float* sbase, const uint32_t (&voff)[2],\n"
         "                                             uint32_t go) {\n"
         "  asm volatile(\n"
         "      \"s_cmp_eq_u32 %[go], 0\\n\\t\"\n"
         "      \"s_cbranch_scc1 1f\\n\\t\"\n"
         "      \"global_load_dwordx4 %0, %2, %[b]\\n\\t\"\n"
         "      \"global_load_dwordx4 %1, %3, %[b]\\n\"\n"
         "      \"1:\"\n"
         "      : \"+v\"(x[0]), \"+v\"(x[1])\n"
         "      : \"v\"(voff[0]), \"v\"(voff[1]), [b] \"s\"(sbase), [go] \"s\"(go)\n"
         "      : \"memory\", \"scc\");\n"
         "}\n"
         "__device__ __forceinline__ void ld_scales_if(u32x2 (&x)[2], const float* sbase, const uint32_t (&voff)[2],\n"),
        ("template <int BM, int BN, bool GS>\n__global__", "template <int BM, int BN, int G>\n__global__"),
        ("* (uint32_t)kblocks * 4u + (GS ? 8u * (lane >> 5) : 0u);",
         "* (uint32_t)kblocks * 4u + (G > 1 ? 2u * G * (uint32_t)(lane >> 5) : 0u);"),
        ("  std::conditional_t<GS, u32x2, float> sa_n[FM];",
         "  constexpr bool GS = G > 1;\n  constexpr int LG = G == 8 ? 3 : G == 4 ? 2 : 0;\n"
         "  std::conditional_t<G == 8, u32x4, std::conditional_t<G == 4, u32x2, float>> sa_n[FM];"),
        ("      ld_scales_if(sa_n, sA + min(j + 1, kblocks - 4), sa_off, (uint32_t)(((j & 3) + 1) >> 2));",
         "      ld_scales_if(sa_n, sA + min(j + 1, kblocks - G), sa_off, (uint32_t)(((j & (G - 1)) + 1) >> LG));"),
        ("    if constexpr (GS) {\n      const uint32_t v = (t & 1) ? sa_n[mf][1] : sa_n[mf][0];",
         "    if constexpr (G == 8) {\n      const uint32_t v01 = (t & 1) ? sa_n[mf][1] : sa_n[mf][0];\n"
         "      const uint32_t v23 = (t & 1) ? sa_n[mf][3] : sa_n[mf][2];\n      const uint32_t v = (t & 2) ? v23 : v01;\n"
         "      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);\n"
         "      return __uint_as_float(t < 4 ? r[0] : r[1]);\n    } else if constexpr (G == 4) {\n"
         "      const uint32_t v = (t & 1) ? sa_n[mf][1] : sa_n[mf][0];"),
        ("s_m[mf] = sa_of(j & 3, mf) * sb_n;", "s_m[mf] = sa_of(j & (G - 1), mf) * sb_n;"),
        ("template <int BM, int BN, bool GS>\nstatic int launch(", "template <int BM, int BN, int G>\nstatic int launch("),
        ("  constexpr auto kern = gemm_fp8_bs_kernel<BM, BN, GS>;", "  constexpr auto kern = gemm_fp8_bs_kernel<BM, BN, G>;"),
        ("  if (K % 512 == 0 && ((uintptr_t)sA & 7) == 0)\n"
         "    return big ? mx::gemm8::launch<256, 256, true>(A, sA, B, sB, C, M, N, K, s)\n"
         "               : mx::gemm8::launch<128, 128, true>(A, sA, B, sB, C, M, N, K, s);\n"
         "  return big ? mx::gemm8::launch<256, 256, false>(A, sA, B, sB, C, M, N, K, s)\n"
         "             : mx::gemm8::launch<128, 128, false>(A, sA, B, sB, C, M, N, K, s);",
         "  if (K % 1024 == 0 && ((uintptr_t)sA & 15) == 0)\n"
         "    return big ? mx::gemm8::launch<256, 256, 8>(A, sA, B, sB, C, M, N, K, s)\n"
         "               : mx::gemm8::launch<128, 128, 8>(A, sA, B, sB, C, M, N, K, s);\n"
         "  if (K % 512 == 0 && ((uintptr_t)sA & 7) == 0)\n"
         "    return big ? mx::gemm8::launch<256, 256, 4>(A, sA, B, sB, C, M, N, K, s)\n"
         "               : mx::gemm8::launch<128, 128, 4>(A, sA, B, sB, C, M, N, K, s);\n"
         "  return big ? mx::gemm8::launch<256, 256, 1>(A, sA, B, sB, C, M, N, K, s)\n"
         "             : mx::gemm8::launch<128, 128, 1>(A, sA, B, sB, C, M, N, K, s);"),
    ],
    # Each block's LDS read bases (lane address + slot offset) computed once
    # and hidden from the compiler, so every fragment read carries its own
    # offset as an immediate (8 address adds per block instead of 24).
    "read_bases": [
        ("  auto read_b = [&](uint32_t so, int nf) {\n    u32x2 v[4];\n#pragma unroll\n"
         "    for (int r = 0; r < 4; ++r) v[r] = lds_read_tr8_at(b_col[nf] + so + 8 * r * BN);",
         "  auto read_b = [&](uint32_t base) {\n    u32x2 v[4];\n#pragma unroll\n"
         "    for (int r = 0; r < 4; ++r) v[r] = lds_read_tr8_at(base + 8 * r * BN);"),
        ("  auto read_a = [&](uint32_t so, int kh, int mf) {\n    const uint32_t r = so + 32 * mf * SBK;\n"
         "    const u32x4 lo = lds_ld128(a_col[kh][0] + r);\n    const u32x4 hi = lds_ld128(a_col[kh][1] + r);",
         "  auto read_a = [&](const uint32_t (&base)[2], int mf) {\n"
         "    const u32x4 lo = lds_ld128(base[0] + 32 * mf * SBK);\n    const u32x4 hi = lds_ld128(base[1] + 32 * mf * SBK);"),
        ("    const uint32_t so0 = ((2 * j) % NSB) * CF::B_S, so1 = ((2 * j + 1) % NSB) * CF::B_S;\n",
         "    const uint32_t so0 = ((2 * j) % NSB) * CF::B_S, so1 = ((2 * j + 1) % NSB) * CF::B_S;\n"
         "    uint32_t ab[2][2], bb0[FN], bb1[FN];\n#pragma unroll\n    for (int kh = 0; kh < 2; ++kh)\n#pragma unroll\n"
         "      for (int h = 0; h < 2; ++h) {\n        ab[kh][h] = a_col[kh][h] + ao;\n        asm(\"\" : \"+v\"(ab[kh][h]));\n      }\n"
         "#pragma unroll\n    for (int nf = 0; nf < FN; ++nf) {\n      bb0[nf] = b_col[nf] + so0;\n      bb1[nf] = b_col[nf] + so1;\n"
         "      asm(\"\" : \"+v\"(bb0[nf]));\n      asm(\"\" : \"+v\"(bb1[nf]));\n    }\n"),
        ("    bf0[0] = read_b(so0, 0);\n    a0 = read_a(ao, 0, 0);\n    bf1[0] = read_b(so1, 0);\n    a1 = read_a(ao, 1, 0);",
         "    bf0[0] = read_b(bb0[0]);\n    a0 = read_a(ab[0], 0);\n    bf1[0] = read_b(bb1[0]);\n    a1 = read_a(ab[1], 0);"),
        ("          bf0[nf + 1] = read_b(so0, nf + 1);\n          bf1[nf + 1] = read_b(so1, nf + 1);",
         "          bf0[nf + 1] = read_b(bb0[nf + 1]);\n          bf1[nf + 1] = read_b(bb1[nf + 1]);"),
        ("          if (mf + 1 < FM) a0 = read_a(ao, 0, mf + 1);", "          if (mf + 1 < FM) a0 = read_a(ab[0], mf + 1);"),
        ("        if (nf == FN - 1 && mf + 1 < FM) a1 = read_a(ao, 1, mf + 1);",
         "        if (nf == FN - 1 && mf + 1 < FM) a1 = read_a(ab[1], mf + 1);"),
    ],
}
FP8_VARIANTS = {
    "as_built": ("the kernel as built", []),
    "alt_loads_b_first": ("both B stages in the first row block's share, the A block over the next ones",
                          ["loads_b_first"], True),
    "alt_loads_after_barrier": ("all eight tile loads right after the barrier", ["loads_after_barrier"], True),
    "alt_b_loads_after_barrier": ("the B stages right after the barrier, the A block spread",
                                  ["b_loads_after_barrier"], True),
    "alt_act_scales_8": ("activation scales eight blocks per 16-byte load (K % 1024 == 0)", ["act_scales_8"], True),
    "alt_read_bases": ("per-block LDS read bases, fragment offsets as immediates", ["read_bases"], True),
}

# ---------------------------------------------------------------------------
# Causal GQA forward (csrc/gqa_fwd.hip): B1 Hq32 Hkv8
# S4096 D128 bf16, default tile.  Only the default kernel is launched.
# ---------------------------------------------------------------------------
GQA_PARTS = {
    # ---- alternative designs (each computes what the kernel as built does) ----
    # The next tile's loads unconditional and branch-free, valid when S is a
    # multiple of 64 (the timed shape): past the last tile the last tile
    # again into the free stage, from a scalar tile base plus the
    # precomputed lane offsets (no row clamp, no address VALU, no branch);
    # the loop then waits for those loads before the ring is reused.
    "branch_free_loads": [
        ("  auto issue = [&](int blk) {\n    const int kv0 = blk * BN;",
         "  auto issue_full = [&](int src, int slot, int n) {\n    const int ld = wave * L::LPW + n;\n"
         "    const bool vt = ld >= L::NLK;\n    const int kv0 = src * BN;\n"
         "    dma16((vt ? Vh + (size_t)kv0 * L::ROWV : Kh + (size_t)kv0 * L::ROWK), ld_off[n],\n"
         "          lds0 + slot * L::STAGE + ld * 1024);\n  };\n"
         "  auto issue = [&](int blk) {\n    const int kv0 = blk * BN;"),
        ("          if (dc == n * DC / L::LPW && load_next) issue_part(blk + NS - 1, n);",
         "          if (dc == n * DC / L::LPW) issue_full(load_next ? blk + NS - 1 : nblk - 1, (blk + NS - 1) % NS, n);"),
        ("      if (blk + 2 < nblk) tile(blk + 2, std::integral_constant<int, 2>{});\n  }\n",
         "      if (blk + 2 < nblk) tile(blk + 2, std::integral_constant<int, 2>{});\n  }\n  wait_vmcnt<0>();\n"),
    ],
    # K fragments read three k-steps ahead instead of two.
    "k_lookahead_3": [
        ("      constexpr int KLA = DQK > 128 ? 1 : 2;", "      constexpr int KLA = DQK > 128 ? 1 : 3;"),
    ],
    # No wave priority (s_setprio) around the MFMA phases.
    "no_setprio": [
        ("      __builtin_amdgcn_s_setprio(1);\n", "", 2),
        ("      __builtin_amdgcn_s_setprio(0);\n", "", 2),
    ],
}
GQA_VARIANTS = {
    "as_built": ("the kernel as built", []),
    "alt_branch_free_loads": ("next tile's loads unconditional and branch-free (S % 64 == 0 only)",
                              ["branch_free_loads"], True),
    "alt_k_lookahead_3": ("K fragment reads three k-steps ahead instead of two", ["k_lookahead_3"], True),
    "alt_no_setprio": ("no wave priority around the MFMA phases", ["no_setprio"], True),
}

KERNELS = {
    "fp8": {"source": "gemm_fp8_bs.hip", "parts": FP8_PARTS, "variants": FP8_VARIANTS,
            "workload": "gemm_fp8_bs M8192 N8192 K8192 e4m3 1x128/128x128 scales",
            "kernel_prefix": "_ZN2mx5gemm818gemm_fp8_bs_kernel"},
    "gqa": {"source": "gqa_fwd.hip", "parts": GQA_PARTS, "variants": GQA_VARIANTS,
            "workload": "gqa_fwd causal B1 Hq32 Hkv8 S4096 D128 bf16, default tile",
            "kernel_prefix": "_ZN2mx3gqa14gqa_fwd_kernel"},
    "bf16_8192": {"source": "gemm_bf16.hip", "parts": {}, "variants": {"as_built": ("the kernel as built", [])},
                  "workload": "gemm_bf16 M8192 N8192 K8192 U[-1,1] (gemm_bf16_dma16s_kernel)",
                  "kernel_prefix": "_ZN2mx4gemm23gemm_bf16_dma16s_kernel"},
    "mla": {"source": "mla_decode.hip", "parts": {}, "variants": {"as_built": ("the decode and merge as built", [])},
            "workload": "mla_decode absorbed B32 H128 T4096 576/512 bf16, decode + merge, same buffers",
            "kernel_prefix": "_ZN2mx3mla17mla_decode_kernel"},
}


def _package_build():
    sys.path.insert(0, str(PKG_DIR))
    import build  # the package's build module (flags, hipcc)

    return build


def variant_exact(kernel: str, variant: str) -> bool:
    """Whether the variant is marked as computing what the kernel as built
    computes (every variant here but the kernel as built itself)."""
    v = KERNELS[kernel]["variants"][variant]
    return len(v) > 2 and bool(v[2])


def patched_source(kernel: str, variant: str) -> str:
    """The kernel source with the variant's patches: (anchor, replacement)
    pairs whose anchor must occur exactly once, or (anchor, replacement,
    count) for an anchor that must occur exactly count times."""
    spec = KERNELS[kernel]
    text = (PKG_DIR / "csrc" / spec["source"]).read_text()
    for part in spec["variants"][variant][1]:
        for patch in spec["parts"][part]:
            anchor, repl = patch[0], patch[1]
            want = patch[2] if len(patch) > 2 else 1
            n = text.count(anchor)
            if n != want:
                raise RuntimeError(f"{kernel}/{variant}: patch anchor of part {part!r} occurs {n} times, not {want}: "
                                   f"{anchor!r}")
            text = text.replace(anchor, repl)
    return text


def _check_fp8_scale_loads(asm: str, prefix: str) -> None:
    sys.path.insert(0, str(REPO_ROOT / "tests"))
    import asm_walk  # noqa: F401  (used by the check below)
    import importlib.util

    spec = importlib.util.spec_from_file_location("fp8_scale_check", REPO_ROOT / "tests" / "test_fp8_scale_loads.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    kernels = {n: b for n, b in asm_walk.kernels(asm).items() if n.startswith(prefix)}
    if not kernels:
        raise RuntimeError("no fp8 GEMM kernel in the variant's assembly")
    for name, body in kernels.items():
        nloads, problems = mod._check_kernel(body)
        if nloads == 0 or problems:
            raise RuntimeError(f"{name}: {nloads} scale loads; " + "; ".join(problems[:3]))


def build_variants(kernel: str, variants: list[str]) -> None:
    b = _package_build()
    spec = KERNELS[kernel]
    src_name = spec["source"]
    others = sorted(p for p in (PKG_DIR / "_build").glob("*.o") if p.stem != Path(src_name).stem)
    if not others:
        raise RuntimeError("build the package first (python cuda-oxide-bench_amd/build.py)")
    flags = b.common_flags() + b.source_flags(PKG_DIR / "csrc" / src_name)
    for v in variants:
        d = OUT_ROOT / kernel / v
        d.mkdir(parents=True, exist_ok=True)
        src = d / src_name
        src.write_text(patched_source(kernel, v))
        asm = d / (src.stem + ".s")
        dev = [f for f in flags if f != "-fPIC"]
        for cmd in ([b.hipcc(), *dev, "--cuda-device-only", "-S", str(src), "-o", str(asm)],
                    [b.hipcc(), *flags, "-c", str(src), "-o", str(d / (src.stem + ".o"))]):
            p = subprocess.run(cmd, capture_output=True, text=True)
            if p.returncode != 0:
                raise RuntimeError(f"{kernel}/{v}: compile failed\n{p.stderr[-3000:]}")
        if kernel == "fp8":
            _check_fp8_scale_loads(asm.read_text(), spec["kernel_prefix"])
        lib = d / "libmxkernels.so"
        p = subprocess.run([b.hipcc(), f"--offload-arch={b.ARCH}", "-shared", "-fPIC", "-o", str(lib),
                            str(d / (src.stem + ".o")), *map(str, others)], capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError(f"{kernel}/{v}: link failed\n{p.stderr[-3000:]}")
        print(f"built {kernel}/{v}: {lib}", flush=True)


def time_one(kernel: str, inputs: str = "random", steps: int = 20, warmup: int = 3,
             settle_ms: float = 300.0) -> tuple[float, str]:
    """Mean µs per launch of one graph replay (this process's kernel
    library), and the SHA-256 of the output of one more call.  inputs
    "constant" fills every operand with one value (fp8: code 0x38 = 1.0 with
    unit scales; otherwise 0.5): the same work on operands that switch
    nothing in the MFMA datapath."""
    import hashlib
    import importlib
    import time

    import torch

    sys.path.insert(0, str(REPO_ROOT))
    pkg = importlib.import_module("cuda-oxide-bench_amd")
    ops = pkg.load_ops()
    if kernel == "fp8":
        a8, sa, b8, sb = (t.cuda() for t in
                          pkg.inputs.fp8_gemm_inputs(pkg.shapes.FP8GemmShape("t", 8192, 8192, 8192)))
        out = torch.empty((8192, 8192), dtype=torch.bfloat16, device="cuda")
        fn = lambda: ops.gemm_fp8_bs(a8, sa, b8, sb, out=out)  # noqa: E731
    elif kernel == "gqa":
        gen = torch.Generator(device="cuda").manual_seed(0)
        q = torch.randn((1, 32, 4096, 128), device="cuda", generator=gen).to(torch.bfloat16)
        k = torch.randn((1, 8, 4096, 128), device="cuda", generator=gen).to(torch.bfloat16)
        v = torch.randn((1, 8, 4096, 128), device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty_like(q)
        fn = lambda: ops.gqa_fwd(q, k, v, causal=True, out=out)  # noqa: E731
    elif kernel == "mla":
        gen = torch.Generator(device="cuda").manual_seed(0)
        q = torch.randn((32, 128, 576), device="cuda", generator=gen).to(torch.bfloat16)
        kv = torch.randn((32, 4096, 576), device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty((32, 128, 512), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(max(1, ops.mla_decode_workspace_bytes(32, 128, 4096)), dtype=torch.uint8, device="cuda")
        fn = lambda: ops.mla_decode(q, kv, 192 ** -0.5, out=out, workspace=ws)  # noqa: E731
    elif kernel == "bf16_8192":
        gen = torch.Generator(device="cuda").manual_seed(0)
        a = (torch.rand((8192, 8192), device="cuda", generator=gen) * 2 - 1).to(torch.bfloat16)
        b = (torch.rand((8192, 8192), device="cuda", generator=gen) * 2 - 1).to(torch.bfloat16)
        out = torch.empty((8192, 8192), dtype=torch.bfloat16, device="cuda")
        fn = lambda: ops.gemm_bf16(a, b, out=out)  # noqa: E731
    else:
        raise ValueError(kernel)
    if inputs == "constant":
        for name, t in list(locals().items()):
            if name in ("a8", "b8"):
                t.view(torch.uint8).fill_(0x38)
            elif name in ("sa", "sb"):
                t.fill_(1.0)
            elif name in ("a", "b", "q", "k", "v", "kv"):
                t.fill_(0.5)
    elif inputs != "random":
        raise ValueError(inputs)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(steps):
            fn()
    torch.cuda.synchronize()
    x = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        x @ x
        torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    out.zero_()
    fn()
    torch.cuda.synchronize()
    return us, hashlib.sha256(out.cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def run_variants(kernel: str, variants: list[str], runs: int, inputs: list[str] | None = None) -> str:
    """Time the variants in turn; an exact variant's output is compared, bit
    for bit (SHA-256 of the output tensor), with the kernel as built."""
    spec = KERNELS[kernel]
    if any(variant_exact(kernel, v) for v in variants) and "as_built" not in variants:
        variants = ["as_built", *variants]
    modes = inputs or ["random"]
    res = {(v, m): [] for v in variants for m in modes}
    digest: dict[tuple, set] = {}
    for r in range(runs):
        for v, mode in [(v, m) for v in variants for m in modes]:
            lib = OUT_ROOT / kernel / v / "libmxkernels.so"
            if not lib.exists():
                raise RuntimeError(f"{lib} missing: run the build step first")
            print(f"[alternatives] run {r + 1}/{runs}: {kernel}/{v} ({mode} inputs)", file=sys.stderr, flush=True)
            env = dict(os.environ, MX_KERNELS_LIB=str(lib))
            p = subprocess.run([sys.executable, str(Path(__file__).resolve()), "time", kernel, "--inputs", mode], env=env,
                               capture_output=True, text=True, timeout=300)
            m = re.search(r"^us_per_launch ([\d.]+)$", p.stdout, re.M)
            h = re.search(r"^out_sha256 ([0-9a-f]+)$", p.stdout, re.M)
            if p.returncode != 0 or not m or not h:
                raise RuntimeError(f"{kernel}/{v} failed (rc {p.returncode})\n{p.stdout[-2000:]}\n{p.stderr[-2000:]}")
            res[(v, mode)].append(float(m.group(1)))
            digest.setdefault((v, mode), set()).add(h.group(1))
            print(f"[alternatives] {kernel}/{v} ({mode} inputs): {res[(v, mode)][-1]:.1f} us", file=sys.stderr, flush=True)
    lines = [f"| variant ({spec['workload']}) | µs per launch, run by run | min–max | output |",
             "|---|---|---:|---|"]
    for v, mode in [(v, m) for v in variants for m in modes]:
        t = res[(v, mode)]
        d = 1 if max(t) < 100 else 0  # decimals of the range
        if len(digest[(v, mode)]) != 1:
            out = "differs between runs"
        elif v == "as_built":
            out = "reference"
        else:
            out = "bit-identical" if digest[(v, mode)] == digest.get(("as_built", mode)) else "DIFFERS"
        name = spec["variants"][v][0] + ("" if mode == "random" else f", {mode} inputs")
        lines.append(f"| {name} | {', '.join(f'{x:.1f}' for x in t)} | {min(t):.{d}f}–{max(t):.{d}f} | {out} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("action", choices=["build", "run", "time"])
    ap.add_argument("kernel", choices=sorted(KERNELS))
    ap.add_argument("--variants", default="", help="comma-separated subset (default: all)")
    ap.add_argument("--runs", type=int, default=3)
    ap.add_argument("--inputs", default="random",
                    help="run: comma-separated input modes timed in turn (random, constant); time: one of them")
    args = ap.parse_args()
    variants = [v for v in args.variants.split(",") if v] or list(KERNELS[args.kernel]["variants"])
    for v in variants:
        if v not in KERNELS[args.kernel]["variants"]:
            ap.error(f"unknown variant {v}")
    if args.action == "build":
        build_variants(args.kernel, variants)
    elif args.action == "run":
        print(run_variants(args.kernel, variants, args.runs, args.inputs.split(",")))
    else:
        us, sha = time_one(args.kernel, args.inputs)
        print(f"us_per_launch {us:.3f}\nout_sha256 {sha}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
