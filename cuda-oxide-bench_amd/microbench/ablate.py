"""Where a kernel's time goes: variants of one kernel source with one part
switched off, each built as its own kernel library and timed on the GPU.

    python cuda-oxide-bench_amd/microbench/ablate.py build fp8   # CPU: patch, compile, check, link
    python cuda-oxide-bench_amd/microbench/ablate.py run fp8     # GPU: time every variant, interleaved

build: for each variant, a copy of the kernel source gets the variant's
text patches (each anchor must occur exactly once, so a patch cannot drift
onto other code), is compiled with the library's own flags and linked with
the package's other objects (from its last build) into
microbench/_ablate/<kernel>/<variant>/libmxkernels.so.  Before linking, the
variant's gfx950 assembly goes through the same check as
tests/test_fp8_scale_loads.py: every untracked scale load is landed by its
wait before any instruction names its register; a variant that fails is not
built.

run: each variant's library is loaded in a process of its own
(MX_KERNELS_LIB) and timed like bench.py's graph-replayed cases (warm-up
calls, one graph of 20 launches, replayed after 300 ms of a device GEMM);
the variants take turns, --runs times.  The variants compute wrong results,
which is the point, so nothing checks their output; every variant keeps
every memory access in bounds and every wait count exact, as its
description says.  Unless its description says it removes them, a variant
issues the MFMAs of the kernel as built (a variant whose operands became
equal could let the compiler merge MFMAs and time less work: the
register-operand GQA variant feeds its two key halves from different
registers for that reason).
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
OUT_ROOT = HERE / "_ablate"

# ---------------------------------------------------------------------------
# fp8 block-scaled GEMM (csrc/gemm_fp8_bs.hip), 8192^3.  Patches as
# (anchor, replacement); a variant is the concatenation of its parts.
# ---------------------------------------------------------------------------
FP8_PARTS = {
    # The MFMAs accumulate straight into the accumulators: no fresh partial,
    # no promotion FMAs.  Memory accesses unchanged.
    "promotion": [
        ("        pp = mfma32_fp8(bf0[nf], a0, f32x16{});",
         "        acc[nf][mf] = mfma32_fp8(bf0[nf], a0, acc[nf][mf]); (void)pp;"),
        ("        pp = mfma32_fp8(bf1[nf], a1, pp);",
         "        acc[nf][mf] = mfma32_fp8(bf1[nf], a1, acc[nf][mf]);"),
        ("    auto promote = [&](int nf, int mf) { acc[nf][mf] += s_m[mf] * p[(mf * FN + nf) & 1]; };",
         "    auto promote = [&](int nf, int mf) { (void)nf; (void)mf; (void)p; };"),
    ],
    # The activation-scale loads read one cache line instead of 32: every
    # lane reads row 0's scales (lanes 32-63 the next two blocks, as built).
    # Same instructions and registers as built (a variant that skipped
    # the loads changed the register allocation enough for the compiler to
    # copy an in-flight weight-scale register, which the check refuses).
    "act_scales": [
        ("    sa_off[mf] = (uint32_t)min(m0 + am + 32 * mf, M - 1) * (uint32_t)kblocks * 4u + (GS ? 8u * (lane >> 5) : 0u);",
         "    sa_off[mf] = GS ? 8u * (lane >> 5) : 0u;"),
    ],
    # No tile loads inside the block loop: the prologue's A blocks 0, 1 and B
    # stages 0, 1 are the only ones loaded, the slots of later blocks are
    # read as they are (in bounds).  With no tile loads issued after the
    # scale loads, a wait for all but A_LPW loads would no longer land them,
    # so every block waits for all loads (vmcnt(0)).
    "tile_loads": [
        ("    const int src = min(j, kblocks - 1);\n    dma16(a_tile",
         "    const int src = min(j, kblocks - 1);\n    if (j >= 2) return;\n    dma16(a_tile"),
        ("    const int src = min(s, nst - 1);\n    dma16(b_tile",
         "    const int src = min(s, nst - 1);\n    if (s >= 2) return;\n    dma16(b_tile"),
        ("    wait_scales<CF::A_LPW>(sa_n, sb_n);\n", "    wait_scales<0>(sa_n, sb_n);\n"),
    ],
    # No barrier per block: waves read slots that other waves' loads may be
    # overwriting (wrong values, in bounds).  Waits unchanged.
    "barrier": [
        ("    lds_barrier();\n    float s_m[FM];\n", "    float s_m[FM];\n"),
    ],
}
FP8_VARIANTS = {
    "as_built": ("the kernel as built", []),
    "no_promotion": ("without the promotion (MFMAs accumulate straight into the accumulators)", ["promotion"]),
    "act_scales_one_line": ("activation-scale loads from one cache line (row 0's scales for every row)",
                            ["act_scales"]),
    "no_tile_loads": ("without the tile loads of the block loop (the prologue's two blocks re-read; every "
                      "block waits for all loads)", ["tile_loads"]),
    "no_barrier": ("without the per-block barrier", ["barrier"]),
    "mfma_and_lds_reads": ("no promotion, no tile loads in the loop, no barrier, activation scales from one "
                           "line: the MFMAs, their LDS fragment reads and the scale loads",
                           ["promotion", "act_scales", "tile_loads", "barrier"]),
}

# ---------------------------------------------------------------------------
# Causal GQA forward (csrc/gqa_fwd.hip): B1 Hq32 Hkv8
# S4096 D128 bf16, default tile.  Only the default kernel is launched.
# ---------------------------------------------------------------------------
GQA_PARTS = {
    # Scores go to P as they are (no v_exp_f32); every other instruction,
    # access and wait unchanged.
    "exp2": [
        ("        for (int e = 0; e < 8; ++e) s[qt][0][e] = __builtin_amdgcn_exp2f(s[qt][0][e]);\n",
         "        for (int e = 0; e < 8; ++e) (void)s[qt][0][e];\n"),
        ("            for (int e = 0; e < 8; ++e) s[qt][t1][j1 + e] = __builtin_amdgcn_exp2f(s[qt][t1][j1 + e]);\n",
         "            for (int e = 0; e < 8; ++e) (void)s[qt][t1][j1 + e];\n"),
    ],
    # K and V fragments come from registers (the wave's Q fragments) instead
    # of LDS reads.  The MFMAs still chain on loop-carried accumulators, and
    # the two key halves take different registers so that the compiler does
    # not merge their (then identical) score chains.
    "lds_reads": [
        ("        return lds_ld128(koff[dc] + st + t * 32 * L::ROWK);",
         "        (void)st; return qf[0][(dc + t) % DC];"),
        ("        const uint32_t vb = v_off[dt] + st + (16 * c) * L::ROWV;\n"
         "        const u32x2 lo = lds_read_tr16_at(vb);\n"
         "        const u32x2 hi = lds_read_tr16_at(vb + 8 * L::ROWV);\n"
         "        return u32x4{lo[0], lo[1], hi[0], hi[1]};",
         "        (void)c; return qf[0][dt];"),
    ],
    # Only key tile 0 is loaded (each query block's first); later tiles read
    # the stages as they are (in bounds).  Every tile still waits for all of
    # its wave's loads (vmcnt(0)).
    "kv_loads": [
        ("  auto issue_part = [&](int blk, int n) {\n", "  auto issue_part = [&](int blk, int n) {\n    if (blk >= 1) return;\n"),
        ("  auto issue = [&](int blk) {\n", "  auto issue = [&](int blk) {\n    if (blk >= 1) return;\n"),
    ],
    # No barrier per key tile: waves may read a stage another wave's loads
    # are overwriting (wrong values, in bounds).
    "barrier": [
        ("    __syncthreads();\n    // the next tile's loads go out one per k step",
         "    // the next tile's loads go out one per k step"),
    ],
}
GQA_VARIANTS = {
    "as_built": ("the kernel as built", []),
    "no_exp2": ("without exp2 (scores passed through)", ["exp2"]),
    "no_lds_reads": ("without the K and V fragment reads (register operands)", ["lds_reads"]),
    "no_exp2_lds_reads": ("without both", ["exp2", "lds_reads"]),
    "no_exp2_lds_reads_kv_loads": ("... and without the K/V loads after the first tile", ["exp2", "lds_reads", "kv_loads"]),
    "no_exp2_lds_reads_kv_loads_barrier": ("... and without the per-tile barrier",
                                           ["exp2", "lds_reads", "kv_loads", "barrier"]),
}

# ---------------------------------------------------------------------------
# Absorbed MLA decode (csrc/mla_decode.hip): B32 H128
# T4096, 576/512 bf16, the same buffers every launch; each launch is the
# decode kernel and the split merge.
# ---------------------------------------------------------------------------
MLA_PARTS = {
    # Every stage loads the split's first two stages' cache rows again, so
    # the cache reads after the first two stages come from L2, not HBM.
    # Same loads, slots and waits.
    "l2_loads": [
        ("    issue_part(kvb, t0 + i * BT, t1, lds0", "    issue_part(kvb, t0 + (i & 1) * BT, t1, lds0"),
    ],
    # No direct loads inside the stage loop: the prologue's stages 0 and 1
    # are the only ones loaded, later stages read their slots as they are (in
    # bounds).  The kernel has no untracked register loads, so the waits
    # (now waiting for less) cannot leave a register in flight.
    "loop_loads": [
        ("  scores_alone(0, nblk > 2 ? 2 : -1);", "  scores_alone(0, -1);"),
        ("    f32x16 sc = score_mfma(i, i + 2 < nblk ? i + 2 : -1);", "    f32x16 sc = score_mfma(i, -1);"),
    ],
    # P = s * scale - m instead of exp2 of it (no v_exp_f32).
    "exp2": [
        ("    for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(fmaf(sc[8 * k2 + e], sl2, -m_run));",
         "    for (int e = 0; e < 8; ++e) p[e] = fmaf(sc[8 * k2 + e], sl2, -m_run);"),
    ],
    # No partial-output stores at the end of a split (the merge then reads
    # the workspace as it is, in bounds).  The single-split store path that
    # keeps the accumulators live is unchanged.
    "partial_stores": [
        ("          st64(po + (slot * 64 + lane) * 2, u32x2{pack_bf16x2(a[4 * i] * inv, a[4 * i + 1] * inv),\n"
         "                                                  pack_bf16x2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)});",
         "          (void)po; (void)slot; (void)a; (void)inv;"),
    ],
}
MLA_VARIANTS = {
    "as_built": ("the decode and merge as built", []),
    "l2_loads": ("every stage's cache rows from L2 (all stages reload the split's first 64 tokens)", ["l2_loads"]),
    "no_loop_loads": ("without the direct loads inside the stage loop (stages past the first two read stale "
                      "slots)", ["loop_loads"]),
    "no_exp2": ("without exp2 (P = scaled score minus the running max)", ["exp2"]),
    "no_partial_stores": ("without the partial-output stores at the end of each split", ["partial_stores"]),
}

# ---------------------------------------------------------------------------
# bf16 GEMM 1024^3 (csrc/gemm_bf16.hip, gemm_bf16_sdma_kernel), BASELINE
# what a launch of about one 64x64 tile per CU spends its time
# on.  These variants remove work on purpose (MFMAs included).
# ---------------------------------------------------------------------------
BF16_PARTS = {
    # No MFMAs and no fragment reads: the accumulators stay zero.
    "mfma_reads": [
        ("    compute(kt % CF::NSL);\n", "    (void)compute;\n"),
    ],
    # No tile loads at all (prologue and loop): the slots are read as they
    # are (in bounds); the kernel has no untracked register loads.
    "loads": [
        ("  for (int p = 0; p < CF::NSL - 1; ++p) issue(min(p, nk - 1), p);\n",
         "  for (int p = 0; p < CF::NSL - 1; ++p) (void)p;\n"),
        ("    issue(min(kt + CF::NSL - 1, nk - 1), (kt + CF::NSL - 1) % CF::NSL);\n", "    (void)issue;\n"),
    ],
    # No C stores (the reduction of the two K groups through LDS stays).
    "stores": [
        ("    st64(crow + 8 * i, u32x2{pack_bf16x2(acc[4 * i], acc[4 * i + 1]), "
         "pack_bf16x2(acc[4 * i + 2], acc[4 * i + 3])});",
         "    (void)crow;"),
    ],
    # Every workgroup returns at once.
    "all": [
        ("  using CF = SCfg;\n  extern __shared__ __align__(1024) unsigned char smem[];\n  const int lane = threadIdx.x & 63;\n",
         "  using CF = SCfg;\n  if (M > 0) return;\n  extern __shared__ __align__(1024) unsigned char smem[];\n"
         "  const int lane = threadIdx.x & 63;\n"),
    ],
}
BF16_VARIANTS = {
    "as_built": ("the kernel as built", []),
    "no_mfma_reads": ("without the MFMAs and their fragment reads", ["mfma_reads"]),
    "no_loads": ("without the tile loads", ["loads"]),
    "no_mfma_reads_loads": ("without both", ["mfma_reads", "loads"]),
    "no_mfma_reads_loads_stores": ("... and without the C stores", ["mfma_reads", "loads", "stores"]),
    "return_at_once": ("every workgroup returning at once", ["all"]),
}

KERNELS = {
    "fp8": {"source": "gemm_fp8_bs.hip", "parts": FP8_PARTS, "variants": FP8_VARIANTS,
            "workload": "gemm_fp8_bs M8192 N8192 K8192 e4m3 1x128/128x128 scales",
            "kernel_prefix": "_ZN2mx5gemm818gemm_fp8_bs_kernel"},
    "gqa": {"source": "gqa_fwd.hip", "parts": GQA_PARTS, "variants": GQA_VARIANTS,
            "workload": "gqa_fwd causal B1 Hq32 Hkv8 S4096 D128 bf16, default tile",
            "kernel_prefix": "_ZN2mx3gqa14gqa_fwd_kernel"},
    "bf16_1024": {"source": "gemm_bf16.hip", "parts": BF16_PARTS, "variants": BF16_VARIANTS,
                  "workload": "gemm_bf16 M1024 N1024 K1024 U[-1,1] (gemm_bf16_sdma_kernel)",
                  "kernel_prefix": "_ZN2mx4gemm21gemm_bf16_sdma_kernel"},
    "mla": {"source": "mla_decode.hip", "parts": MLA_PARTS, "variants": MLA_VARIANTS,
            "workload": "mla_decode absorbed B32 H128 T4096 576/512 bf16, decode + merge, same buffers",
            "kernel_prefix": "_ZN2mx3mla17mla_decode_kernel"},
}


def _package_build():
    sys.path.insert(0, str(PKG_DIR))
    import build  # the package's build module (flags, hipcc)

    return build


def patched_source(kernel: str, variant: str) -> str:
    spec = KERNELS[kernel]
    text = (PKG_DIR / "csrc" / spec["source"]).read_text()
    for part in spec["variants"][variant][1]:
        for anchor, repl in spec["parts"][part]:
            n = text.count(anchor)
            if n != 1:
                raise RuntimeError(f"{kernel}/{variant}: patch anchor of part {part!r} occurs {n} times: {anchor!r}")
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


def time_one(kernel: str, steps: int = 20, warmup: int = 3, settle_ms: float = 300.0) -> float:
    """Mean µs per launch of one graph replay (this process's kernel library)."""
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
    elif kernel == "bf16_1024":
        a = (torch.rand((1024, 1024), device="cuda") * 2 - 1).to(torch.bfloat16)
        b = (torch.rand((1024, 1024), device="cuda") * 2 - 1).to(torch.bfloat16)
        out = torch.empty((1024, 1024), dtype=torch.bfloat16, device="cuda")
        fn = lambda: ops.gemm_bf16(a, b, out=out)  # noqa: E731
    elif kernel == "mla":
        gen = torch.Generator(device="cuda").manual_seed(0)
        q = torch.randn((32, 128, 576), device="cuda", generator=gen).to(torch.bfloat16)
        kv = torch.randn((32, 4096, 576), device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty((32, 128, 512), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(max(1, ops.mla_decode_workspace_bytes(32, 128, 4096)), dtype=torch.uint8, device="cuda")
        fn = lambda: ops.mla_decode(q, kv, 192 ** -0.5, out=out, workspace=ws)  # noqa: E731
    else:
        raise ValueError(kernel)
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
    return e0.elapsed_time(e1) * 1e3 / steps


def run_variants(kernel: str, variants: list[str], runs: int) -> str:
    spec = KERNELS[kernel]
    res = {v: [] for v in variants}
    for r in range(runs):
        for v in variants:
            lib = OUT_ROOT / kernel / v / "libmxkernels.so"
            if not lib.exists():
                raise RuntimeError(f"{lib} missing: run the build step first")
            print(f"[ablate] run {r + 1}/{runs}: {kernel}/{v}", file=sys.stderr, flush=True)
            env = dict(os.environ, MX_KERNELS_LIB=str(lib))
            p = subprocess.run([sys.executable, str(Path(__file__).resolve()), "time", kernel], env=env,
                               capture_output=True, text=True, timeout=300)
            m = re.search(r"^us_per_launch ([\d.]+)$", p.stdout, re.M)
            if p.returncode != 0 or not m:
                raise RuntimeError(f"{kernel}/{v} failed (rc {p.returncode})\n{p.stdout[-2000:]}\n{p.stderr[-2000:]}")
            res[v].append(float(m.group(1)))
            print(f"[ablate] {kernel}/{v}: {res[v][-1]:.1f} us", file=sys.stderr, flush=True)
    lines = [f"| variant ({spec['workload']}) | µs per launch, run by run | min–max |", "|---|---|---:|"]
    for v in variants:
        t = res[v]
        d = 1 if max(t) < 100 else 0  # decimals of the range
        lines.append(f"| {spec['variants'][v][0]} | {', '.join(f'{x:.1f}' for x in t)} | {min(t):.{d}f}–{max(t):.{d}f} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("action", choices=["build", "run", "time"])
    ap.add_argument("kernel", choices=sorted(KERNELS))
    ap.add_argument("--variants", default="", help="comma-separated subset (default: all)")
    ap.add_argument("--runs", type=int, default=3)
    args = ap.parse_args()
    variants = [v for v in args.variants.split(",") if v] or list(KERNELS[args.kernel]["variants"])
    for v in variants:
        if v not in KERNELS[args.kernel]["variants"]:
            ap.error(f"unknown variant {v}")
    if args.action == "build":
        build_variants(args.kernel, variants)
    elif args.action == "run":
        print(run_variants(args.kernel, variants, args.runs))
    else:
        print(f"us_per_launch {time_one(args.kernel):.3f}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
