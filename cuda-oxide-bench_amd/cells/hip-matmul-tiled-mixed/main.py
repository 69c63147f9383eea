"""Mixed-dtype GEMM harness cell, bf16 row: gfx950 HIP kernel (mx_gemm_bf16).

Drop-in for cutile-matmul-tiled-mixed/main.py: the same flags (--smoke,
the default; --bench; --export-cubins; --n, default 512; --csv-out;
--cubin-dir), the same variant names (VARIANTS, :121-130), inputs
(PCG64 seed 0xC0FFEE, U[0,1) drawn as fp32 then rounded, A then B,
:138-150), per-variant relative gate max|out-ref|/max|ref| < tol (bf16
3e-2, :66 and :172-178), bench sweep N in [1024, 2048, 4096] with 1
warm-up + 10 timed launches (:55-61, :195-283), results.csv columns
(impl,kernel,n,iter,gpu_ms,tflops) and smoke exit codes (0 every built
variant passed, 1 some failed, 2 all failed; :368-381).

Only the bf16 row (mma_bf16xbf16_f32acc: bf16 in, fp32 accumulate, bf16
out) is on this path; the f16, tf32 and f32 rows are listed, reported as
not built here and left out of the pass/fail count.  The reference for the
check is the fp32 product of the rounded inputs (this repository's oracle
restatement), not a bf16 library matmul.  --iters overrides the timed
launch count.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import importlib  # noqa: E402

H = importlib.import_module("cuda-oxide-bench_amd.harness")

CORRECTNESS_N = 512
BENCH_SIZES = [1024, 2048, 4096]
WARMUP = 1
ITERS = 10
TOL_F16, TOL_BF16, TOL_TF32, TOL_F32 = 1e-2, 3e-2, 1e-3, 1e-3

# (variant name, built on this path, relative tolerance) in the reference's order
VARIANTS = [
    ("mma_f16xf16_f32acc", False, TOL_F16),
    ("mma_bf16xbf16_f32acc", True, TOL_BF16),
    ("mma_tf32xtf32_f32acc", False, TOL_TF32),
    ("mma_f32xf32_f32acc", False, TOL_F32),
]
NOT_BUILT = "not on this path (only the bf16 row of the mixed-dtype harness is built for gfx950)"


def make_inputs(n: int):
    """A, B [n, n] bf16 from PCG64(0xC0FFEE) U[0,1) fp32, A drawn first."""
    pkg = H.package()
    a, b = pkg.inputs.gemm_inputs(pkg.shapes.GemmShape("mixed", n, n, n), seed=0xC0FFEE, dist="reference")
    return a, b


def run_correctness(n: int) -> dict:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    results = {}
    for name, built, tol in VARIANTS:
        if not built:
            results[name] = (None, float("nan"), NOT_BUILT)
            print(f"[{name}] N={n} SKIP {NOT_BUILT}")
            continue
        a, b = make_inputs(n)
        out = ops.gemm_bf16(a.cuda(), b.cuda())
        torch.cuda.synchronize()
        ref = a.float() @ b.float()
        max_err = float((out.float().cpu() - ref).abs().max())
        rel = max_err / max(float(ref.abs().max()), 1e-6)
        ok = rel < tol
        results[name] = (ok, rel, "")
        print(f"[{name}] N={n} tol={tol:.0e}  max_abs={max_err:.3e} rel={rel:.3e}  {'OK' if ok else 'FAIL'}")
    return results


def run_bench(csv_path: str, iters: int, sizes=BENCH_SIZES) -> None:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    rows, summary = [], []
    for n in sizes:
        flops = 2.0 * n ** 3
        for name, built, _tol in VARIANTS:
            if not built:
                print(f"[hip-{name}] N={n} SKIP {NOT_BUILT}")
                continue
            a, b = (t.cuda() for t in make_inputs(n))
            out = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
            ms = H.time_iters(lambda: ops.gemm_bf16(a, b, out=out), WARMUP, iters)
            for i, m in enumerate(ms):
                tf = flops / 1e12 / (m / 1e3)
                print(f"[hip-{name}] N={n} iter={i} gpu_ms={m:.3f} tflops={tf:.3f}")
                rows.append(["hip", name, n, i, f"{m:.6f}", f"{tf:.6f}"])
            med = sorted(ms)[len(ms) // 2]
            summary.append((n, name, med, flops / 1e12 / (med / 1e3)))
            del a, b, out
    H.write_csv(csv_path, ["impl", "kernel", "n", "iter", "gpu_ms", "tflops"], rows)
    print()
    print("=" * 72)
    print(" BENCH SUMMARY — median of", iters, "iters")
    print("=" * 72)
    print(f"  {'N':>5}  {'variant':<28}  {'ms':>9}  {'TFLOPS':>8}")
    for n, name, ms, tf in summary:
        print(f"  {n:>5}  {name:<28}  {ms:>9.3f}  {tf:>8.3f}")
    H.write_sidecar(csv_path, {"kernel": "mma_bf16xbf16_f32acc (mx_gemm_bf16)",
                               "peak_tflops": pkg.flops.PEAK_BF16_TFLOPS,
                               "medians": [{"n": n, "variant": v, "ms": ms, "tflops": tf,
                                            "frac_mfma_peak": tf / pkg.flops.PEAK_BF16_TFLOPS}
                                           for n, v, ms, tf in summary]})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=True, help="correctness check only (default)")
    ap.add_argument("--bench", action="store_true", default=False, help="run timed sweep")
    ap.add_argument("--export-cubins", action="store_true", default=False)
    ap.add_argument("--n", type=int, default=CORRECTNESS_N, help="size for correctness check")
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--cubin-dir", default=".")
    ap.add_argument("--iters", type=int, default=ITERS, help="timed launches per (N, variant)")
    args = ap.parse_args()

    H.banner()
    print("bf16 row: mx_gemm_bf16 (bf16 MFMA kernels chosen by shape, fp32 accumulate, bf16 out)")
    print()
    if args.export_cubins:
        lib = importlib.import_module("cuda-oxide-bench_amd._lib")
        print(f"gfx950 code objects are embedded in {lib.lib_path()} (built in-tree); no cubins exist on this "
              f"target, nothing written to {args.cubin_dir}")
        print()
    if args.bench:
        print(f"Running correctness first at N={args.n}…")
        run_correctness(args.n)
        print()
        print(f"Running bench sweep {BENCH_SIZES} ({WARMUP} warm + {args.iters} iters)…")
        run_bench(args.csv_out, args.iters)
        return H.EXIT_OK

    results = run_correctness(args.n)
    print()
    print("=" * 48)
    built = {k: r for k, r in results.items() if r[0] is not None}
    all_ok = all(r[0] for r in built.values())
    any_ok = any(r[0] for r in built.values())
    for k, (ok, rel, err) in results.items():
        label = "SKIP" if ok is None else ("PASS" if ok else "FAIL")
        tail = f"  rel={rel:.3e}" if err == "" else f"  {err}"
        print(f"  {k}: {label}{tail}")
    print("=" * 48)
    if all_ok:
        print(f"SMOKE TEST OK ({len(built)} of {len(results)} variants built)")
        return 0
    if any_ok:
        print("SMOKE TEST PARTIAL — some variant(s) failed")
        return 1
    print("SMOKE TEST FAILED — all variants failed")
    return 2


if __name__ == "__main__":
    sys.exit(main())
