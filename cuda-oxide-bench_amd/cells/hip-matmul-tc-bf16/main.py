"""bf16 GEMM harness cell: hand-written gfx950 HIP kernel (mx_gemm_bf16).

Drop-in for cutile-matmul-tc-bf16/main.py: same flags (--smoke, --bench,
--n, --csv-out), same defaults (bench at N=4096, 5 warm-up + 50 timed
launches, 200 sampled cells checked against an f32 CPU dot product with
|err| <= 0.2 + 0.05|ref|, exit code 2 on a correctness failure), same
results.csv columns (impl,kernel,n,iter,gpu_ms,tflops).  Extra flags:
--dist {reference,baseline} (U[0,1) PCG64 inputs as the reference, or
U[-1,1]) and --sweep (N in 1024, 2048, 4096, 8192 as
cutile-matmul-tiled-mixed/main.py:55-60 sweeps).  A roofline.json sidecar
reports the rate against the MI355X bf16 MFMA peak.
"""
from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import importlib  # noqa: E402

H = importlib.import_module("cuda-oxide-bench_amd.harness")

N = 4096
WARMUP = 5
ITERS = 50
NUM_SAMPLES = 200
ATOL = 2e-1
RTOL = 5e-2
SWEEP = [1024, 2048, 4096, 8192]


def make_inputs(n: int, dist: str):
    pkg = H.package()
    a, b = pkg.inputs.gemm_inputs(pkg.shapes.GemmShape("cell", n, n, n), dist=dist)
    return a.cuda(), b.cuda(), a, b


def sample_reference(a, b, rows, cols):
    """f32 dot products of the bf16 inputs for the sampled cells (the
    reference harness's inline check, cutile-matmul-tc-bf16/main.py:98-107)."""
    import numpy as np

    a32, b32 = a.float().numpy(), b.float().numpy()
    return np.array([np.dot(a32[r, :], b32[:, c]) for r, c in zip(rows, cols)], dtype=np.float32)


def run_correctness(n: int, dist: str):
    import numpy as np
    import torch

    ops = H.package().load_ops()
    a, b, a_h, b_h = make_inputs(n, dist)
    out = ops.gemm_bf16(a, b)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0xBEEF)
    rows = rng.integers(0, n, size=NUM_SAMPLES)
    cols = rng.integers(0, n, size=NUM_SAMPLES)
    got = out[torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()].float().cpu().numpy()
    refs = sample_reference(a_h, b_h, rows, cols)
    abs_err = np.abs(got - refs)
    rel_err = abs_err / np.maximum(np.abs(refs), 1e-6)
    n_fail = int((abs_err > ATOL + RTOL * np.abs(refs)).sum())
    return n_fail == 0, float(abs_err.max()), float(rel_err.max()), n_fail


def run_bench(sizes: list[int], dist: str, csv_path: str, iters: int = ITERS) -> dict:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    rows, summaries = [], {}
    for n in sizes:
        a, b, _, _ = make_inputs(n, dist)
        out = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
        flops = 2.0 * n ** 3
        t0 = time.perf_counter()
        ms = H.time_iters(lambda: ops.gemm_bf16(a, b, out=out), WARMUP, iters)
        wall = time.perf_counter() - t0
        for i, m in enumerate(ms):
            rows.append(["hip", "matmul_tc_bf16", n, i, f"{m:.6f}", f"{flops / 1e12 / (m / 1e3):.6f}"])
        st = H.summarize_ms(ms)
        tf_best = flops / 1e12 / (st["best_ms"] / 1e3)
        tf_med = flops / 1e12 / (st["median_ms"] / 1e3)
        H.print_summary(f"bf16 GEMM N={n}", st, tf_best, tf_med, "TFLOPS", pkg.flops.PEAK_BF16_TFLOPS)
        print(f"  CPU wall: {wall:.3f} s for {WARMUP + iters} timed and warm-up samples")
        summaries[str(n)] = {**st, "tflops_best": tf_best, "tflops_median": tf_med,
                             "frac_mfma_peak_median": tf_med / pkg.flops.PEAK_BF16_TFLOPS}
        del a, b, out
    H.write_csv(csv_path, ["impl", "kernel", "n", "iter", "gpu_ms", "tflops"], rows)
    H.write_sidecar(csv_path, {"kernel": "matmul_tc_bf16", "peak_tflops": pkg.flops.PEAK_BF16_TFLOPS,
                               "dist": dist, "sizes": summaries})
    return summaries


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False, help="correctness check only, default N=512")
    ap.add_argument("--bench", action="store_true", default=False, help="full bench at N=4096 (default mode)")
    ap.add_argument("--n", type=int, default=None)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--dist", choices=["reference", "baseline"], default="reference")
    ap.add_argument("--sweep", action="store_true", help="bench N in 1024, 2048, 4096, 8192")
    ap.add_argument("--iters", type=int, default=ITERS, help="timed launches (default 50)")
    args = ap.parse_args()
    if not args.smoke and not args.bench:
        args.bench = True
    n = args.n if args.n is not None else (512 if args.smoke and not args.bench else N)

    H.banner()
    print(f"kernel: mx_gemm_bf16 (32x32x16 bf16 MFMA)  N={n}  ITERS={args.iters}")
    print()
    print(f"=== correctness (sampled, N={n}) ===")
    ok, mae, mre, n_fail = run_correctness(n, args.dist)
    print(f"  max_abs={mae:.4e}  max_rel={mre:.4e}  failed={n_fail}/{NUM_SAMPLES}  atol={ATOL}  rtol={RTOL}")
    if not ok:
        print("  CORRECTNESS FAIL", file=sys.stderr)
        return H.EXIT_CORRECTNESS_FAIL
    print("  CORRECTNESS OK")
    if args.smoke and not args.bench:
        return H.EXIT_OK
    print()
    run_bench(SWEEP if args.sweep else [n], args.dist, args.csv_out, args.iters)
    return H.EXIT_OK


if __name__ == "__main__":
    sys.exit(main())
