"""fp8 (OCP e4m3) block-scaled GEMM harness cell: gfx950 HIP kernel (mx_gemm_fp8_bs).

The reference's fp8 GEMM (mojo-matmul-fp8/matmul_fp8.mojo) is a single
Mojo program: e4m3 x e4m3 -> f32 at 4096^3, 1 warm-up + 10 timed runs,
median reported, and a correctness check on 1024 cells picked by a Knuth
multiplicative hash with |err| <= 0.2 + 0.1|ref| (:330-361).  This cell
keeps that protocol and the GEMM harness CLI of cutile-matmul-tc-bf16/main.py
(--smoke / --bench / --n / --csv-out, exit 2 on a correctness failure,
results.csv columns impl,kernel,n,iter,gpu_ms,tflops) and adds what this
path specifies: 1x128 (A) / 128x128 (B) fp32 block scales and bf16 output.
Inputs: --dist baseline (N(0,1) quantised per block, the default) or
--dist kat (the reference's exact multiples of 1/16 with unit scales, for
which the result is bit-exact up to the bf16 output rounding).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import importlib  # noqa: E402

H = importlib.import_module("cuda-oxide-bench_amd.harness")

N = 8192
WARMUP = 1
ITERS = 10
NUM_SAMPLES = 1024
ATOL = 2e-1
RTOL = 1e-1


def kat_inputs(n: int):
    """mojo-matmul-fp8/matmul_fp8.mojo:267-270: byte hash % 16 times 1/16."""
    import numpy as np
    import torch

    ia = (np.arange(n * n, dtype=np.uint64) * 2654435761 % 16).reshape(n, n).astype(np.float32) * 0.0625
    ib = ((np.arange(n * n, dtype=np.uint64) + 17) * 2654435761 % 16).reshape(n, n).astype(np.float32) * 0.0625
    a8 = torch.from_numpy(ia).to(torch.float8_e4m3fn)
    b8 = torch.from_numpy(ib).to(torch.float8_e4m3fn)
    sa = torch.ones((n, n // 128), dtype=torch.float32)
    sb = torch.ones((n // 128, (n + 127) // 128), dtype=torch.float32)
    return a8, sa, b8, sb


def make_inputs(n: int, dist: str):
    pkg = H.package()
    if dist == "kat":
        return kat_inputs(n)
    return pkg.inputs.fp8_gemm_inputs(pkg.shapes.FP8GemmShape("cell", n, n, n))


def sample_cells(n: int):
    """The reference's 1024 hashed (row, col) cells (matmul_fp8.mojo:341-344)."""
    out = []
    for s in range(NUM_SAMPLES):
        seed = s * 2654435761
        out.append((((seed >> 20) % n + n) % n, ((seed >> 11) % n + n) % n))
    return out


def run_correctness(n: int, dist: str):
    import numpy as np
    import torch

    ops = H.package().load_ops()
    a8, sa, b8, sb = make_inputs(n, dist)
    c = ops.gemm_fp8_bs(a8.cuda(), sa.cuda(), b8.cuda(), sb.cuda())
    torch.cuda.synchronize()
    cells = sample_cells(n)
    rows = np.array([r for r, _ in cells])
    cols = np.array([c_ for _, c_ in cells])
    got = c[torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()].float().cpu().numpy()
    # dequantised operands, summed in double for the sampled cells
    af = a8[torch.from_numpy(rows)].float() * sa[torch.from_numpy(rows)].repeat_interleave(128, dim=1)
    bcols = b8[:, torch.from_numpy(cols)].float()
    bscale = sb[:, torch.from_numpy(cols // 128)].repeat_interleave(128, dim=0)
    ref = (af.double() * (bcols * bscale).double().t()).sum(dim=1).numpy()
    abs_err = np.abs(got - ref)
    rel_err = abs_err / np.maximum(np.abs(ref), 1e-30)
    n_fail = int((abs_err > ATOL + RTOL * np.abs(ref)).sum())
    exact = None
    if dist == "kat":  # bit-exact: the bf16 rounding of the exact product
        exact = bool(np.array_equal(got, torch.from_numpy(ref.astype(np.float32)).to(torch.bfloat16).float().numpy()))
    return n_fail == 0 and exact is not False, float(abs_err.max()), float(rel_err.max()), n_fail, exact


def run_bench(n: int, dist: str, csv_path: str, iters: int = ITERS) -> dict:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    a8, sa, b8, sb = (t.cuda() for t in make_inputs(n, dist))
    out = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
    flops = 2.0 * n ** 3
    ms = H.time_iters(lambda: ops.gemm_fp8_bs(a8, sa, b8, sb, out=out), WARMUP, iters)
    rows = [["hip", "matmul_fp8_bs", n, i, f"{m:.6f}", f"{flops / 1e12 / (m / 1e3):.6f}"] for i, m in enumerate(ms)]
    H.write_csv(csv_path, ["impl", "kernel", "n", "iter", "gpu_ms", "tflops"], rows)
    st = H.summarize_ms(ms)
    tf_best = flops / 1e12 / (st["best_ms"] / 1e3)
    tf_med = flops / 1e12 / (st["median_ms"] / 1e3)
    H.print_summary(f"fp8 e4m3 block-scaled GEMM N={n}", st, tf_best, tf_med, "TFLOPS", pkg.flops.PEAK_FP8_TFLOPS)
    shape = pkg.shapes.FP8GemmShape("cell", n, n, n)
    H.write_sidecar(csv_path, {"kernel": "matmul_fp8_bs", "n": n, "dist": dist, **st,
                               "tflops_best": tf_best, "tflops_median": tf_med,
                               "peak_tflops": pkg.flops.PEAK_FP8_TFLOPS,
                               "frac_mfma_peak_median": tf_med / pkg.flops.PEAK_FP8_TFLOPS,
                               "algorithmic_bytes": pkg.flops.gemm_fp8_bytes(shape)})
    return st


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False, help="correctness only, default N=512")
    ap.add_argument("--bench", action="store_true", default=False, help="bench at N=8192 (default mode)")
    ap.add_argument("--n", type=int, default=None)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--dist", choices=["baseline", "kat"], default="baseline")
    ap.add_argument("--iters", type=int, default=ITERS, help="timed launches")
    args = ap.parse_args()
    if not args.smoke and not args.bench:
        args.bench = True
    n = args.n if args.n is not None else (512 if args.smoke and not args.bench else N)
    if n % 128:
        print(f"N={n} must be a multiple of 128 (scale block depth)", file=sys.stderr)
        return H.EXIT_CORRECTNESS_FAIL

    H.banner()
    print(f"kernel: mx_gemm_fp8_bs (32x32x64 f8f6f4 MFMA, per-128-K scale promotion)  N={n}")
    print()
    print(f"=== correctness ({NUM_SAMPLES} hashed cells, N={n}, dist={args.dist}) ===")
    ok, mae, mre, n_fail, exact = run_correctness(n, args.dist)
    extra = "" if exact is None else f"  bit-exact={exact}"
    print(f"  max_abs={mae:.4e}  max_rel={mre:.4e}  failed={n_fail}/{NUM_SAMPLES}  atol={ATOL}  rtol={RTOL}{extra}")
    if not ok:
        print("  CORRECTNESS FAIL", file=sys.stderr)
        return H.EXIT_CORRECTNESS_FAIL
    print("  CORRECTNESS OK")
    if args.smoke and not args.bench:
        return H.EXIT_OK
    print()
    run_bench(n, args.dist, args.csv_out, args.iters)
    return H.EXIT_OK


if __name__ == "__main__":
    sys.exit(main())
