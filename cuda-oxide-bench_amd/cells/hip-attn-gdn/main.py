"""GDN decode harness cell: gfx950 HIP gated-delta-rule decode (mx_gdn_decode).

Drop-in for cutile-attn-gdn/main.py: flags --smoke (default), --bench,
--csv-out, --shape {registry} (default qwen3_next_decode), --export-cubin /
--cubin-out (accepted), --inputs-dir / --fixture (replay a
gdn_<fixture>_*.npy set written in the reference's inputs/ layout).  --smoke runs the reference's SHAPE_CORRECTNESS
(B2 H4 d64, f16, reference inputs) against the committed golden oracle
output with the reference's gates (o: f16 allclose 5e-3; S: max_abs < 5e-3
or rel < 5e-3, :283-298) and this path's normwise bounds (o 2e-2, S 1e-3).
--bench uses 2 warm-up + 50 timed launches and writes results.csv with
the reference columns (impl,kernel,batch,n_heads,d_k,d_v,block_v,iter,
gpu_us,gbps,tflops) plus n_k_heads,dtype,frac_hbm at the end.  The
registry adds qwen3_next_b64 (B64, Hk16, Hv32, d128, bf16, exp(-softplus)
/ sigmoid gates), the configuration this path is measured on.
--sweep times the reference sweep's shapes (qwen3_next_decode, tiny, small,
large, wide; only --shape's when --shape is given) with --warmup/--iters
(2/50) and writes results_sweep.csv (or --sweep-csv) with the columns of
cuda-attn-gdn-tma/bench_sweep.cu:314-315 (impl,kernel,shape,batch,n_heads,
d_k,d_v,block_v,n_blocks,iter,gpu_ms,gbps,gflops).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import importlib  # noqa: E402

H = importlib.import_module("cuda-oxide-bench_amd.harness")

WARMUP = 2
ITERS = 50


def run_smoke(inputs_dir: str | None = None, fixture: str = "correctness") -> bool:
    """The correctness check: the committed golden set, or with inputs_dir a
    fixture set in the reference's inputs/ layout (gdn_<fixture>_*.npy:
    f16 q/k/v/alpha/beta, f32 S_in, f16 o and f32 S_out expected;
    cutile-attn-gdn/main.py:193-204)."""
    import numpy as np
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    if inputs_dir:
        fx = H.reference_fixtures(inputs_dir, "gdn", fixture)
        args = [torch.from_numpy(fx[n]).cuda() for n in ("q", "k", "v")]
        # gates are f16 on disk; the kernel takes them as fp32 (exact widening)
        args += [torch.from_numpy(fx[n].astype(np.float32)).cuda() for n in ("alpha", "beta")]
        args += [torch.from_numpy(fx["S_in"]).cuda()]
        g = {"o": fx["o_expected"].astype(np.float32), "S_out": fx["S_out_expected"]}
        print(f"[smoke] fixture={fixture} B={args[0].shape[0]} H={args[0].shape[1]} d_k={args[0].shape[2]} "
              f"d_v={args[2].shape[2]}")
    else:
        s = pkg.shapes.GDN_CORRECTNESS
        print(f"[smoke] shape={s.name} B={s.batch} H={s.n_heads} d_k={s.d_k} d_v={s.d_v}")
        g = H.load_golden("gdn_correctness_f16")
        dt = torch.float16
        args = [H.from_bits(g[n], dt).cuda() for n in ("q", "k", "v")]
        args += [torch.from_numpy(g[n]).cuda() for n in ("alpha", "beta", "S_in")]
    o, so = ops.gdn_decode(*args)
    torch.cuda.synchronize()
    o32, s32 = o.float().cpu().numpy(), so.cpu().numpy()
    tol = pkg.tolerances.get("f16")
    ok_o = bool(np.allclose(o32, g["o"], atol=tol.atol, rtol=tol.rtol))
    max_o = float(np.abs(o32 - g["o"]).max())
    rel_o = max_o / (float(np.abs(g["o"]).max()) + 1e-30)
    max_s = float(np.abs(s32 - g["S_out"]).max())
    rel_s = max_s / (float(np.abs(g["S_out"]).max()) + 1e-30)
    ok_s = (max_s < 5e-3 or rel_s < 5e-3) and rel_s <= pkg.tolerances.NORMWISE_STATE
    ok_o = ok_o and rel_o <= pkg.tolerances.NORMWISE_OUTPUT
    print(f"[smoke] o    max_abs={max_o:.3e} rel={rel_o:.3e}  {'OK' if ok_o else 'FAIL'}")
    print(f"[smoke] S_out max_abs={max_s:.3e} rel={rel_s:.3e}  {'OK' if ok_s else 'FAIL'}")
    return ok_o and ok_s


def run_bench(shape, csv_path: str, iters: int = ITERS) -> None:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    baseline = shape.n_k_heads is not None
    dt = torch.bfloat16 if baseline else torch.float16
    x = {n: t.cuda() for n, t in pkg.inputs.gdn_inputs(shape, dtype=dt,
                                                        dist="baseline" if baseline else "reference").items()}
    print(f"[bench] shape={shape.name} B={shape.batch} H={shape.n_heads} Hk={shape.hk} d_k={shape.d_k} "
          f"d_v={shape.d_v} dtype={dt}")
    so = torch.empty_like(x["S_in"])
    o = torch.empty((shape.batch, shape.n_heads, shape.d_v), dtype=dt, device="cuda")
    nb, fl = F.gdn_decode_bytes(shape), F.gdn_decode_flops(shape)
    print(f"[bench] flops/iter = {fl / 1e6:.3f} MFLOPS   bytes/iter = {nb / 1024:.1f} KB")
    ms = H.time_iters(lambda: ops.gdn_decode(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"],
                                             S_out=so, o=o), WARMUP, iters)
    bv = ops.gdn_block_v(shape.batch, shape.n_heads, shape.d_k, shape.d_v)
    dname = "bf16" if dt == torch.bfloat16 else "f16"
    rows = []
    for i, m in enumerate(ms):
        if i < 3 or i == iters - 1:
            print(f"[bench] iter={i:2d} gpu_us={m * 1e3:.2f} gbps={F.gbps(nb, m):.1f} tflops={F.tflops(fl, m):.3f}")
        rows.append(["hip", "gdn_decode_fused", shape.batch, shape.n_heads, shape.d_k, shape.d_v, bv, i,
                     f"{m * 1e3:.3f}", f"{F.gbps(nb, m):.3f}", f"{F.tflops(fl, m):.6f}", shape.hk, dname,
                     f"{F.gbps(nb, m) / F.PEAK_HBM_GBPS:.5f}"])
    H.write_csv(csv_path, ["impl", "kernel", "batch", "n_heads", "d_k", "d_v", "block_v", "iter", "gpu_us", "gbps",
                           "tflops", "n_k_heads", "dtype", "frac_hbm"], rows)
    st = H.summarize_ms(ms)
    H.print_summary(f"{shape.name} (HBM-bound)", st, F.gbps(nb, st["best_ms"]), F.gbps(nb, st["median_ms"]),
                    "GB/s", F.PEAK_HBM_GBPS)
    H.write_sidecar(csv_path, {"kernel": "gdn_decode_fused", "shape": shape.name, **st, "bytes": nb,
                               "gbps_median": F.gbps(nb, st["median_ms"]), "peak_gbps": F.PEAK_HBM_GBPS,
                               "frac_hbm_peak_median": F.gbps(nb, st["median_ms"]) / F.PEAK_HBM_GBPS})


SWEEP_HEADER = ["impl", "kernel", "shape", "batch", "n_heads", "d_k", "d_v", "block_v", "n_blocks", "iter",
                "gpu_ms", "gbps", "gflops"]


def run_sweep(names, csv_path: str, warmup: int, iters: int) -> None:
    """The reference sweep (cuda-attn-gdn-tma/bench_sweep.cu:302-380): every
    shape on its reference-distribution f16 inputs, one CSV row per (shape,
    iteration), then a best-of summary table."""
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    reg = pkg.shapes.GDN_REGISTRY
    rows, summary = [], []
    for name in names:
        shape = reg[name]
        x = {n: t.cuda() for n, t in pkg.inputs.gdn_inputs(shape, dtype=torch.float16, dist="reference").items()}
        so = torch.empty_like(x["S_in"])
        o = torch.empty((shape.batch, shape.n_heads, shape.d_v), dtype=torch.float16, device="cuda")
        bv = ops.gdn_block_v(shape.batch, shape.n_heads, shape.d_k, shape.d_v)
        nblk = shape.batch * shape.n_heads * (shape.d_v // bv)
        print(f"[sweep] ===== shape={name} B={shape.batch} H={shape.n_heads} d_k={shape.d_k} d_v={shape.d_v}  "
              f"BV={bv}  n_blocks={nblk} =====")
        ms = H.time_iters(lambda: ops.gdn_decode(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"],
                                                 S_out=so, o=o), warmup, iters)
        nb, fl = F.gdn_decode_bytes(shape), F.gdn_decode_flops(shape)
        for i, m in enumerate(ms):
            rows.append(["hip", "gdn_decode_fused", name, shape.batch, shape.n_heads, shape.d_k, shape.d_v, bv, nblk, i,
                         f"{m:.6f}", f"{F.gbps(nb, m):.3f}", f"{fl / (m * 1e-3) / 1e9:.3f}"])
        best = min(ms)
        summary.append((name, shape, nblk, best * 1e3, F.gbps(nb, best), fl / (best * 1e-3) / 1e9))
        del x, so, o
    H.write_csv(csv_path, SWEEP_HEADER, rows)
    print()
    print(f"{'shape':20s} {'(B,H,d_k,d_v)':22s} {'n_blocks':9s} {'best_us':9s} {'best_gbps':9s} {'best_gf':7s}")
    for name, sh, nblk, us, gb, gf in summary:
        shp = f"({sh.batch},{sh.n_heads},{sh.d_k},{sh.d_v})"
        print(f"{name:20s} {shp:22s} {nblk:<9d} {us:<9.2f} {gb:<9.1f} {gf:<7.2f}")
    print(f"[sweep] CSV: {csv_path}  (one row per (shape, iter))")


def main() -> int:
    pkg = H.package()
    reg = pkg.shapes.GDN_REGISTRY
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False)
    ap.add_argument("--bench", action="store_true", default=False)
    ap.add_argument("--export-cubin", action="store_true", default=False)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--cubin-out", default="gdn_decode_fused.cubin")
    ap.add_argument("--shape", default=None, choices=sorted(reg.keys()),
                    help="bench shape (default qwen3_next_decode); with --sweep, only this shape")
    ap.add_argument("--sweep", action="store_true", default=False)
    ap.add_argument("--sweep-csv", default="results_sweep.csv")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--inputs-dir", default=None,
                    help="replay a fixture set written in the reference's inputs/ layout")
    ap.add_argument("--fixture", default="correctness", help="fixture shape name (gdn_<fixture>_*.npy)")
    args = ap.parse_args()
    if not (args.smoke or args.bench or args.export_cubin or args.sweep):
        args.smoke = True
    H.banner()
    print()
    rc = H.EXIT_OK
    if args.smoke:
        if not run_smoke(args.inputs_dir, args.fixture):
            rc = H.EXIT_SMOKE_FAIL
        print()
    if args.bench:
        run_bench(reg[args.shape or "qwen3_next_decode"], args.csv_out, args.iters)
        print()
    if args.sweep:
        run_sweep([args.shape] if args.shape else list(pkg.shapes.GDN_SWEEP), args.sweep_csv, args.warmup,
                  args.iters)
        print()
    if args.export_cubin:
        lib = importlib.import_module("cuda-oxide-bench_amd._lib")
        print(f"gfx950 code objects are embedded in {lib.lib_path()}; no cubin exists on this target")
    return rc


if __name__ == "__main__":
    sys.exit(main())
