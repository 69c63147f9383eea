"""KDA decode harness cell: gfx950 HIP Kimi-Delta-Attention decode (mx_kda_decode).

Drop-in for cutile-attn-kda/main.py (+ its bench.py --shape): flags --smoke
(default), --bench, --csv-out, --shape {registry} (default
kimi_linear_decode, as bench.py), --export-cubin / --cubin-out (accepted),
--inputs-dir / --fixture (replay a kda_<fixture>_*.npy set written in the
reference's inputs/ layout instead of the committed golden set).
--smoke runs the reference's SHAPE_CORRECTNESS (B1 H2 d64, f16, the
reference's seed-17 recipe) against the committed golden oracle output with
the reference's gate (max_abs <= 1e-3 or rel <= 1e-3 on o and S,
main.py:374-380) and this path's normwise bounds (o 2e-2, S 1e-3).  --bench
uses 2 warm-up + 50 timed launches and writes results.csv with the
reference columns (impl,kernel,batch,n_heads,d_k,d_v,block_v,iter,gpu_us,
gbps,tflops) plus dtype,frac_hbm at the end, and a roofline.json sidecar.
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
    fixture set in the reference's inputs/ layout (kda_<fixture>_*.npy:
    f16 q/k/v/g/beta, f32 S_in, f16 o and f32 S_out expected;
    gen_kda_inputs.py:40-60)."""
    import numpy as np
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    if inputs_dir:
        fx = H.reference_fixtures(inputs_dir, "kda", fixture)
        x = [torch.from_numpy(fx[n]).cuda() for n in ("q", "k", "v", "g", "beta")]
        s_in = torch.from_numpy(fx["S_in"]).cuda()
        g = {"o": fx["o_expected"].astype(np.float32), "S_out": fx["S_out_expected"]}
        print(f"[smoke] fixture={fixture} B={x[0].shape[0]} H={x[0].shape[1]} d_k={x[0].shape[2]} d_v={x[2].shape[2]}")
    else:
        s = pkg.shapes.KDA_CORRECTNESS
        print(f"[smoke] shape={s.name} B={s.batch} H={s.n_heads} d_k={s.d_k} d_v={s.d_v}")
        g = H.load_golden("kda_correctness_f16")
        x = [H.from_bits(g[n], torch.float16).cuda() for n in ("q", "k", "v", "g", "beta")]
        s_in = torch.from_numpy(g["S_in"]).cuda()
    o, so = ops.kda_decode(*x, s_in)
    torch.cuda.synchronize()
    ok = True
    for name, got, want, bound in (("o", o.float().cpu().numpy(), g["o"], pkg.tolerances.NORMWISE_OUTPUT),
                                   ("S_out", so.cpu().numpy(), g["S_out"], pkg.tolerances.NORMWISE_STATE)):
        mx = float(np.abs(got - want).max())
        rel = mx / (float(np.abs(want).max()) + 1e-30)
        good = (mx <= 1e-3 or rel <= 1e-3) and rel <= bound
        ok = ok and good
        print(f"[smoke] {name:5s} max_abs={mx:.3e} rel={rel:.3e}  {'OK' if good else 'FAIL'}")
    return ok


def run_bench(shape, csv_path: str, iters: int = ITERS) -> None:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    x = {n: t.cuda() for n, t in pkg.inputs.kda_inputs(shape).items()}
    print(f"[bench] shape={shape.name} B={shape.batch} H={shape.n_heads} d_k={shape.d_k} d_v={shape.d_v} "
          f"dtype=f16")
    so = torch.empty_like(x["S_in"])
    o = torch.empty((shape.batch, shape.n_heads, shape.d_v), dtype=torch.float16, device="cuda")
    nb, fl = F.kda_decode_bytes(shape), F.kda_decode_flops(shape)
    print(f"[bench] flops/iter = {fl / 1e6:.3f} MFLOPS   bytes/iter = {nb / 1024:.1f} KB")
    ms = H.time_iters(lambda: ops.kda_decode(x["q"], x["k"], x["v"], x["g"], x["beta"], x["S_in"],
                                             S_out=so, o=o), WARMUP, iters)
    bv = ops.gdn_block_v(shape.batch, shape.n_heads, shape.d_k, shape.d_v)
    rows = []
    for i, m in enumerate(ms):
        if i < 3 or i == iters - 1:
            print(f"[bench] iter={i:2d} gpu_us={m * 1e3:.2f} gbps={F.gbps(nb, m):.1f} tflops={F.tflops(fl, m):.3f}")
        rows.append(["hip", "kda_decode_fused", shape.batch, shape.n_heads, shape.d_k, shape.d_v, bv, i,
                     f"{m * 1e3:.3f}", f"{F.gbps(nb, m):.3f}", f"{F.tflops(fl, m):.6f}", "f16",
                     f"{F.gbps(nb, m) / F.PEAK_HBM_GBPS:.5f}"])
    H.write_csv(csv_path, ["impl", "kernel", "batch", "n_heads", "d_k", "d_v", "block_v", "iter", "gpu_us", "gbps",
                           "tflops", "dtype", "frac_hbm"], rows)
    st = H.summarize_ms(ms)
    H.print_summary(f"{shape.name} (HBM-bound)", st, F.gbps(nb, st["best_ms"]), F.gbps(nb, st["median_ms"]),
                    "GB/s", F.PEAK_HBM_GBPS)
    H.write_sidecar(csv_path, {"kernel": "kda_decode_fused", "shape": shape.name, **st, "bytes": nb,
                               "gbps_median": F.gbps(nb, st["median_ms"]), "peak_gbps": F.PEAK_HBM_GBPS,
                               "frac_hbm_peak_median": F.gbps(nb, st["median_ms"]) / F.PEAK_HBM_GBPS})


def main() -> int:
    pkg = H.package()
    reg = pkg.shapes.KDA_REGISTRY
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False)
    ap.add_argument("--bench", action="store_true", default=False)
    ap.add_argument("--export-cubin", action="store_true", default=False)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--cubin-out", default="kda_decode_fused.cubin")
    ap.add_argument("--shape", default="kimi_linear_decode", choices=sorted(reg.keys()))
    ap.add_argument("--iters", type=int, default=ITERS, help="timed launches (default 50)")
    ap.add_argument("--inputs-dir", default=None,
                    help="replay a fixture set written in the reference's inputs/ layout")
    ap.add_argument("--fixture", default="correctness", help="fixture shape name (kda_<fixture>_*.npy)")
    args = ap.parse_args()
    if not (args.smoke or args.bench or args.export_cubin):
        args.smoke = True
    H.banner()
    print()
    rc = H.EXIT_OK
    if args.smoke:
        if not run_smoke(args.inputs_dir, args.fixture):
            rc = H.EXIT_SMOKE_FAIL
        print()
    if args.bench:
        run_bench(reg[args.shape], args.csv_out, args.iters)
        print()
    if args.export_cubin:
        lib = importlib.import_module("cuda-oxide-bench_amd._lib")
        print(f"gfx950 code objects are embedded in {lib.lib_path()}; no cubin exists on this target")
    return rc


if __name__ == "__main__":
    sys.exit(main())
