"""MLA harness cell: gfx950 HIP absorbed latent-cache decode (mx_mla_decode).

Keeps the CLI of cutile-attn-mla/main.py (--smoke default, --bench,
--csv-out, --export-cubin / --cubin-out accepted) and its results.csv
columns (impl,kernel,batch,seq,n_h,qk_head_dim,qk_pad,d_v,block_m,block_n,
iter,gpu_ms,tflops) with gpu_us,gbps,frac_hbm,n_split appended.  The
kernel is the weight-absorbed decode form of the reference's MLA attention
(one query token per sequence over a 576-wide latent cache, values = the
first 512 latent columns, scale 1/sqrt(192)), so in the CSV `seq` is the
context length T, `qk_head_dim` / `qk_pad` are the 576-wide latent dot
product (no padding) and `d_v` is 512.  --smoke checks the committed
golden oracle output (H16, T40) with the bf16 normwise bound 2e-2;
--bench times B32 H128 T4096 (DeepSeek-V3 shape) with 2 warm-up + 10
timed launches.  GB/s counts the latent cache read once plus Q and O.
--batch / --ctx (not in the reference CLI) replace B and T of the bench
shape, e.g. B1 T32768 for a long-context single sequence.

--mode prefill runs the reference cell's own kernel instead: pre-projected
multi-head attention over q/k of qk_head_dim and v of d_v
(mx_mla_prefill_fwd, cutile-attn-mla/main.py:81-163) with qk_head_dim used
natively, so qk_pad = qk_head_dim in the CSV.  --smoke checks the
reference's SHAPE_CORRECTNESS_MLA (1,128,4, qk 96, v 64, f16) against the
committed golden output with the reference's f16 allclose gate
(:259-266), or with --inputs-dir / --fixture a mla_<fixture>_*.npy set in
the reference's inputs/ layout; --bench times SHAPE_BENCH_MLA
(deepseek_v3: B1 S2048 H128, qk 192, v 128) with 2 warm-up + 10 timed
launches, TFLOPS by the reference's formula 2*B*H*S^2*(qk+d_v)
(flops_mla.py:32-45); causal and dtype columns are appended.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import importlib  # noqa: E402

H = importlib.import_module("cuda-oxide-bench_amd.harness")

WARMUP = 2
ITERS = 10
TOL = 2e-2


def run_smoke() -> bool:
    import numpy as np
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    g = H.load_golden("mla_decode_h16_t40")
    q, kv = H.from_bits(g["q"], torch.bfloat16).cuda(), H.from_bits(g["kv"], torch.bfloat16).cuda()
    print(f"[smoke] absorbed decode B={q.shape[0]} H={q.shape[1]} T={kv.shape[1]} d_qk={q.shape[2]} d_v=512")
    o = ops.mla_decode(q, kv, float(g["scale"][0]))
    torch.cuda.synchronize()
    o32 = o.float().cpu().numpy()
    err = np.abs(o32 - g["o"])
    rel = float(err.max() / (np.abs(g["o"]).max() + 1e-30))
    ok = rel <= TOL
    print(f"[smoke] max_abs={float(err.max()):.3e} rel={rel:.3e}  bound={TOL}  {'OK' if ok else 'FAIL'}")
    return ok


def run_bench(csv_path: str, iters: int, batch: int | None = None, ctx: int | None = None) -> None:
    import dataclasses

    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    s = pkg.shapes.MLA_BASELINE
    if batch is not None or ctx is not None:
        s = dataclasses.replace(s, name="custom", batch=batch or s.batch, ctx=ctx or s.ctx)
    print(f"[bench] shape={s.name} B={s.batch} H={s.n_h} T={s.ctx} d_qk={s.d_qk} d_v={s.d_latent}")
    q, kv = (t.cuda() for t in pkg.inputs.mla_inputs(s))
    out = torch.empty((s.batch, s.n_h, s.d_latent), dtype=torch.bfloat16, device="cuda")
    ws_bytes = ops.mla_decode_workspace_bytes(s.batch, s.n_h, s.ctx)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    n_split = ops.mla_decode_splits(s.batch, s.n_h, s.ctx)
    ms = H.time_iters(lambda: ops.mla_decode(q, kv, s.scale, out=out, workspace=ws), WARMUP, iters)
    fl, nb = F.mla_decode_flops(s), F.mla_decode_bytes(s)
    rows = []
    for i, m in enumerate(ms):
        print(f"[bench] iter={i} gpu_us={m * 1e3:.2f} gbps={F.gbps(nb, m):.1f} tflops={F.tflops(fl, m):.3f}")
        rows.append(["hip", "mla_decode_absorbed", s.batch, s.ctx, s.n_h, s.d_qk, s.d_qk, s.d_latent, 64, 32, i,
                     f"{m:.6f}", f"{F.tflops(fl, m):.6f}", f"{m * 1e3:.3f}", f"{F.gbps(nb, m):.3f}",
                     f"{F.gbps(nb, m) / F.PEAK_HBM_GBPS:.5f}", n_split])
    H.write_csv(csv_path, ["impl", "kernel", "batch", "seq", "n_h", "qk_head_dim", "qk_pad", "d_v", "block_m",
                           "block_n", "iter", "gpu_ms", "tflops", "gpu_us", "gbps", "frac_hbm", "n_split"], rows)
    st = H.summarize_ms(ms)
    H.print_summary(f"{s.name} (HBM-bound)", st, F.gbps(nb, st["best_ms"]), F.gbps(nb, st["median_ms"]), "GB/s",
                    F.PEAK_HBM_GBPS)
    H.write_sidecar(csv_path, {"kernel": "mla_decode_absorbed", "shape": s.name, **st, "bytes": nb, "flops": fl,
                               "gbps_median": F.gbps(nb, st["median_ms"]), "peak_gbps": F.PEAK_HBM_GBPS,
                               "frac_hbm_peak_median": F.gbps(nb, st["median_ms"]) / F.PEAK_HBM_GBPS,
                               "tflops_median": F.tflops(fl, st["median_ms"]), "n_split": n_split})


def run_prefill_smoke(inputs_dir: str | None, fixture: str) -> bool:
    import numpy as np
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    if inputs_dir:
        fx = H.reference_fixtures(inputs_dir, "mla", fixture)
        q, k, v = (torch.from_numpy(fx[x]).cuda() for x in "qkv")
        expected = fx["expected"]
    else:
        g = H.load_golden("mla_prefill_correctness_f16")
        q, k, v = (H.from_bits(g[x], torch.float16).cuda() for x in "qkv")
        expected = g["o"]
    print(f"[smoke] prefill B={q.shape[0]} S={q.shape[2]} n_h={q.shape[1]} qk_head_dim={q.shape[3]} d_v={v.shape[3]}")
    o = ops.mla_prefill_fwd(q, k, v)
    torch.cuda.synchronize()
    o32 = o.float().cpu().numpy()
    tol = pkg.tolerances.get("f16")
    err = np.abs(o32 - expected)
    rel = float(err.max() / (np.abs(expected).max() + 1e-30))
    ok = bool(np.allclose(o32, expected, atol=tol.atol, rtol=tol.rtol))
    print(f"[smoke] max_abs={float(err.max()):.3e} rel={rel:.3e}  atol={tol.atol} rtol={tol.rtol}  "
          f"{'OK' if ok else 'FAIL'}")
    return ok


def run_prefill_bench(csv_path: str, iters: int, causal: bool, dtype_name: str) -> None:
    import dataclasses

    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    s = dataclasses.replace(pkg.shapes.MLA_PREFILL_BENCH, causal=causal)
    dt = torch.bfloat16 if dtype_name == "bf16" else torch.float16
    print(f"[bench] prefill shape={s.name} B={s.batch} S={s.seq} n_h={s.n_h} qk={s.qk_head_dim} d_v={s.d_v} "
          f"causal={causal} dtype={dtype_name}")
    q, k, v = (t.cuda() for t in pkg.inputs.mla_prefill_inputs(s, dtype=dt))
    out = torch.empty((s.batch, s.n_h, s.seq, s.d_v), dtype=dt, device="cuda")
    ms = H.time_iters(lambda: ops.mla_prefill_fwd(q, k, v, causal=causal, out=out), WARMUP, iters)
    conv, alg = F.mla_attention_flops(s), F.mla_algorithmic_flops(s)
    rows = []
    for i, m in enumerate(ms):
        print(f"[bench] iter={i} gpu_ms={m:.3f} tflops={F.tflops(conv, m):.3f}")
        rows.append(["hip", "mla_fwd_fused", s.batch, s.seq, s.n_h, s.qk_head_dim, s.qk_head_dim, s.d_v, 32, 64, i,
                     f"{m:.6f}", f"{F.tflops(conv, m):.6f}", int(causal), dtype_name, f"{F.tflops(alg, m):.6f}"])
    H.write_csv(csv_path, ["impl", "kernel", "batch", "seq", "n_h", "qk_head_dim", "qk_pad", "d_v", "block_m",
                           "block_n", "iter", "gpu_ms", "tflops", "causal", "dtype", "tflops_algorithmic"], rows)
    st = H.summarize_ms(ms)
    H.print_summary(f"{s.name} prefill (algorithmic FLOPs)", st, F.tflops(alg, st["best_ms"]),
                    F.tflops(alg, st["median_ms"]), "TFLOPS", F.PEAK_BF16_TFLOPS)
    H.write_sidecar(csv_path, {"kernel": "mla_fwd_fused", "shape": s.name, "causal": causal, "dtype": dtype_name,
                               **st, "flops_algorithmic": alg, "flops_reference_convention": conv,
                               "tflops_algorithmic_median": F.tflops(alg, st["median_ms"]),
                               "peak_tflops": F.PEAK_BF16_TFLOPS,
                               "frac_mfma_peak_median": F.tflops(alg, st["median_ms"]) / F.PEAK_BF16_TFLOPS,
                               "bytes": F.mla_attention_bytes(s)})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False)
    ap.add_argument("--bench", action="store_true", default=False)
    ap.add_argument("--export-cubin", action="store_true", default=False)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--cubin-out", default="mla_fwd_fused.cubin")
    ap.add_argument("--iters", type=int, default=None)
    ap.add_argument("--mode", choices=["decode", "prefill"], default="decode",
                    help="decode: absorbed latent-cache decode (the measured path); prefill: the reference "
                         "cell's pre-projected attention with native qk_head_dim")
    ap.add_argument("--causal", action="store_true", default=False, help="prefill: causal mask")
    ap.add_argument("--dtype", choices=["f16", "bf16"], default="f16", help="prefill: I/O dtype")
    ap.add_argument("--inputs-dir", default=None,
                    help="prefill: replay a fixture set written in the reference's inputs/ layout")
    ap.add_argument("--fixture", default="correctness_mla", help="prefill fixture shape name (mla_<fixture>_*.npy)")
    ap.add_argument("--batch", type=int, default=None, help="decode --bench: batch size (default 32)")
    ap.add_argument("--ctx", type=int, default=None, help="decode --bench: context length T (default 4096)")
    args = ap.parse_args()
    if not (args.smoke or args.bench or args.export_cubin):
        args.smoke = True
    H.banner()
    print()
    rc = H.EXIT_OK
    iters = args.iters if args.iters is not None else ITERS
    if args.smoke:
        ok = run_prefill_smoke(args.inputs_dir, args.fixture) if args.mode == "prefill" else run_smoke()
        if not ok:
            rc = H.EXIT_SMOKE_FAIL
        print()
    if args.bench:
        if args.mode == "prefill":
            run_prefill_bench(args.csv_out, iters, args.causal, args.dtype)
        else:
            run_bench(args.csv_out, iters, args.batch, args.ctx)
        print()
    if args.export_cubin:
        lib = importlib.import_module("cuda-oxide-bench_amd._lib")
        print(f"gfx950 code objects are embedded in {lib.lib_path()}; no cubin exists on this target")
    return rc


if __name__ == "__main__":
    sys.exit(main())
