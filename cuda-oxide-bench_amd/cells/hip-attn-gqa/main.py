"""Fused GQA forward harness cell: gfx950 HIP flash-attention kernel (mx_gqa_fwd).

Drop-in for cutile-attn-gqa/main.py: flags --smoke (default), --bench,
--csv-out, --block-m, --block-n, --iters (and --export-cubin / --cubin-out,
accepted; gfx950 code objects are produced by the in-tree build, so the
flag prints where the library is).  --smoke checks the reference's
SHAPE_CORRECTNESS (1,128,4,2,64), f16, reference-distribution inputs
against the committed golden oracle output with the reference's f16
allclose gate (atol = rtol = 5e-3, :258-265); --bench times SHAPE_BENCH
(llama3_8b, B1 S2048 Hq32 Hkv8 D128) with 2 warm-up + 10 timed launches
and writes results.csv with the reference columns
(impl,kernel,batch,seq,n_q,n_kv,d_head,block_m,block_n,iter,gpu_ms,tflops)
plus, at the end, causal,dtype,tflops_causal.  Extra flags select the
configuration this path is measured on: --shape baseline (S4096, causal,
bf16, N(0,1) inputs), --causal, --dtype.  TFLOPS uses the reference's
convention (4*B*Hq*S^2*D, flops.py:31-47); tflops_causal the causal
algorithmic count 2*B*Hq*D*S*(S+1).

Tile overrides keep the reference's pick_blocks semantics
(cutile-attn-gqa/main.py:202-230): --block-m and --block-n must divide the
sequence (checked by assertion) and select the tile the gfx950 kernel runs
(mx_gqa_fwd_tile): BLOCK_M query rows of each head per workgroup, BLOCK_N
keys per LDS stage.  BLOCK_N is the kernels' 64-key stage; an unset
--block-n takes 64 (the reference defaults it to BLOCK_M, and its own
BLOCK_M sweep holds it at 64, sweep_block_m.py).  BLOCK_M sets how many
heads of a KV group a workgroup covers (hpw = workgroup rows / BLOCK_M):
64, 128 and 256 at the bench shape's G = 4, 64 (4-wave kernel), 128 and 256
at the correctness shape's G = 2.  --wave-m (added) picks the queries per
wave: 32 (two waves per SIMD, default) or 64 (one wave per SIMD).  A tile no
kernel has fails the pick_blocks assertion, as an untileable shape does in
the reference.  Without overrides the default tile runs at any seq (ragged
tiles are masked).  The tile in use is what results.csv reports;
sweep_block_m.py in this directory runs the reference's BLOCK_M sweep.
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
BLOCK_N = 64  # keys per LDS stage


def kernel_tile(n_q: int, n_kv: int, d_head: int = 128) -> tuple[int, int]:
    """(BLOCK_M, BLOCK_N) of the default tile: 8 waves of 32 queries over
    hpw = 4, 2 or 1 heads of a KV group (mx_gqa_fwd_default_block_m)."""
    ops = H.package().load_ops()
    return ops.gqa_default_block_m(n_q, n_kv, d_head), BLOCK_N


def pick_blocks(seq: int, n_q: int, n_kv: int, block_m_override: int | None = None,
                block_n_override: int | None = None, d_head: int = 128, wave_m: int = 32):
    """(BLOCK_M, BLOCK_N) for a sequence length, with the reference's override
    semantics (cutile-attn-gqa/main.py:202-230): an override must divide seq
    (an unset BLOCK_M is 64; an unset BLOCK_N is the kernels' 64-key stage)
    and must be a tile the library has a kernel for at this head grouping.
    Without overrides the default tile runs at any seq."""
    if block_m_override is not None or block_n_override is not None or wave_m != 32:
        bm = block_m_override if block_m_override is not None else 64
        bn = block_n_override if block_n_override is not None else BLOCK_N
        assert seq % bm == 0, f"BLOCK_M={bm} does not divide seq={seq}"
        assert seq % bn == 0, f"BLOCK_N={bn} does not divide seq={seq}"
        ops = H.package().load_ops()
        assert ops.gqa_tile_supported(n_q, n_kv, d_head, bm, bn, wave_m), (
            f"no gfx950 GQA kernel has BLOCK_M={bm} BLOCK_N={bn} wave_m={wave_m} at n_q={n_q} n_kv={n_kv} "
            f"d={d_head} (BLOCK_N is the 64-key stage; a workgroup's rows must cover a whole number of heads "
            f"dividing the group size)")
        return bm, bn
    return kernel_tile(n_q, n_kv, d_head)


def run_smoke(inputs_dir: str | None = None, fixture: str = "correctness", block_m: int | None = None,
              block_n: int | None = None, wave_m: int = 32) -> bool:
    """The correctness check: the committed golden set, or with inputs_dir a
    fixture set in the reference's inputs/ layout (gqa_<fixture>_*.npy,
    f16 inputs, f32 expected output; cutile-attn-gqa/main.py:177-183)."""
    import numpy as np
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    if inputs_dir:
        fx = H.reference_fixtures(inputs_dir, "gqa", fixture)
        q, k, v = (torch.from_numpy(fx[x]).cuda() for x in "qkv")
        expected = fx["expected"]
        print(f"[smoke] fixture={fixture} B={q.shape[0]} S={q.shape[2]} n_q={q.shape[1]} n_kv={k.shape[1]} "
              f"d={q.shape[3]}")
    else:
        s = pkg.shapes.GQA_CORRECTNESS
        print(f"[smoke] shape={s.name} B={s.batch} S={s.seq} n_q={s.n_q} n_kv={s.n_kv} d={s.d_head}")
        g = H.load_golden("gqa_correctness_f16")
        q, k, v = (H.from_bits(g[x], torch.float16).cuda() for x in "qkv")
        expected = g["o"]
    bm, bn = pick_blocks(q.shape[2], q.shape[1], k.shape[1], block_m, block_n, q.shape[3], wave_m)
    print(f"[smoke] BLOCK_M={bm} BLOCK_N={bn} wave_m={wave_m}")
    o = ops.gqa_fwd(q, k, v, causal=False, block_m=bm, block_n=bn, wave_m=wave_m)
    torch.cuda.synchronize()
    o32 = o.float().cpu().numpy()
    tol = pkg.tolerances.get("f16")
    abs_err = np.abs(o32 - expected)
    max_abs = float(abs_err.max())
    rel = max_abs / (np.abs(expected).max() + 1e-30)
    ok = bool(np.allclose(o32, expected, atol=tol.atol, rtol=tol.rtol))
    print(f"[smoke] max_abs={max_abs:.3e} rel={rel:.3e}  atol={tol.atol} rtol={tol.rtol}  {'OK' if ok else 'FAIL'}")
    if not ok:
        worst = np.unravel_index(abs_err.argmax(), abs_err.shape)
        print(f"        worst offender at {worst}: got={o32[worst]:.4f} expected={expected[worst]:.4f}")
    return ok


def run_bench(shape, dtype, dist, csv_path: str, iters: int, block_m: int | None = None,
              block_n: int | None = None, wave_m: int = 32) -> None:
    import torch

    pkg = H.package()
    ops = pkg.load_ops()
    F = pkg.flops
    print(f"[bench] shape={shape.name} B={shape.batch} S={shape.seq} n_q={shape.n_q} n_kv={shape.n_kv} "
          f"d={shape.d_head} causal={shape.causal} dtype={dtype}")
    bm, bn = pick_blocks(shape.seq, shape.n_q, shape.n_kv, block_m, block_n, shape.d_head, wave_m)
    print(f"[bench] BLOCK_M={bm} BLOCK_N={bn} wave_m={wave_m}")
    q, k, v = (t.cuda() for t in pkg.inputs.gqa_inputs(shape, dtype=dtype, dist=dist))
    out = torch.empty_like(q)
    ms = H.time_iters(lambda: ops.gqa_fwd(q, k, v, causal=shape.causal, out=out, block_m=bm, block_n=bn,
                                          wave_m=wave_m), WARMUP, iters)
    conv = F.gqa_attention_flops(shape)
    alg = F.gqa_algorithmic_flops(shape)
    dname = "bf16" if dtype == torch.bfloat16 else "f16"
    rows = []
    for i, m in enumerate(ms):
        print(f"[bench] iter={i} gpu_ms={m:.3f} tflops={F.tflops(conv, m):.3f}")
        rows.append(["hip", "gqa_fwd_fused", shape.batch, shape.seq, shape.n_q, shape.n_kv, shape.d_head, bm,
                     bn, i, f"{m:.6f}", f"{F.tflops(conv, m):.6f}", int(shape.causal), dname,
                     f"{F.tflops(alg, m):.6f}", wave_m])
    H.write_csv(csv_path, ["impl", "kernel", "batch", "seq", "n_q", "n_kv", "d_head", "block_m", "block_n", "iter",
                           "gpu_ms", "tflops", "causal", "dtype", "tflops_causal", "wave_m"], rows)
    st = H.summarize_ms(ms)
    H.print_summary(f"{shape.name} (algorithmic {'causal' if shape.causal else 'full'} FLOPs)", st,
                    F.tflops(alg, st["best_ms"]), F.tflops(alg, st["median_ms"]), "TFLOPS", F.PEAK_BF16_TFLOPS)
    H.write_sidecar(csv_path, {"kernel": "gqa_fwd_fused", "shape": shape.name, "causal": shape.causal,
                               "dtype": dname, "block_m": bm, "block_n": bn, "wave_m": wave_m,
                               **st, "flops_algorithmic": alg, "flops_reference_convention": conv,
                               "tflops_algorithmic_median": F.tflops(alg, st["median_ms"]),
                               "peak_tflops": F.PEAK_BF16_TFLOPS,
                               "frac_mfma_peak_median": F.tflops(alg, st["median_ms"]) / F.PEAK_BF16_TFLOPS,
                               "bytes": F.gqa_attention_bytes(shape)})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--smoke", action="store_true", default=False)
    ap.add_argument("--bench", action="store_true", default=False)
    ap.add_argument("--export-cubin", action="store_true", default=False)
    ap.add_argument("--csv-out", default="results.csv")
    ap.add_argument("--cubin-out", default="gqa_fwd_fused.cubin")
    ap.add_argument("--block-m", type=int, default=None)
    ap.add_argument("--block-n", type=int, default=None)
    ap.add_argument("--iters", type=int, default=None)
    ap.add_argument("--wave-m", type=int, choices=[32, 64], default=32,
                    help="query rows per wave: 32 (two waves per SIMD) or 64 (one wave per SIMD)")
    ap.add_argument("--shape", choices=["llama3_8b", "baseline"], default="llama3_8b")
    ap.add_argument("--causal", action="store_true", default=None)
    ap.add_argument("--dtype", choices=["f16", "bf16"], default=None)
    ap.add_argument("--inputs-dir", default=None,
                    help="replay a fixture set written in the reference's inputs/ layout")
    ap.add_argument("--fixture", default="correctness", help="fixture shape name (gqa_<fixture>_*.npy)")
    args = ap.parse_args()
    if not (args.smoke or args.bench or args.export_cubin):
        args.smoke = True

    import dataclasses

    import torch

    H.banner()
    if args.block_m is not None or args.block_n is not None or args.wave_m != 32:
        print(f"[tile] override: BLOCK_M={args.block_m} BLOCK_N={args.block_n} wave_m={args.wave_m}")
    print()
    rc = H.EXIT_OK
    if args.smoke:
        if not run_smoke(args.inputs_dir, args.fixture, args.block_m, args.block_n, args.wave_m):
            rc = H.EXIT_SMOKE_FAIL
        print()
    if args.bench:
        pkg = H.package()
        if args.shape == "baseline":
            shape, dtype, dist = pkg.shapes.GQA_BASELINE, torch.bfloat16, "baseline"
        else:
            shape, dtype, dist = pkg.shapes.GQA_LLAMA3_8B, torch.float16, "reference"
        if args.causal is not None:
            shape = dataclasses.replace(shape, causal=True)
        if args.dtype is not None:
            dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
        run_bench(shape, dtype, dist, args.csv_out, args.iters if args.iters is not None else ITERS, args.block_m,
                  args.block_n, args.wave_m)
        print()
    if args.export_cubin:
        lib = importlib.import_module("cuda-oxide-bench_amd._lib")
        print(f"gfx950 code objects are embedded in {lib.lib_path()} (built in-tree by build.py); "
              f"no cubin exists on this target")
    return rc


if __name__ == "__main__":
    sys.exit(main())
