"""Benchmark of the quant-inference kernel path on one MI355X.

Headline (the `value` of the JSON line): the fused causal GQA forward at
BASELINE configs[1] — B=1, Hq=32, Hkv=8, S=4096, D=128, bf16, N(0,1)
inputs, scale 1/sqrt(128) — reported in algorithmic TFLOP/s (causal work
2*B*Hq*D*S*(S+1)).  A "step" is one forward pass over that batch with
inputs already resident in HBM.  The other kernels (bf16 GEMM at 1024^3
and 8192^3, fp8 block-scaled GEMM at 8192^3, MLA absorbed decode, GDN
decode, KDA decode at the reference's "large" shape, the fp8 activation
quantiser at 8192x8192, the pre-projected MLA prefill at the reference
cell's bench shape) are measured the same way and reported under "others".

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       [--only-headline]
Prints exactly one JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))

METRIC = "TFLOPS & %MFMA peak (GEMM, GQA fwd); GB/s & %HBM peak (MLA/GDN decode)"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, steps: int, warmup: int):
    """Run fn `warmup` times, then time exactly `steps` back-to-back calls,
    bracketed by torch.cuda.synchronize() and one HIP event pair on the
    current stream (the stream the kernels are launched on).  Returns
    (mean ms per launch from the events, wall ms per step from the host
    clock).  One pair around the whole timed region instead of a pair per
    launch: per-launch event pairs add ~10 us each on ROCm."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall_ms


def cpu_info() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def bench_gqa(pkg, ops, steps, warmup, cpu_baseline: bool):
    import torch

    S, F = pkg.shapes, pkg.flops
    shape = S.GQA_BASELINE
    q, k, v = pkg.inputs.gqa_inputs(shape)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = torch.empty_like(qd)
    fn = lambda: ops.gqa_fwd(qd, kd, vd, causal=True, out=out)  # noqa: E731
    mean_ms, wall_ms = time_launches(fn, steps, warmup)
    flops = F.gqa_causal_flops(shape)
    res = {
        "shape": shape,
        "wall_ms": wall_ms,
        "mean_ms": mean_ms,
        "flops": flops,
        "tflops_mean": F.tflops(flops, mean_ms),
        "tflops_ref_convention_mean": F.tflops(F.gqa_attention_flops(shape), mean_ms),
    }
    if cpu_baseline:
        res["cpu"] = cpu_baseline_gqa(shape, q, k, v, out)
    return res


def cpu_baseline_gqa(shape, q, k, v, out_gpu) -> dict:
    """The oracle (CPU restatement of gqa_naive + causal mask) on a bounded
    sample of the same workload: whole query heads at S=4096, in a fixed
    order, until ~15 s of CPU work or all heads are done.  Also compares the
    GPU output on those heads (a parity spot check on the bench inputs)."""
    import torch

    from oracle import gqa as ogqa
    from oracle.metrics import normwise_rel_err

    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    budget_s = float(os.environ.get("MX_CPU_BASELINE_SECONDS", "15"))
    order = [(7 * i) % shape.n_q for i in range(shape.n_q)]  # 7 is coprime to n_q = 32
    heads, elapsed = [], 0.0
    ogqa.gqa_naive(q, k, v, causal=True, heads=[order[0]])  # warm-up (allocator, threads)
    ref = None
    for h in order:
        t0 = time.perf_counter()
        r = ogqa.gqa_naive(q, k, v, causal=True, heads=[h])
        elapsed += time.perf_counter() - t0
        ref = r if ref is None else ref + r
        heads.append(h)
        if elapsed >= budget_s:
            break
    per_head_flops = 2 * shape.batch * shape.d_head * shape.seq * (shape.seq + 1)
    tfl = per_head_flops * len(heads) / elapsed / 1e12
    got = out_gpu.cpu()
    err = normwise_rel_err(got[:, heads], ref[:, heads])
    return {
        "value": tfl,
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(heads)} of {shape.n_q} query heads (causal, S={shape.seq}, D={shape.d_head}), "
                  f"fp32 torch CPU oracle, {elapsed:.1f} s, {threads} threads on {os.cpu_count()} logical CPUs "
                  f"({cpu_info()})",
        "parity_normwise_on_sample": err,
    }


def bench_others(pkg, ops, steps, warmup) -> dict:
    import torch

    S, F, I = pkg.shapes, pkg.flops, pkg.inputs
    res = {}

    for shape in (S.GEMM_PARITY, S.GEMM_TARGET):
        a, b = I.gemm_inputs(shape)
        ad, bd = a.cuda(), b.cuda()
        c = torch.empty((shape.m, shape.n), dtype=torch.bfloat16, device="cuda")
        ms, _ = time_launches(lambda: ops.gemm_bf16(ad, bd, out=c), steps, warmup)
        fl = F.gemm_flops(shape)
        res[f"gemm_bf16_{shape.m}"] = {
            "unit": "TFLOPS", "mean_ms": ms, "tflops_mean": F.tflops(fl, ms),
            "frac_mfma_peak_mean": F.tflops(fl, ms) / F.PEAK_BF16_TFLOPS,
        }
        del ad, bd, c
        log(f"gemm_bf16 {shape.m}^3: {res[f'gemm_bf16_{shape.m}']['tflops_mean']:.1f} TFLOPS mean")

    shape = S.FP8_TARGET
    a8, sa, b8, sb = I.fp8_gemm_inputs(shape)
    a8d, sad, b8d, sbd = a8.cuda(), sa.cuda(), b8.cuda(), sb.cuda()
    c = torch.empty((shape.m, shape.n), dtype=torch.bfloat16, device="cuda")
    ms, _ = time_launches(lambda: ops.gemm_fp8_bs(a8d, sad, b8d, sbd, out=c), steps, warmup)
    fl = F.gemm_flops(shape)
    res["gemm_fp8_bs_8192"] = {
        "unit": "TFLOPS", "mean_ms": ms, "tflops_mean": F.tflops(fl, ms),
        "frac_mfma_peak_mean": F.tflops(fl, ms) / F.PEAK_FP8_TFLOPS,
    }
    del a8d, sad, b8d, sbd, c
    log(f"gemm_fp8_bs 8192^3: {res['gemm_fp8_bs_8192']['tflops_mean']:.1f} TFLOPS mean")

    shape = S.MLA_BASELINE
    q, kv = I.mla_inputs(shape)
    qd, kvd = q.cuda(), kv.cuda()
    o = torch.empty((shape.batch, shape.n_h, shape.d_latent), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(max(1, ops.mla_decode_workspace_bytes(shape.batch, shape.n_h, shape.ctx)),
                     dtype=torch.uint8, device="cuda")
    ms, _ = time_launches(lambda: ops.mla_decode(qd, kvd, shape.scale, out=o, workspace=ws), steps, warmup)
    nb, fl = F.mla_decode_bytes(shape), F.mla_decode_flops(shape)
    res["mla_decode"] = {
        "unit": "GB/s", "mean_us": ms * 1e3, "gbps_mean": F.gbps(nb, ms),
        "frac_hbm_peak_mean": F.gbps(nb, ms) / F.PEAK_HBM_GBPS, "tflops_mean": F.tflops(fl, ms),
    }
    log(f"mla_decode: {res['mla_decode']['gbps_mean']:.0f} GB/s mean")
    # the whole absorbed step: q_nope W_UK -> latent decode -> o_lat W_UV
    x = {n: t.cuda() for n, t in I.mla_projection_inputs(shape).items()}
    od = torch.empty((shape.batch, shape.n_h, 128), dtype=torch.bfloat16, device="cuda")
    wsa = torch.empty(ops.mla_decode_absorbed_workspace_bytes(shape.batch, shape.n_h, shape.ctx) + 256,
                      dtype=torch.uint8, device="cuda")
    ms, _ = time_launches(lambda: ops.mla_decode_absorbed(x["q_nope"], x["q_rope"], kvd, x["w_uk"], x["w_uv"],
                                                          shape.scale, out=od, workspace=wsa), steps, warmup)
    nb2 = nb + sum(x[n].numel() * 2 for n in ("w_uk", "w_uv", "q_nope", "q_rope")) + od.numel() * 2
    res["mla_decode_absorbed_step"] = {
        "unit": "GB/s", "mean_us": ms * 1e3, "gbps_mean": F.gbps(nb2, ms),
        "note": "one mx_mla_decode_absorbed call: absorb + latent decode + combine + up-projection",
    }
    del qd, kvd, o, ws, x, od, wsa
    log(f"mla_decode_absorbed_step: {res['mla_decode_absorbed_step']['mean_us']:.1f} us mean")

    shape = S.GDN_BASELINE
    x = {n: t.cuda() for n, t in I.gdn_inputs(shape).items()}
    so = torch.empty_like(x["S_in"])
    od = torch.empty((shape.batch, shape.n_heads, shape.d_v), dtype=torch.bfloat16, device="cuda")
    ms, _ = time_launches(lambda: ops.gdn_decode(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"],
                                                 S_out=so, o=od), steps, warmup)
    nb = F.gdn_decode_bytes(shape)
    res["gdn_decode"] = {
        "unit": "GB/s", "mean_us": ms * 1e3, "gbps_mean": F.gbps(nb, ms),
        "frac_hbm_peak_mean": F.gbps(nb, ms) / F.PEAK_HBM_GBPS,
    }
    log(f"gdn_decode: {res['gdn_decode']['gbps_mean']:.0f} GB/s mean")
    del x, so, od

    shape = S.KDA_LARGE
    x = {n: t.cuda() for n, t in I.kda_inputs(shape).items()}
    so = torch.empty_like(x["S_in"])
    od = torch.empty((shape.batch, shape.n_heads, shape.d_v), dtype=torch.float16, device="cuda")
    ms, _ = time_launches(lambda: ops.kda_decode(x["q"], x["k"], x["v"], x["g"], x["beta"], x["S_in"],
                                                 S_out=so, o=od), steps, warmup)
    nb = F.kda_decode_bytes(shape)
    res["kda_decode"] = {
        "unit": "GB/s", "shape": f"B{shape.batch} H{shape.n_heads} d{shape.d_k}", "mean_us": ms * 1e3,
        "gbps_mean": F.gbps(nb, ms), "frac_hbm_peak_mean": F.gbps(nb, ms) / F.PEAK_HBM_GBPS,
    }
    log(f"kda_decode: {res['kda_decode']['gbps_mean']:.0f} GB/s mean")
    del x, so, od

    m = k = 8192
    xa = torch.randn((m, k), generator=torch.Generator().manual_seed(I.SEED)).to(torch.bfloat16).cuda()
    qa = torch.empty((m, k), dtype=torch.float8_e4m3fn, device="cuda")
    sa_ = torch.empty((m, k // 128), dtype=torch.float32, device="cuda")
    ms, _ = time_launches(lambda: ops.quant_fp8_act(xa, q=qa, scales=sa_), steps, warmup)
    nb = F.quant_fp8_act_bytes(m, k)
    res["quant_fp8_act"] = {
        "unit": "GB/s", "shape": f"{m}x{k} bf16 -> e4m3 + 1x128 scales", "mean_us": ms * 1e3,
        "gbps_mean": F.gbps(nb, ms), "frac_hbm_peak_mean": F.gbps(nb, ms) / F.PEAK_HBM_GBPS,
    }
    log(f"quant_fp8_act: {res['quant_fp8_act']['gbps_mean']:.0f} GB/s mean")
    del xa, qa, sa_

    # pre-projected MLA prefill at the reference cell's bench shape (qk 192, v 128, native)
    shape = S.MLA_PREFILL_BENCH
    q, k, v = (t.cuda() for t in I.mla_prefill_inputs(shape, dtype=torch.bfloat16))
    o = torch.empty((shape.batch, shape.n_h, shape.seq, shape.d_v), dtype=torch.bfloat16, device="cuda")
    ms, _ = time_launches(lambda: ops.mla_prefill_fwd(q, k, v, out=o), steps, warmup)
    fl = F.mla_attention_flops(shape)
    res["mla_prefill"] = {
        "unit": "TFLOPS", "shape": f"B{shape.batch} S{shape.seq} H{shape.n_h} qk{shape.qk_head_dim} v{shape.d_v} bf16",
        "mean_ms": ms, "tflops_mean": F.tflops(fl, ms), "frac_mfma_peak_mean": F.tflops(fl, ms) / F.PEAK_BF16_TFLOPS,
    }
    log(f"mla_prefill: {res['mla_prefill']['tflops_mean']:.1f} TFLOPS mean")
    return res


def calibrate_copy(steps: int) -> int:
    """A plain device-to-device copy of a known size (1 GiB read + 1 GiB
    written per launch), for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE
    readings of the kernels above to bytes."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read_per_launch": n, "bytes_written_per_launch": n,
                      "launches": steps}), flush=True)
    return 0


def load_traffic(workload: str):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated), if it covers this workload."""
    p = REPO_ROOT / "profiles" / "gqa_fwd_causal_s4096_traffic.json"
    try:
        d = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload:
        return None
    return d.get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 1 GiB device copy (profiler calibration of byte counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every kernel is single-device; sharding is described in DESIGN.md). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch

    if args.calibrate_copy:
        return calibrate_copy(args.steps)
    pkg = importlib.import_module("cuda-oxide-bench_amd")
    ops = pkg.load_ops()
    F = pkg.flops
    log(f"device: {torch.cuda.get_device_name(0)}")

    g = bench_gqa(pkg, ops, args.steps, args.warmup, cpu_baseline=not args.no_cpu_baseline)
    shape = g["shape"]
    log(f"gqa_fwd causal S{shape.seq}: mean {g['mean_ms']:.4f} ms  {g['tflops_mean']:.1f} TFLOPS")
    others = {} if args.only_headline else bench_others(pkg, ops, args.steps, args.warmup)

    workload = (f"gqa_fwd causal B{shape.batch} Hq{shape.n_q} Hkv{shape.n_kv} S{shape.seq} "
                f"D{shape.d_head} bf16")
    achieved = g["tflops_mean"]
    traffic = load_traffic(workload)
    line = {
        "metric": METRIC,
        "value": round(F.tflops(g["flops"], g["wall_ms"]), 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, seed 0xC0FFEE)",
        "config": {
            "workload": workload,
            "batch": shape.batch, "seq": shape.seq, "n_q": shape.n_q, "n_kv": shape.n_kv,
            "d_head": shape.d_head, "causal": True, "softmax_scale": shape.d_head ** -0.5,
            "flops_per_step": g["flops"], "flops_convention": "causal algorithmic 2*B*Hq*D*S*(S+1)",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": F.PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / F.PEAK_BF16_TFLOPS, 5),
            "traffic": traffic,
            "kernel": "gqa_fwd_kernel<128, 128, BF16, causal, 1>",
            "launch_mean_ms": round(g["mean_ms"], 5),
        },
        "cpu_baseline": g.get("cpu"),
        "tflops_reference_convention": round(g["tflops_ref_convention_mean"], 3),
        "others": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
