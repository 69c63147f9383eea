"""Aggregate the harness cells' results.csv files into one master table.

The reference keeps one long-format table of every timed iteration
(results/scaling.csv:1, columns impl,kernel,N,iter,gpu_ms,cpu_wall_ms,
tflops) and a per-configuration summary with best / median / p95 / IQR /
CV% (results/scaling-summary.md).  Its per-cell CSVs differ in their
configuration columns (GEMM: n; GQA: batch,seq,n_q,n_kv,d_head,...; GDN:
gpu_us and gbps instead of gpu_ms and tflops), so the master table keeps
the common measurement columns and folds every configuration column into
one `config` key:

  cell,impl,kernel,config,iter,gpu_ms,rate,unit

`rate` is the cell's headline rate (TFLOPS where the cell reports
`tflops`, GB/s where it reports `gbps`, which the decode cells lead
with).  The summary groups by (cell, impl, kernel, config).

Usage: python collect_results.py --out master.csv [--summary summary.md] CSV...
       (a CSV's cell name is its parent directory's name)
"""
from __future__ import annotations

import argparse
import csv
import statistics
import sys
from pathlib import Path

MEASURE_COLS = {"iter", "gpu_ms", "gpu_us", "tflops", "gbps", "cpu_wall_ms"}
MASTER_HEADER = ["cell", "impl", "kernel", "config", "iter", "gpu_ms", "rate", "unit"]


def read_cell_csv(path: str | Path) -> list[dict]:
    """Rows of one cell CSV in the master schema."""
    path = Path(path)
    with open(path, newline="") as f:
        reader = csv.DictReader(f)
        cols = reader.fieldnames or []
        missing = [c for c in ("impl", "kernel", "iter") if c not in cols]
        if missing:
            raise ValueError(f"{path}: not a results.csv (missing {', '.join(missing)})")
        if "gpu_ms" not in cols and "gpu_us" not in cols:
            raise ValueError(f"{path}: no gpu_ms or gpu_us column")
        if "gbps" in cols:
            rate_col, unit = "gbps", "GB/s"
        elif "tflops" in cols:
            rate_col, unit = "tflops", "TFLOPS"
        else:
            rate_col, unit = None, ""
        cfg_cols = [c for c in cols if c not in MEASURE_COLS and c not in ("impl", "kernel")]
        rows = []
        for r in reader:
            ms = float(r["gpu_ms"]) if "gpu_ms" in cols else float(r["gpu_us"]) / 1e3
            rows.append({
                "cell": path.parent.name or path.stem,
                "impl": r["impl"],
                "kernel": r["kernel"],
                "config": ";".join(f"{c}={r[c]}" for c in cfg_cols),
                "iter": int(r["iter"]),
                "gpu_ms": ms,
                "rate": float(r[rate_col]) if rate_col else float("nan"),
                "unit": unit,
            })
    return rows


def summarize(rows: list[dict]) -> list[dict]:
    """best / median / p95 / IQR / CV% of gpu_ms and the median rate per configuration."""
    groups: dict[tuple, list[dict]] = {}
    for r in rows:
        groups.setdefault((r["cell"], r["impl"], r["kernel"], r["config"]), []).append(r)
    out = []
    for (cell, impl, kernel, config), rs in groups.items():
        ms = sorted(r["gpu_ms"] for r in rs)
        n = len(ms)
        q = statistics.quantiles(ms, n=4, method="inclusive") if n >= 2 else [ms[0]] * 3
        p95 = ms[min(n - 1, int(round(0.95 * (n - 1))))]
        mean = statistics.fmean(ms)
        cv = (statistics.stdev(ms) / mean * 100.0) if n >= 2 and mean > 0 else 0.0
        out.append({
            "cell": cell, "impl": impl, "kernel": kernel, "config": config, "n": n,
            "best_ms": ms[0], "median_ms": statistics.median(ms), "p95_ms": p95, "iqr_ms": q[2] - q[0],
            "cv_pct": cv, "rate_median": statistics.median(r["rate"] for r in rs), "unit": rs[0]["unit"],
        })
    return out


def write_master(path: str | Path, rows: list[dict]) -> None:
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(MASTER_HEADER)
        for r in rows:
            w.writerow([r["cell"], r["impl"], r["kernel"], r["config"], r["iter"], f"{r['gpu_ms']:.6f}",
                        f"{r['rate']:.6f}", r["unit"]])


def write_summary(path: str | Path, summary: list[dict]) -> None:
    lines = ["| cell | impl | kernel | config | n | best ms | median ms | p95 ms | IQR ms | CV % | rate (median) |",
             "|---|---|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for s in summary:
        lines.append(f"| {s['cell']} | {s['impl']} | {s['kernel']} | {s['config']} | {s['n']} | {s['best_ms']:.4f} | "
                     f"{s['median_ms']:.4f} | {s['p95_ms']:.4f} | {s['iqr_ms']:.4f} | {s['cv_pct']:.1f} | "
                     f"{s['rate_median']:.2f} {s['unit']} |")
    Path(path).write_text("\n".join(lines) + "\n")


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", required=True, help="master CSV to write")
    ap.add_argument("--summary", default=None, help="markdown summary to write")
    ap.add_argument("csvs", nargs="+")
    args = ap.parse_args(argv)
    rows: list[dict] = []
    for p in args.csvs:
        rows.extend(read_cell_csv(p))
    write_master(args.out, rows)
    if args.summary:
        write_summary(args.summary, summarize(rows))
    print(f"{len(rows)} rows from {len(args.csvs)} file(s) -> {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
