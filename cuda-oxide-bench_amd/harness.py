"""Shared plumbing for the per-kernel harness cells (cells/*/main.py).

Mirrors what every reference harness does inline (e.g.
cutile-attn-gqa/main.py:281-341, cutile-attn-gdn/main.py:323-409):
device banner, warm-up + per-launch event timing, results.csv rows with
the reference's column order, best/median/worst summary, and a
`roofline.json` sidecar carrying what the reference's CSV cannot
(achieved rate vs MI355X peak).  Timing uses torch.cuda.Event pairs on the
current stream, the stream the operators launch on.
"""
from __future__ import annotations

import csv
import importlib
import json
import statistics
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
GOLDEN_DIR = REPO_ROOT / "tests" / "golden"

# Exit codes of the reference harnesses: 0 ok, 1 smoke failure
# (cutile-attn-gqa/main.py:419-420), 2 correctness failure before a bench
# (cutile-matmul-tc-bf16/main.py:224-226).
EXIT_OK, EXIT_SMOKE_FAIL, EXIT_CORRECTNESS_FAIL = 0, 1, 2


def package():
    if str(REPO_ROOT) not in sys.path:
        sys.path.insert(0, str(REPO_ROOT))
    return importlib.import_module(PKG_DIR.name)


def banner() -> None:
    import torch

    pkg = package()
    lib = importlib.import_module(f"{PKG_DIR.name}._lib")
    print(f"library: {lib.load().mx_version().decode()}")
    print(f"torch: {torch.__version__} (HIP {torch.version.hip})")
    print(f"device: {torch.cuda.get_device_name(0)}")
    props = torch.cuda.get_device_properties(0)
    print(f"arch: {getattr(props, 'gcnArchName', '?')}  CUs: {props.multi_processor_count}")
    print(f"package: {pkg.__name__} {pkg.__version__}")


def time_iters(fn, warmup: int, iters: int, min_group_ms: float = 0.5, graph: bool = True) -> list[float]:
    """warmup untimed calls, then `iters` timed samples of the per-launch time.

    Each sample is one event pair around a group of back-to-back launches,
    divided by the group size; the group is sized (from an untimed probe)
    to last at least `min_group_ms`.  With graph=True the group is captured
    once into a HIP graph (torch.cuda.CUDAGraph) and replayed, so the
    sample measures the kernels rather than the host cost of issuing them
    (~10 us per operator call from Python).  An event pair around every
    single launch, as the reference's CUDA harnesses use, also adds ~10 us
    per launch on ROCm, which would swamp the few-microsecond decode kernels.
    """
    import time

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    est_ms = max((time.perf_counter() - t0) * 1e3, 1e-3)
    reps = max(1, min(200, int(min_group_ms / est_ms + 0.999)))
    run_group = None
    if graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()  # first call on the capture stream outside the capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        run_group = g.replay
    else:
        def run_group():
            for _ in range(reps):
                fn()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record()
        run_group()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) / reps for s, e in zip(starts, ends)]


def summarize_ms(ms: list[float]) -> dict:
    srt = sorted(ms)
    n = len(srt)
    return {"best_ms": srt[0], "median_ms": statistics.median(srt), "worst_ms": srt[-1],
            "mean_ms": sum(srt) / n, "q1_ms": srt[n // 4], "q3_ms": srt[(3 * n) // 4]}


def write_csv(path: str, header: list[str], rows: list[list]) -> None:
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def write_sidecar(csv_path: str, payload: dict) -> Path:
    """roofline.json next to results.csv (columns of the CSV stay the reference's)."""
    p = Path(csv_path).resolve().with_name("roofline.json")
    p.write_text(json.dumps(payload, indent=2, default=float) + "\n")
    return p


def load_golden(name: str) -> dict:
    import numpy as np

    path = GOLDEN_DIR / f"{name}.npz"
    if not path.exists():
        raise FileNotFoundError(f"golden fixture {path} is missing")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def reference_fixtures(inputs_dir: str, kind: str, name: str) -> dict:
    """A fixture set written under the reference's inputs/ names (see npy.py)."""
    npy = importlib.import_module(f"{PKG_DIR.name}.npy")
    fx = npy.load_fixture_set(inputs_dir, kind, name)
    print(f"[fixtures] {kind}_{name}_* from {inputs_dir}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in fx.items()))
    return fx


def from_bits(arr, dtype):
    """uint16 bit patterns (as stored in the fixtures) -> torch bf16/f16 tensor."""
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(dtype)


def print_summary(title: str, st: dict, rate_best: float, rate_median: float, unit: str, peak: float) -> None:
    print()
    print("=" * 72)
    print(f" BENCH SUMMARY — {title}")
    print(f"   median : {st['median_ms']:.4f} ms   {rate_median:10.2f} {unit}   ({rate_median / peak:.1%} of peak)")
    print(f"   best   : {st['best_ms']:.4f} ms   {rate_best:10.2f} {unit}   ({rate_best / peak:.1%} of peak)")
    print(f"   worst  : {st['worst_ms']:.4f} ms")
    print("=" * 72)
