"""Run the MI355X characterisation probes (libmxprobes.so, built with the
kernel library) and print their results as Markdown tables.

    python cuda-oxide-bench_amd/microbench/run.py [--overlap] [--mfma-rate] [--contend] [--promote]
                                                  [--wg-read] [--stream]

--overlap: how much of a wave's other work runs beside its own MFMAs at one
wave per SIMD.  For each instruction mix: shader-clock cycles per iteration
of 8 independent 32x32x16 bf16 MFMAs alone, of the mix alone, and of both
interleaved (one MFMA, then its share of the mix); "hidden" is the part of
the mix's own time that the combination does not add.

--mfma-rate: chip-wide MFMA throughput (two waves per SIMD, ~70 ms
launches) for bf16 32x32x16 and 16x16x32 and fp8 32x32x64 and 16x16x128
MFMAs, on random operands that change from one MFMA to the next and on
constant ones: at the power cap the first run at a lower clock than the
second.

--contend: shader-clock cycles per MFMA of a wave issuing independent MFMAs
(bf16 32x32x16 or fp8 32x32x64, accumulators in VGPRs or AGPRs) while the
other wave on its SIMD idles, runs independent v_fma_f32, v_exp_f32 or
v_dot2_f32_bf16 work, issues the same MFMAs or streams LDS reads, with the
clock the chip held meanwhile.

--promote: the fp8 GEMM's block promotion (two 32x32x64 fp8 MFMAs into a
fresh partial, then acc += s * partial) in shader-clock cycles per
fragment-block and SIMD, against the MFMAs alone and against the same FMAs
on registers no MFMA writes, at one and two waves per SIMD.

--wg-read: the read bandwidth of one workgroup (256 threads, 16-byte loads,
eight in flight per thread) against many, on data just written and on data
evicted by a 512 MB write: event time per launch, less an empty launch.

--stream: the same reads with 4 to 32 loads in flight, into registers
(per thread) or by direct global -> LDS loads (per wave, the kernels' tile
copies), by one workgroup and by 256 workgroups (one per CU) that read
either distinct data or all the same 256 KB.

All start after the device settle bench.py uses (300 ms of a device GEMM),
so the GPU runs at its load clocks.
"""
from __future__ import annotations

import argparse
import ctypes
import statistics
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmxprobes.so"

OVERLAP_PROBES = [
    (1, "32 v_exp_f32"),
    (2, "32 v_cvt_pk_bf16_f32"),
    (3, "32 v_dot2_f32_bf16"),
    (4, "32 v_add_f32"),
    (5, "32 v_mul_f32"),
    (6, "32 v_fma_f32"),
    (7, "8 s_nop 0 (one per MFMA)"),
    (8, "8 s_nop 1 (one per MFMA)"),
    (9, "32 v_exp_f32 + 8 s_nop 1 (one per MFMA)"),
    (10, "8 ds_read_b128 of 1 KB, each the B operand of the next iteration's MFMA (alone: consumed by a v_xor)"),
]


def load() -> ctypes.CDLL:
    # torch first: the library binds to whichever libamdhip64.so.7 the process
    # loaded first, and it must be torch's, which owns the device here.
    import torch  # noqa: F401

    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build the package first (python cuda-oxide-bench_amd/build.py)")
    lib = ctypes.CDLL(str(LIB_PATH))
    i, vp, ll = ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong
    lib.mxp_overlap_launch.argtypes = [i, i, i, i, vp, vp, vp]
    lib.mxp_overlap_launch.restype = i
    lib.mxp_wg_read_launch.argtypes = [vp, ll, ll, i, vp, vp]
    lib.mxp_wg_read_launch.restype = i
    lib.mxp_mfma_rate_launch.argtypes = [i, i, i, vp, vp, vp]
    lib.mxp_mfma_rate_launch.restype = i
    lib.mxp_contend_launch.argtypes = [i, i, i, i, i, vp, vp, vp, vp, vp, vp]
    lib.mxp_contend_launch.restype = i
    lib.mxp_promote_launch.argtypes = [i, i, i, i, i, vp, vp, vp, vp]
    lib.mxp_promote_launch.restype = i
    lib.mxp_stream_launch.argtypes = [i, i, vp, ll, ll, i, vp, vp]
    lib.mxp_stream_launch.restype = i
    lib.mxp_error_string.argtypes = [i]
    lib.mxp_error_string.restype = ctypes.c_char_p
    return lib


def settle(ms: float = 300.0) -> None:
    import torch

    a = torch.randn(8192, 8192, device="cuda").to(torch.bfloat16)
    c = torch.empty_like(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            torch.matmul(a, a, out=c)
        torch.cuda.synchronize()


def overlap_cycles(lib, probe: int, with_mfma: int, iters: int, reps: int) -> float:
    """Median over reps of the workgroups' mean cycles per iteration."""
    import torch

    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(nwg * 256, dtype=torch.float32, device="cuda")
    cyc = torch.zeros(nwg, dtype=torch.int64, device="cuda")
    vals = []
    for _ in range(reps):
        rc = lib.mxp_overlap_launch(probe, with_mfma, nwg, iters, out.data_ptr(), cyc.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"mxp_overlap_launch({probe}, {with_mfma}): {lib.mxp_error_string(rc).decode()} ({rc})")
        torch.cuda.synchronize()
        vals.append(cyc.double().mean().item() / iters)
    return statistics.median(vals)


def overlap(lib, iters: int = 2000, reps: int = 3) -> list[str]:
    mfma = overlap_cycles(lib, 0, 1, iters, reps)
    lines = ["| mix per iteration | mix alone | beside 8 MFMAs | 8 MFMAs alone | hidden |", "|---|---:|---:|---:|---:|"]
    for probe, name in OVERLAP_PROBES:
        alone = overlap_cycles(lib, probe, 0, iters, reps)
        both = overlap_cycles(lib, probe, 1, iters, reps)
        hidden = max(0.0, min(1.0, (alone + mfma - both) / alone)) if alone > 0 else 0.0
        lines.append(f"| {name} | {alone:.1f} | {both:.1f} | {mfma:.1f} | {100 * hidden:.0f}% |")
    return lines


def mfma_rate(lib, target_ms: float = 70.0, reps: int = 3) -> list[str]:
    import torch

    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    threads = nwg * 512
    out = torch.empty(threads, dtype=torch.float32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(5)
    bf16 = {"random": torch.randn(threads * 64, device="cuda", generator=g).to(torch.bfloat16),
            "constant (all 0.5)": torch.full((threads * 64,), 0.5, device="cuda", dtype=torch.bfloat16)}
    fp8 = {k: v.float().to(torch.float8_e4m3fn) for k, v in
           (("random", torch.randn(threads * 128, device="cuda", generator=g)),
            ("constant (all 0.5)", torch.full((threads * 128,), 0.5, device="cuda")))}
    stream = torch.cuda.current_stream().cuda_stream

    def launch(shape, ops, iters):
        rc = lib.mxp_mfma_rate_launch(shape, nwg, iters, ops.data_ptr(), out.data_ptr(), stream)
        if rc != 0:
            raise RuntimeError(f"mxp_mfma_rate_launch: {lib.mxp_error_string(rc).decode()} ({rc})")

    def ms_of(shape, ops, iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        launch(shape, ops, iters)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    lines = ["| MFMA | operands | iterations per launch | ms per launch | PFLOP/s |", "|---|---|---:|---:|---:|"]
    for shape, name, flop, operands in ((0, "32x32x16 bf16, VGPR accumulators", 32768, bf16),
                                        (2, "32x32x16 bf16, AGPR accumulators", 32768, bf16),
                                        (1, "16x16x32 bf16, VGPR accumulators", 16384, bf16),
                                        (5, "16x16x32 bf16, AGPR accumulators", 16384, bf16),
                                        (3, "32x32x64 fp8, VGPR accumulators", 131072, fp8),
                                        (6, "32x32x64 fp8, AGPR accumulators", 131072, fp8),
                                        (4, "16x16x128 fp8, VGPR accumulators", 65536, fp8),
                                        (7, "16x16x128 fp8, AGPR accumulators", 65536, fp8)):
        for label, ops in operands.items():
            iters = 2000
            t = ms_of(shape, ops, iters)
            iters = max(1, int(iters * target_ms / max(t, 1e-3)))
            ms_of(shape, ops, iters)  # at load clocks before the timed launches
            ms = statistics.median(ms_of(shape, ops, iters) for _ in range(reps))
            flops = nwg * 8 * iters * 8 * flop
            lines.append(f"| {name} | {label} | {iters} | {ms:.2f} | {flops / ms / 1e12:.3f} |")
    return lines


WG_READ_CASES = [  # (name, workgroups, element stride between workgroups, elements per workgroup)
    ("1 workgroup x 896 KB", 1, 0, 896 * 1024 // 16),
    ("32 workgroups x 896 KB", 32, (1 << 20) // 16, 896 * 1024 // 16),
    ("256 workgroups x 112 KB", 256, 7168, 7168),
]


def wg_read(lib, reps: int = 20) -> list[str]:
    import torch

    total = (32 << 20) // 16
    src = torch.empty(total * 16, dtype=torch.uint8, device="cuda")
    evict = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    out = torch.empty(256 * 256, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for _, nwg, stride, n in WG_READ_CASES:
        assert (nwg - 1) * stride + n <= total

    def timed(nwg, stride, n, cold):
        ts = []
        for r in range(reps):
            src.fill_(r & 0xff)  # freshly written
            if cold:
                evict.fill_(r & 0xff)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            rc = lib.mxp_wg_read_launch(src.data_ptr(), stride, n, nwg, out.data_ptr(), stream)
            if rc != 0:
                raise RuntimeError(f"mxp_wg_read_launch: {lib.mxp_error_string(rc).decode()} ({rc})")
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return statistics.mean(ts)

    lines = ["| case | data | µs per launch | less an empty launch | GB/s per workgroup |", "|---|---|---:|---:|---:|"]
    for cold in (False, True):
        empty = timed(1, 0, 0, cold)
        for name, nwg, stride, n in WG_READ_CASES:
            us = timed(nwg, stride, n, cold)
            net = us - empty
            rate = f"{n * 16 / net / 1e3:.1f}" if net >= 0.5 else "below the timing resolution"
            lines.append(f"| {name} | {'evicted' if cold else 'just written'} | {us:.2f} | {net:.2f} | {rate} |")
        lines.append(f"| empty launch | {'evicted' if cold else 'just written'} | {empty:.2f} | | |")
    return lines


CONTEND_FORMS = [(0, "32x32x16 bf16, VGPR accumulators"), (1, "32x32x16 bf16, AGPR accumulators"),
                 (2, "32x32x64 fp8, VGPR accumulators"), (3, "32x32x64 fp8, AGPR accumulators"),
                 (4, "16x16x32 bf16, VGPR accumulators")]


def contend(lib, iters: int = 4000, reps: int = 3) -> list[str]:
    import torch

    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda").manual_seed(7)
    bf16 = torch.randn(nwg * 512 * 32, device="cuda", generator=g).to(torch.bfloat16)
    fp8 = torch.randn(nwg * 512 * 64, device="cuda", generator=g).to(torch.float8_e4m3fn)
    out = torch.empty(nwg * 512, dtype=torch.float32, device="cuda")
    cycles = torch.zeros(nwg * 8, dtype=torch.int64, device="cuda")
    rtime = torch.zeros(nwg * 8, dtype=torch.int64, device="cuda")
    hwid = torch.zeros(nwg * 8, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream

    def run(form, busy):
        """Median over reps of: cycles per MFMA of waves 0-3, their clock (GHz from the
        100 MHz real-time counter), waves 4-7's cycles, and the share of workgroups whose
        waves w and w + 4 report the same SIMD."""
        valu_iters = {1: 12 * iters, 3: 3 * iters, 4: 6 * iters, 5: 12 * iters}.get(busy, 0)
        mf, clk, other, paired = [], [], [], []
        for _ in range(reps):
            ops = bf16 if form in (0, 1, 4) else fp8
            rc = lib.mxp_contend_launch(form, busy, nwg, iters, valu_iters, ops.data_ptr(), out.data_ptr(),
                                        cycles.data_ptr(), rtime.data_ptr(), hwid.data_ptr(), st)
            if rc != 0:
                raise RuntimeError(f"mxp_contend_launch: {lib.mxp_error_string(rc).decode()} ({rc})")
            torch.cuda.synchronize()
            c = cycles.view(nwg, 8).double()
            rt = rtime.view(nwg, 8).double()
            mf.append(c[:, :4].median().item() / (iters * 8))
            clk.append((c[:, :4] / rt[:, :4].clamp(min=1)).median().item() / 10)
            other.append(c[:, 4:].median().item())
            simd = (hwid.view(nwg, 8) >> 4) & 3
            paired.append((simd[:, :4] == simd[:, 4:]).all(dim=1).float().mean().item())
        return statistics.median(mf), statistics.median(clk), statistics.median(other), min(paired)

    lines = ["| MFMA (operands random) | waves 4-7 | waves 0-3: cycles per MFMA | clock GHz | "
             "waves 4-7: cycles per instruction | waves 4-7 took (cycles) | waves 0-3 took | waves share a SIMD | "
             "MFMA cycles lost per KB read |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for form, name in CONTEND_FORMS:
        idle = None
        for busy, label in ((0, "idle"), (1, "v_fma_f32 stream"), (2, "the same MFMA stream"),
                            (3, "128-bit LDS reads (1 KB each, conflict-free)"),
                            (4, "v_exp_f32 stream"), (5, "v_dot2_f32_bf16 stream")):
            if busy >= 4 and form not in (0, 1, 4):
                continue  # the softmax instructions sit beside bf16 MFMAs only
            per_wave, ghz, other, paired = run(form, busy)
            n_other = {1: 12 * iters * 32, 2: iters * 8, 3: 3 * iters * 8, 4: 6 * iters * 32,
                       5: 12 * iters * 32}.get(busy, 1)
            o_per = f"{other / n_other:.1f}" if busy else ""
            o_tot = f"{other:.0f}" if busy else ""
            if busy == 0:
                idle = per_wave
            lost = ""
            if busy == 3:
                # KB the partner wave read while this wave's MFMAs ran, at its own rate
                t_m = per_wave * iters * 8
                kb = (3 * iters * 8) * t_m / max(other, 1.0)
                lost = f"{(per_wave - idle) * iters * 8 / kb:.1f}"
            lines.append(f"| {name} | {label} | {per_wave:.1f} | {ghz:.2f} | {o_per} | {o_tot} | "
                         f"{per_wave * iters * 8:.0f} | {100 * paired:.0f}% | {lost} |")
    return lines


PROMOTE_CASES = [(0, 1, "MFMAs only (accumulating straight into the accumulators)"),
                 (2, 1, "MFMAs only, beside the same FMAs on registers no MFMA writes"),
                 (1, 1, "promotion, the compiler's order (lag 1: two partial sets)"),
                 (1, 3, "promotion, the compiler's order (lag 3: four partial sets)"),
                 (3, 1, "promotion after the next fragment's two MFMAs (enforced)"),
                 (3, 2, "promotion after two more fragments' MFMAs (enforced)"),
                 (3, 3, "promotion after three more fragments' MFMAs (enforced)")]


def promote(lib, iters: int = 2000, reps: int = 3) -> list[str]:
    import torch

    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda").manual_seed(11)
    ops = torch.randn(nwg * 512 * 64, device="cuda", generator=g).to(torch.float8_e4m3fn)
    out = torch.empty(nwg * 512, dtype=torch.float32, device="cuda")
    cycles = torch.zeros(nwg * 8, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream

    def run(mode, lag, waves):
        vals = []
        for _ in range(reps):
            rc = lib.mxp_promote_launch(mode, lag, waves, nwg, iters, ops.data_ptr(), out.data_ptr(),
                                        cycles.data_ptr(), st)
            if rc != 0:
                raise RuntimeError(f"mxp_promote_launch: {lib.mxp_error_string(rc).decode()} ({rc})")
            torch.cuda.synchronize()
            c = cycles[: nwg * waves].view(nwg, waves).double()
            vals.append(c.max(dim=1).values.median().item() / (iters * 8 * (waves // 4)))
        return statistics.median(vals)

    lines = ["| per fragment and scale block (2 MFMAs = 128 MFMA cycles, 16 v_fma) | one wave per SIMD | two waves per SIMD |",
             "|---|---:|---:|"]
    for mode, lag, name in PROMOTE_CASES:
        one, two = run(mode, lag, 4), run(mode, lag, 8)
        lines.append(f"| {name} | {one:.1f} | {two:.1f} |")
    return lines


STREAM_CASES = [  # (name, workgroups, element stride between workgroups, elements per workgroup)
    ("1 workgroup x 1 MB", 1, 0, (1 << 20) // 16),
    ("256 workgroups x 256 KB, distinct", 256, (256 << 10) // 16, (256 << 10) // 16),
    ("256 workgroups x 256 KB, all the same", 256, 0, (256 << 10) // 16),
]
STREAM_DEPTHS = (4, 8, 16, 32)


def stream(lib, reps: int = 20) -> list[str]:
    import torch

    total = (64 << 20) // 16
    src = torch.empty(total * 16, dtype=torch.uint8, device="cuda")
    out = torch.empty(256 * 256, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for _, nwg, stride, n in STREAM_CASES:
        assert (nwg - 1) * stride + n <= total and n % 64 == 0

    def timed(mode, depth, nwg, stride, n):
        ts = []
        for r in range(reps):
            src.fill_(r & 0xff)  # freshly written
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            rc = lib.mxp_stream_launch(mode, depth, src.data_ptr(), stride, n, nwg, out.data_ptr(), st)
            if rc != 0:
                raise RuntimeError(f"mxp_stream_launch: {lib.mxp_error_string(rc).decode()} ({rc})")
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return statistics.mean(ts)

    lines = ["| case | loads | in flight per workgroup | µs less an empty launch | GB/s per workgroup | GB/s in all |",
             "|---|---|---:|---:|---:|---:|"]
    for name, nwg, stride, n in STREAM_CASES:
        for mode, kind in ((0, "registers"), (1, "direct to LDS")):
            for depth in STREAM_DEPTHS:
                empty = timed(mode, depth, 1, 0, 0)
                net = timed(mode, depth, nwg, stride, n) - empty
                kb = 256 * depth * 16 // 1024 if mode == 0 else 4 * depth
                if net >= 0.5:
                    per, total_rate = f"{n * 16 / net / 1e3:.1f}", f"{nwg * n * 16 / net / 1e3:.0f}"
                else:
                    per = total_rate = "below the timing resolution"
                lines.append(f"| {name} | {kind} | {kb} KB | {net:.2f} | {per} | {total_rate} |")
    return lines


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--overlap", action="store_true")
    ap.add_argument("--mfma-rate", action="store_true")
    ap.add_argument("--contend", action="store_true")
    ap.add_argument("--promote", action="store_true")
    ap.add_argument("--wg-read", action="store_true")
    ap.add_argument("--stream", action="store_true")
    ap.add_argument("--iters", type=int, default=2000, help="overlap-probe iterations per launch")
    args = ap.parse_args()
    every = not (args.overlap or args.mfma_rate or args.contend or args.promote or args.wg_read or args.stream)
    import torch

    if not torch.cuda.is_available():
        print("no GPU", file=sys.stderr)
        return 2
    lib = load()
    print(f"device: {torch.cuda.get_device_name(0)}, "
          f"{torch.cuda.get_device_properties(0).multi_processor_count} CUs", flush=True)
    settle()
    if every or args.overlap:
        print("\n## Overlap with a wave's own MFMAs (cycles per iteration, one wave per SIMD)\n")
        print("\n".join(overlap(lib, args.iters)), flush=True)
    if every or args.mfma_rate:
        print("\n## Chip-wide MFMA throughput, two waves per SIMD\n")
        print("\n".join(mfma_rate(lib)), flush=True)
    if every or args.contend:
        print("\n## MFMAs beside another wave's work (cycles per MFMA, two waves per SIMD)\n")
        print("\n".join(contend(lib)), flush=True)
    if every or args.promote:
        print("\n## fp8 block promotion (shader-clock cycles per fragment and scale block, per SIMD)\n")
        print("\n".join(promote(lib)), flush=True)
    if every or args.wg_read:
        print("\n## Read bandwidth of one workgroup against many\n")
        print("\n".join(wg_read(lib)), flush=True)
    if every or args.stream:
        print("\n## Read rate against the loads in flight\n")
        print("\n".join(stream(lib)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
