"""Build the gfx950 kernel library in-tree.

Compiles every ``csrc/*.hip`` and ``csrc/*.cpp`` with ``hipcc
--offload-arch=gfx950`` into ``libmxkernels.so`` next to this file, so the
library travels with the source tree to the GPU box.  hipcc cross-compiles
the device code here without a GPU.

Usage:  python -m <package>.build   or   python cuda-oxide-bench_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libmxkernels.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists() and not shutil.which(cand):
        raise RuntimeError(f"hipcc not found (looked for {cand})")
    return cand


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-fPIC",
        "-std=c++17",
        # Packed-fp32 VALU ops are kept out of every kernel on this target.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        "-Wno-unused-command-line-argument",
    ]


# Flags for single sources.  gqa_fwd.hip: its one-wave-per-SIMD kernels
# (512 registers) would otherwise get every builtin MFMA in AGPR form, so the
# softmax would copy each score tile out of AGPRs; with VGPR-form builtins
# the score MFMAs write VGPRs and only the P.V accumulators, issued as
# inline asm, live in AGPRs.  The kernels with at most 256 registers
# already get the VGPR form.
SOURCE_FLAGS = {
    "gqa_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def source_flags(src: Path) -> list[str]:
    return SOURCE_FLAGS.get(src.name, [])


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *common_flags(), *source_flags(src), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources and link ``libmxkernels.so``; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    build_probes(verbose)
    return LIB_PATH


PROBES_DIR = PKG_DIR / "microbench"
PROBES_LIB = PROBES_DIR / "libmxprobes.so"


def build_probes(verbose: bool = False) -> Path:
    """The hardware characterisation probes (microbench/hw_probes.hip) as
    their own library, libmxprobes.so; the kernel library does not use it."""
    src = PROBES_DIR / "hw_probes.hip"
    tmp = PROBES_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *common_flags(), "-shared", str(src), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"probe build failed\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, PROBES_LIB)
    return PROBES_LIB


ASAN_DIR = PKG_DIR / "_build_asan"
ASAN_DRIVER_SRC = REPO_ROOT / "tests" / "asan" / "capi_validation.cpp"


def clangxx() -> str:
    return str(Path(hipcc()).resolve().parent.parent / "llvm" / "bin" / "clang++")


def build_host_asan(verbose: bool = False, out_dir: Path | None = None) -> Path:
    """Debug variant for host-side checking: every source compiled at -O1
    with AddressSanitizer on the host code only (the gfx950 device code is
    built as usual, uninstrumented), linked into ``libmxkernels_asan.so`` in
    ``out_dir`` (default ``_build_asan/``) together with the C-ABI validation
    driver ``tests/asan/capi_validation.cpp``.  Returns the driver's path; run it
    with ASAN_OPTIONS=detect_leaks=0 (the HIP runtime keeps allocations
    until exit).  Not the product library: ``build()`` makes that."""
    out = Path(out_dir) if out_dir is not None else ASAN_DIR
    out.mkdir(parents=True, exist_ok=True)
    flags = [f"--offload-arch={ARCH}", "-O1", "-fPIC", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
             f"-I{INCLUDE}", f"-I{CSRC}", "-Wno-unused-command-line-argument"]

    def one(src: Path) -> Path:
        obj = out / (src.stem + ".o")
        cmd = [hipcc(), *(["-x", "hip"] if src.suffix == ".cpp" else []), *flags, *source_flags(src), "-c", str(src),
               "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"asan compile failed: {src.name}\n{proc.stdout}\n{proc.stderr}")
        return obj

    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), max(1, min(8, os.cpu_count() or 1)))) as ex:
        objs = list(ex.map(one, srcs))
    lib = out / "libmxkernels_asan.so"
    rocm_lib = Path(hipcc()).resolve().parent.parent / "lib"
    driver = out / "capi_validation"
    for cmd in ([clangxx(), "-shared", "-fsanitize=address", "-o", str(lib), *map(str, objs), f"-L{rocm_lib}",
                 "-lamdhip64", f"-Wl,-rpath,{rocm_lib}"],
                [clangxx(), "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
                 f"-I{INCLUDE}", str(ASAN_DRIVER_SRC), "-o", str(driver), f"-L{out}", "-lmxkernels_asan",
                 f"-Wl,-rpath,{out}"]):
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"asan link failed\n{proc.stdout}\n{proc.stderr}")
    return driver


if __name__ == "__main__":
    if "--asan" in sys.argv:
        print(build_host_asan(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
