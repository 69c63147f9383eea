"""ctypes binding of ``libmxkernels.so`` (the C-ABI declared in include/mx_kernels.h).

The library is loaded from this package directory.  There is no fallback:
if the shared object is missing or does not export a declared symbol, the
import fails with an error naming what is missing.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libmxkernels.so"

MX_OK = 0
MX_ERR_NULL = -1
MX_ERR_SHAPE = -2
MX_ERR_ALIGN = -3
MX_ERR_DTYPE = -4
MX_ERR_WORKSPACE = -5
MX_ERR_ALIAS = -6
MX_ERR_LAUNCH = -7
MX_ERR_UNSUPPORTED = -8

MX_DTYPE_BF16 = 0
MX_DTYPE_F16 = 1

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_ll = ctypes.c_longlong

# name -> (restype, argtypes); mirrors include/mx_kernels.h one to one.
SIGNATURES: dict[str, tuple] = {
    "mx_strerror": (ctypes.c_char_p, [_i]),
    "mx_version": (ctypes.c_char_p, []),
    "mx_gemm_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "mx_gemm_fp8_bs": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mx_gqa_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _i, _vp]),
    "mx_gqa_fwd_tile": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _i, _i, _i, _i, _vp]),
    "mx_gqa_fwd_tile_check": (_i, [_i, _i, _i, _i, _i, _i]),
    "mx_gqa_fwd_default_block_m": (_i, [_i, _i, _i]),
    "mx_gqa_fwd_tile_info": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "mx_mla_decode": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mx_mla_prefill_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _i, _vp]),
    "mx_mla_decode_workspace": (_sz, [_i, _i, _i, _i]),
    "mx_mla_decode_splits": (_i, [_i, _i, _i]),
    "mx_mla_decode_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "mx_gdn_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "mx_gdn_decode_block_v": (_i, [_i, _i, _i, _i]),
    "mx_kda_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "mx_quant_fp8_act": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "mx_gemm_bf16_batched": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _ll, _ll, _ll, _vp]),
    "mx_mla_decode_absorbed": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mx_mla_decode_absorbed_workspace": (_sz, [_i, _i, _i]),
}


class MXError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed: {message} (status {code})")
        self.fn = fn
        self.code = code


_LIB: ctypes.CDLL | None = None


def lib_path() -> Path:
    override = os.environ.get("MX_KERNELS_LIB")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Load the kernel library once and attach the declared signatures."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not path.exists():
        raise ImportError(
            f"{path.name} not found at {path}: build it with "
            f"`python {PKG_DIR.name}/build.py` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(path))
    missing = []
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            missing.append(name)
            continue
        fn.restype = res
        fn.argtypes = args
    if missing:
        raise ImportError(f"{path} does not export {', '.join(missing)}")
    _LIB = lib
    return lib


def strerror(code: int) -> str:
    return load().mx_strerror(code).decode()


def check(fn: str, code: int) -> None:
    if code != MX_OK:
        raise MXError(fn, code, strerror(code))


def call(fn: str, *args) -> None:
    """Call a status-returning entry point and raise MXError on failure."""
    check(fn, getattr(load(), fn)(*args))
