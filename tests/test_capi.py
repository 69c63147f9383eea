"""C-ABI checks that need no GPU: the library loads, exports every entry
point include/mx_kernels.h declares, and rejects invalid arguments before
launching anything (these calls never reach the HIP runtime)."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import REPO_ROOT, import_submodule

_lib = import_submodule("_lib")
HEADER = REPO_ROOT / "include" / "mx_kernels.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("mx_gemm_bf16", "mx_gemm_fp8_bs", "mx_gqa_fwd", "mx_mla_decode", "mx_mla_decode_workspace",
              "mx_gdn_decode", "mx_kda_decode", "mx_quant_fp8_act", "mx_gemm_bf16_batched", "mx_mla_decode_absorbed",
              "mx_mla_decode_absorbed_workspace", "mx_mla_prefill_fwd", "mx_strerror",
              "mx_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for n in declared_functions():
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.lib_path())], capture_output=True, text=True)
    if out.returncode == 0:
        exported = set(re.findall(r" T (mx_[a-z0-9_]+)", out.stdout))
        assert set(declared_functions()) <= exported


def test_strerror_and_version():
    lib = _lib.load()
    assert lib.mx_version().decode().startswith("mxkernels")
    for code in range(0, -9, -1):
        assert lib.mx_strerror(code)
    assert _lib.strerror(_lib.MX_ERR_ALIAS) == "output overlaps an input"


P = ctypes.c_void_p(0x10000)  # never dereferenced: every call below fails validation


@pytest.mark.parametrize("args,code", [
    ((None, P, P, 64, 64, 64, 64, 64, 64, None), _lib.MX_ERR_NULL),
    ((P, P, P, 0, 64, 64, 64, 64, 64, None), _lib.MX_ERR_SHAPE),
    ((P, P, P, 64, 64, 60, 60, 64, 64, None), _lib.MX_ERR_ALIGN),
    ((P, P, P, 64, 64, 64, 32, 64, 64, None), _lib.MX_ERR_SHAPE),
    ((ctypes.c_void_p(0x10008), P, P, 64, 64, 64, 64, 64, 64, None), _lib.MX_ERR_ALIGN),
    # register-staged kernel: 64 rows of A at this stride pass its 2^31-byte buffer range
    ((P, P, P, 64, 64, 64, 20971520, 64, 64, None), _lib.MX_ERR_SHAPE),
])
def test_gemm_bf16_validation(args, code):
    assert _lib.load().mx_gemm_bf16(*args) == code


def test_gemm_fp8_validation():
    f = _lib.load().mx_gemm_fp8_bs
    assert f(P, P, P, P, None, 64, 64, 128, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, P, P, 64, 64, 100, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, P, P, 64, 40, 128, None) == _lib.MX_ERR_ALIGN
    # M*K below the 2^40 element limit, but the sA byte offsets pass 2^32
    assert f(P, P, P, P, P, (1 << 30) + 1, 16, 128, None) == _lib.MX_ERR_SHAPE


def test_gqa_validation():
    f = _lib.load().mx_gqa_fwd
    assert f(None, P, P, P, 1, 4, 2, 16, 64, 0.125, 1, 0, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, P, 1, 4, 3, 16, 64, 0.125, 1, 0, None) == _lib.MX_ERR_SHAPE   # Hq % Hkv
    assert f(P, P, P, P, 1, 4, 2, 16, 96, 0.125, 1, 0, None) == _lib.MX_ERR_SHAPE   # D
    assert f(P, P, P, P, 1, 4, 2, 16, 64, 0.125, 1, 7, None) == _lib.MX_ERR_DTYPE
    assert f(P, P, P, P, 1, 4, 2, 16, 64, -1.0, 1, 0, None) == _lib.MX_ERR_SHAPE


def test_gqa_tile_validation():
    f = _lib.load().mx_gqa_fwd_tile
    ok = (P, P, P, P, 1, 32, 8, 256, 128, 0.088, 1, 0)
    assert f(None, *ok[1:], 64, 64, 32, None) == _lib.MX_ERR_NULL
    assert f(*ok, 64, 32, 32, None) == _lib.MX_ERR_UNSUPPORTED    # BLOCK_N is the 64-key stage
    assert f(*ok, 16, 64, 32, None) == _lib.MX_ERR_UNSUPPORTED    # 8 or 16 heads per workgroup: more than G = 4
    assert f(*ok, 96, 64, 32, None) == _lib.MX_ERR_UNSUPPORTED    # 256 rows are not whole 96-row blocks
    assert f(*ok, 512, 64, 32, None) == _lib.MX_ERR_UNSUPPORTED   # fewer rows than one block
    assert f(*ok, 64, 64, 48, None) == _lib.MX_ERR_UNSUPPORTED    # wave_m
    assert f(P, P, P, P, 1, 32, 8, 256, 128, 0.088, 1, 9, 64, 64, 32, None) == _lib.MX_ERR_DTYPE


@pytest.mark.parametrize("hq,hkv,d,bm,wm,code", [
    # G = 4 (the bench shapes): 8 waves of 32 cover 4, 2 or 1 heads, 4 waves of 32 cover 4 heads in 32-row
    # blocks, 4 waves of 64 cover 4, 2 or 1 heads
    (32, 8, 128, 64, 32, 0), (32, 8, 128, 128, 32, 0), (32, 8, 128, 256, 32, 0), (32, 8, 128, 32, 32, 0),
    (32, 8, 128, 64, 64, 0), (32, 8, 128, 128, 64, 0), (32, 8, 128, 256, 64, 0),
    (32, 8, 128, 16, 32, _lib.MX_ERR_UNSUPPORTED), (32, 8, 128, 32, 64, _lib.MX_ERR_UNSUPPORTED),
    (32, 8, 128, 512, 32, _lib.MX_ERR_UNSUPPORTED), (32, 8, 128, 96, 32, _lib.MX_ERR_UNSUPPORTED),
    # G = 2 (the correctness shape): 64-row blocks on the 4-wave kernel, 128 and 256 on the 8-wave one
    (4, 2, 64, 64, 32, 0), (4, 2, 64, 128, 32, 0), (4, 2, 64, 256, 32, 0), (4, 2, 64, 32, 32, _lib.MX_ERR_UNSUPPORTED),
    (4, 2, 64, 64, 64, _lib.MX_ERR_UNSUPPORTED), (4, 2, 64, 128, 64, 0),
    # G = 1 (MHA): whole-workgroup blocks only
    (4, 4, 64, 256, 32, 0), (4, 4, 64, 128, 32, 0), (4, 4, 64, 64, 32, _lib.MX_ERR_UNSUPPORTED),
    (64, 8, 64, 32, 32, 0),
    (32, 8, 96, 64, 32, _lib.MX_ERR_SHAPE), (32, 7, 128, 64, 32, _lib.MX_ERR_SHAPE),
])
def test_gqa_tile_check(hq, hkv, d, bm, wm, code):
    assert _lib.load().mx_gqa_fwd_tile_check(hq, hkv, d, bm, 64, wm) == code


def test_gqa_default_block_m():
    f = _lib.load().mx_gqa_fwd_default_block_m
    assert [f(32, 8, 128), f(4, 2, 64), f(4, 4, 64), f(64, 8, 128)] == [64, 128, 256, 64]
    assert f(32, 7, 128) == _lib.MX_ERR_SHAPE
    # the default tile is always one mx_gqa_fwd_tile accepts
    for hq, hkv in ((32, 8), (4, 2), (4, 4), (12, 4), (6, 2)):
        assert _lib.load().mx_gqa_fwd_tile_check(hq, hkv, 128, f(hq, hkv, 128), 64, 32) == 0


def test_mla_prefill_validation():
    f = _lib.load().mx_mla_prefill_fwd
    assert f(None, P, P, P, 1, 4, 16, 192, 128, 0.07, 0, 0, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, P, 1, 4, 0, 192, 128, 0.07, 0, 0, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, P, 1, 4, 16, 160, 128, 0.07, 0, 0, None) == _lib.MX_ERR_UNSUPPORTED
    assert f(P, P, P, P, 1, 4, 16, 192, 64, 0.07, 0, 0, None) == _lib.MX_ERR_UNSUPPORTED
    assert f(P, P, P, P, 1, 4, 16, 192, 128, 0.07, 0, 5, None) == _lib.MX_ERR_DTYPE
    assert f(P, P, P, P, 1, 4, 16, 192, 128, 0.0, 0, 0, None) == _lib.MX_ERR_SHAPE


def test_mla_validation_and_workspace():
    lib = _lib.load()
    assert lib.mx_mla_decode_workspace(32, 128, 4096, 512) > 0
    assert lib.mx_mla_decode_workspace(32, 128, 4096, 256) == 0
    assert lib.mx_mla_decode_workspace(1, 16, 64, 512) == 0  # short context: no split
    f = lib.mx_mla_decode
    assert f(P, P, P, 32, 128, 4096, 512, 64, 0.07, None, 0, None) == _lib.MX_ERR_WORKSPACE
    assert f(P, P, P, 1, 16, 64, 256, 64, 0.07, None, 0, None) == _lib.MX_ERR_UNSUPPORTED
    assert f(None, P, P, 1, 16, 64, 512, 64, 0.07, None, 0, None) == _lib.MX_ERR_NULL


def test_gdn_validation():
    f = _lib.load().mx_gdn_decode
    args = [P] * 8
    assert f(None, *args[1:], 2, 2, 4, 64, 64, 0, None) == _lib.MX_ERR_NULL
    assert f(*args, 2, 3, 4, 64, 64, 0, None) == _lib.MX_ERR_SHAPE     # Hv % Hk
    assert f(*args, 2, 2, 4, 96, 64, 0, None) == _lib.MX_ERR_SHAPE     # dk
    assert f(*args, 2, 2, 4, 64, 64, 3, None) == _lib.MX_ERR_DTYPE
    s_in, s_out = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x100000 + 256)
    assert f(P, P, P, P, P, s_in, s_out, P, 2, 2, 4, 64, 64, 0, None) == _lib.MX_ERR_ALIAS


def test_kda_validation():
    f = _lib.load().mx_kda_decode
    args = [P] * 8
    assert f(None, *args[1:], 2, 4, 64, 64, 0, None) == _lib.MX_ERR_NULL
    assert f(*args[:3], None, *args[4:], 2, 4, 64, 64, 0, None) == _lib.MX_ERR_NULL   # g
    assert f(*args, 0, 4, 64, 64, 0, None) == _lib.MX_ERR_SHAPE
    assert f(*args, 2, 4, 96, 64, 0, None) == _lib.MX_ERR_SHAPE      # dk
    assert f(*args, 2, 4, 64, 64, 3, None) == _lib.MX_ERR_DTYPE
    s_in, s_out = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x100000 + 256)
    assert f(P, P, P, P, P, s_in, s_out, P, 2, 4, 64, 64, 0, None) == _lib.MX_ERR_ALIAS


def test_quant_fp8_validation():
    f = _lib.load().mx_quant_fp8_act
    assert f(None, P, P, 4, 128, 128, 0, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, 4, 96, 96, 0, None) == _lib.MX_ERR_SHAPE       # K % 128
    assert f(P, P, P, 4, 128, 64, 0, None) == _lib.MX_ERR_SHAPE      # ldx < K
    assert f(P, P, P, 4, 128, 132, 0, None) == _lib.MX_ERR_ALIGN     # ldx % 8
    assert f(P, P, P, 4, 128, 128, 2, None) == _lib.MX_ERR_DTYPE


def test_gemm_batched_validation():
    f = _lib.load().mx_gemm_bf16_batched
    assert f(None, P, P, 2, 64, 64, 64, 64, 64, 64, 4096, 4096, 4096, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, 0, 64, 64, 64, 64, 64, 64, 4096, 4096, 4096, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, 70000, 64, 64, 64, 64, 64, 64, 0, 0, 0, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, 2, 64, 64, 64, 64, 64, 64, -8, 0, 0, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, 2, 64, 64, 64, 64, 64, 64, 4, 0, 0, None) == _lib.MX_ERR_ALIGN
    assert f(P, P, P, 2, 64, 64, 64, 64, 20971520, 64, 0, 0, 0, None) == _lib.MX_ERR_SHAPE  # ldb past the buffer range


def test_mla_absorbed_validation():
    lib = _lib.load()
    f = lib.mx_mla_decode_absorbed
    need = lib.mx_mla_decode_absorbed_workspace(32, 128, 4096)
    assert need >= 2 * 32 * 128 * 512 * 2
    assert f(None, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07, P, need, None) == _lib.MX_ERR_NULL
    assert f(P, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07, None, 0, None) == _lib.MX_ERR_WORKSPACE
    assert f(P, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07, P, need - 1, None) == _lib.MX_ERR_WORKSPACE
    assert f(P, P, P, P, P, P, 32, 128, 4096, 100, 128, 0.07, P, need, None) == _lib.MX_ERR_SHAPE
    assert f(P, P, P, P, P, P, 32, 128, 4096, 128, 128, -1.0, P, need, None) == _lib.MX_ERR_SHAPE


def test_mla_absorbed_checks_every_launch_before_the_first():
    # Without a GPU any launch attempt returns MX_ERR_LAUNCH, so a validation
    # code shows the call returned before enqueuing the first projection.
    lib = _lib.load()
    f = lib.mx_mla_decode_absorbed
    need = lib.mx_mla_decode_absorbed_workspace(32, 128, 4096)
    bad = ctypes.c_void_p(0x10008)
    # output projection invalid, absorption valid
    assert f(P, P, P, P, bad, P, 32, 128, 4096, 128, 128, 0.07, P, need, None) == _lib.MX_ERR_ALIGN  # W_UV
    assert f(P, P, P, P, P, bad, 32, 128, 4096, 128, 128, 0.07, P, need, None) == _lib.MX_ERR_ALIGN  # O
    assert f(P, P, P, P, P, P, 32, 128, 4096, 128, 4104, 0.07, P, need, None) == _lib.MX_ERR_SHAPE   # d_v
    # decode invalid, both projections valid
    assert f(P, P, bad, P, P, P, 32, 128, 4096, 128, 128, 0.07, P, need, None) == _lib.MX_ERR_ALIGN  # KV
    # a valid call gets as far as the runtime
    assert f(P, P, P, P, P, P, 32, 128, 4096, 128, 128, 0.07, P, need, None) == _lib.MX_ERR_LAUNCH


def test_gdn_block_v_choices():
    """The column-block widths the GDN/KDA kernels use (no GPU needed): within
    the workgroup limit (d_k*BV/64 <= 1024 threads), dividing d_v, and the
    measured choices for the reference and BASELINE shapes."""
    f = _lib.load().mx_gdn_decode_block_v
    assert f(64, 32, 128, 128) == 64      # BASELINE B64 Hv32 d128
    assert f(4, 64, 256, 256) == 64       # reference "large"
    assert f(1, 16, 256, 256) == 16       # reference qwen3_next_decode
    for B, H, dk, dv in ((1, 16, 512, 512), (1, 4, 64, 64), (8, 8, 512, 64), (2, 2, 64, 512)):
        bv = f(B, H, dk, dv)
        assert bv >= 16 and dv % bv == 0 and dk * bv // 64 <= 1024
    assert f(1, 16, 96, 128) == 0 and f(0, 16, 128, 128) == 0
