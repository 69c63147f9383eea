"""fp8 e4m3 codec, block quantisation and the block-scaled GEMM oracle
(test infrastructure only).

The reference's fp8 GEMM is unscaled e4m3 x e4m3 -> f32 with a double
loop reference over the e4m3 values (mojo-matmul-fp8/matmul_fp8.mojo:339-361);
this path adds 1x128 / 128x128 fp32 block scales, so the oracle is the
fp32 matmul of the dequantised operands.  The e4m3 ("fn", OCP) codec is
written out here in numpy — decode table from the format definition,
encode by round-to-nearest-even against that table — so it can be pinned
against torch.float8_e4m3fn independently.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def e4m3_decode_table() -> np.ndarray:
    """float32 value of each of the 256 e4m3fn codes (NaN for 0x7f/0xff)."""
    vals = np.zeros(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals.astype(np.float32)


_TABLE = e4m3_decode_table()
_POS = _TABLE[:0x7F].astype(np.float64)  # codes 0..126: the non-negative finite values, ascending


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even encode of finite values already within +-448."""
    x = np.asarray(x, dtype=np.float64)
    mag = np.abs(x)
    if np.any(mag > E4M3_MAX):
        raise ValueError("e4m3_encode expects |x| <= 448")
    hi = np.searchsorted(_POS, mag, side="left")          # first value >= mag
    hi = np.clip(hi, 0, len(_POS) - 1)
    lo = np.clip(hi - 1, 0, len(_POS) - 1)
    d_hi = _POS[hi] - mag
    d_lo = mag - _POS[lo]
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    pick_hi |= (lo == hi)
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    # The sign bit is kept even when the magnitude rounds to zero (-0 is
    # 0x80), as torch.float8_e4m3fn and IEEE-style conversions do.
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def quantize_blockwise(x: np.ndarray, block: tuple[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Per-block amax/448 scaling then RNE to e4m3; returns (codes uint8, scales f32)."""
    x = np.asarray(x, dtype=np.float32)
    br, bc = block
    R, C = x.shape
    assert R % br == 0 and C % bc == 0
    blk = x.reshape(R // br, br, C // bc, bc)
    amax = np.abs(blk).max(axis=(1, 3))
    scale = np.where(amax > 0, amax / np.float32(E4M3_MAX), np.float32(1.0)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        y = (blk / scale[:, None, :, None]).astype(np.float32)
    y = np.clip(y, -E4M3_MAX, E4M3_MAX).reshape(R, C)
    # Non-finite inputs: a NaN amax fails `amax > 0` (scale 1), an infinite
    # one gives scale inf (finite values -> +-0, inf / inf -> NaN); NaN
    # stays NaN through the clip and takes the NaN code 0x7F.
    nan = np.isnan(y)
    codes = e4m3_encode(np.where(nan, 0.0, y))
    codes[nan] = 0x7F
    return codes, scale


def dequantize_blockwise(codes: np.ndarray, scale: np.ndarray, block: tuple[int, int]) -> np.ndarray:
    br, bc = block
    v = e4m3_decode(codes).astype(np.float32)
    s = np.repeat(np.repeat(scale, br, axis=0), bc, axis=1)[: v.shape[0], : v.shape[1]]
    return v * s


def gemm_fp8_bs_ref(a_codes: np.ndarray, sa: np.ndarray, b_codes: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """fp32 product of the dequantised operands (A blocks 1x128, B blocks 128x128)."""
    a = torch.from_numpy(dequantize_blockwise(a_codes, sa, (1, 128)))
    b = torch.from_numpy(dequantize_blockwise(b_codes, sb, (128, 128)))
    return (a @ b).numpy()


def gemm_fp8_bs_ref_torch(a8: torch.Tensor, sa: torch.Tensor, b8: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """gemm_fp8_bs_ref on torch.float8_e4m3fn tensors: the same dequantised
    fp32 operands (torch's exact e4m3 -> fp32 cast times the block scales)
    and the same fp32 product, without the numpy decode table, so it runs
    at 8192^3 in seconds (the bench's CPU baseline)."""
    a = a8.detach().cpu().to(torch.float32) * sa.detach().cpu().float().repeat_interleave(128, dim=1)
    n = b8.shape[1]
    sbf = sb.detach().cpu().float().repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)[:, :n]
    b = b8.detach().cpu().to(torch.float32) * sbf
    return a @ b


def fp8_tensor_codes(t: torch.Tensor) -> np.ndarray:
    """Raw uint8 codes of a torch.float8_e4m3fn tensor."""
    return t.detach().cpu().view(torch.uint8).numpy()
