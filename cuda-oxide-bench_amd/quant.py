"""Host-side fp8 (OCP e4m3, torch.float8_e4m3fn) block quantiser for inputs.

Recipe (the producer of the fp8 GEMM operands): for each block,
    scale = amax(|x|) / 448          (1.0 for an all-zero block)
    q     = e4m3(round-to-nearest-even(x / scale)), saturated to +-448
so that x ~= q * scale.  Blocks are 1x128 for activations (A) and 128x128
for weights (B).  This runs on the host to build synthetic inputs; it is
not part of any timed kernel.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def quantize_fp8_blockwise(x: torch.Tensor, block: tuple[int, int]) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise a 2-D fp32 tensor; returns (q [R,C] float8_e4m3fn, scales [R/br, C/bc] fp32)."""
    if x.dim() != 2:
        raise ValueError("x must be 2-D")
    br, bc = block
    R, C = x.shape
    if R % br or C % bc:
        # pad to whole blocks with zeros, quantise, crop
        Rp, Cp = -(-R // br) * br, -(-C // bc) * bc
        xp = torch.zeros((Rp, Cp), dtype=torch.float32, device=x.device)
        xp[:R, :C] = x
        q, s = quantize_fp8_blockwise(xp, block)
        return q[:R, :C].contiguous(), s
    xf = x.float()
    blocks = xf.reshape(R // br, br, C // bc, bc)
    amax = blocks.abs().amax(dim=(1, 3))
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    y = blocks / scale[:, None, :, None]
    y = y.clamp(-E4M3_MAX, E4M3_MAX)
    q = y.reshape(R, C).to(torch.float8_e4m3fn)
    return q.contiguous(), scale.contiguous()


def dequantize_fp8_blockwise(q: torch.Tensor, scale: torch.Tensor, block: tuple[int, int]) -> torch.Tensor:
    br, bc = block
    R, C = q.shape
    s = scale.repeat_interleave(br, 0)[:R].repeat_interleave(bc, 1)[:, :C]
    return q.float() * s
