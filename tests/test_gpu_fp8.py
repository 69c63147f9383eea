"""fp8 block-scaled GEMM parity on the GPU vs the CPU oracle (fp32 product
of the dequantised operands).  Bound: normwise <= 2e-2 (bf16 output); the
bit-exact KAT of mojo-matmul-fp8/ANALYSIS.md:91-112; scale linearity."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, import_submodule, load_golden
from oracle import fp8 as ofp8
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def as_fp8(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes, dtype=np.uint8)).view(torch.float8_e4m3fn)


def run(ops, a8, sa, b8, sb):
    c = ops.gemm_fp8_bs(a8.cuda(), sa.cuda(), b8.cuda(), sb.cuda())
    torch.cuda.synchronize()
    return c.cpu()


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def test_golden(ops):
    announce("fp8 golden 48x272x256")
    g = load_golden("gemm_fp8_48x272x256")
    c = run(ops, as_fp8(g["a"]), torch.from_numpy(g["sa"]), as_fp8(g["b"]), torch.from_numpy(g["sb"]))
    assert normwise_rel_err(c, g["c"]) <= TOL


@pytest.mark.parametrize("mnk", [(16, 16, 128), (48, 272, 256), (200, 176, 384), (512, 512, 1024),
                                 (1024, 2048, 512)])
def test_parity_vs_oracle(ops, mnk):
    m, n, k = mnk
    announce(f"fp8 {m}x{n}x{k}")
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k))
    c = run(ops, a8, sa, b8, sb)
    ref = ofp8.gemm_fp8_bs_ref(ofp8.fp8_tensor_codes(a8), sa.numpy(), ofp8.fp8_tensor_codes(b8), sb.numpy())
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"


@pytest.mark.parametrize("mnk", [(1, 7168, 4096), (16, 16, 128), (32, 4096, 7168), (5, 2064, 1152), (33, 512, 1024),
                                 (64, 2048, 7168), (48, 272, 640), (20, 4112, 2944), (256, 512, 4096), (130, 1024, 2048),
                                 (500, 1008, 1024), (512, 1024, 384)])
def test_small_m_path(ops, mnk):
    """M <= 64 (decode batches), or at most 64 tiles of 128x128 with
    M <= 512, runs the weight-streaming kernel: workgroups of 32 columns x
    32 or 64 rows, scale blocks split over the waves.  Single rows, N not a
    multiple of 32 (a last block 16 wide), fewer scale blocks than waves
    (K = 128), block counts that do not divide by the wave count, and both
    the one- and two-fragment (M > 32) variants."""
    m, n, k = mnk
    announce(f"fp8 small-M {m}x{n}x{k}")
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k))
    c = run(ops, a8, sa, b8, sb)
    ref = ofp8.gemm_fp8_bs_ref_torch(a8, sa, b8, sb)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"


@pytest.mark.parametrize("mnk", [(4096, 4096, 128), (4096, 4096, 384), (4000, 4352, 640), (4096, 4112, 256),
                                 (3072, 3072, 1024), (3000, 3056, 640)])
def test_large_tile_path(ops, mnk):
    """Shapes on the 256x256 kernel: >= 256 such tiles, or fewer when 128x128
    tiles would need more than 2.4 times the rounds of workgroups (3072^3:
    144 tiles against 576).  One scale block (fewer stages than the ring
    holds), an odd block count, ragged M and N (N = 4352 and 4112: a partial
    last column tile, and a last 128-column scale block only 16 wide)."""
    m, n, k = mnk
    announce(f"fp8 256-tile {m}x{n}x{k}")
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k))
    c = run(ops, a8, sa, b8, sb)
    ref = ofp8.gemm_fp8_bs_ref_torch(a8, sa, b8, sb)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"


@pytest.mark.parametrize("mnk", [(4096, 4096, 512), (2048, 2048, 1024)])
def test_scale_alignment(ops, mnk):
    """With K a multiple of 512 the kernels read the activation scales four
    blocks per 8-byte load when sA is 8-byte aligned; the interface asks
    only for 4-byte alignment, and an sA 4 bytes off an 8-byte boundary
    takes the one-scale-per-load path.  Both give the same bits."""
    m, n, k = mnk
    announce(f"fp8 sA alignment {m}x{n}x{k}")
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k))
    ad, bd, sbd = a8.cuda(), b8.cuda(), sb.cuda()
    sa_aligned = sa.cuda()
    buf = torch.empty(sa.numel() + 1, dtype=torch.float32, device="cuda")
    sa_off = buf[1:].view(sa.shape)
    sa_off.copy_(sa_aligned)
    assert sa_aligned.data_ptr() % 8 == 0 and sa_off.data_ptr() % 8 == 4
    c_aligned = ops.gemm_fp8_bs(ad, sa_aligned, bd, sbd)
    c_off = ops.gemm_fp8_bs(ad, sa_off, bd, sbd)
    torch.cuda.synchronize()
    assert torch.equal(c_aligned.view(torch.int16), c_off.view(torch.int16))
    ref = ofp8.gemm_fp8_bs_ref_torch(a8, sa, b8, sb)
    err = normwise_rel_err(c_off.cpu(), ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"


def test_bit_exact_kat(ops):
    """Operands that are multiples of 1/16 in [0, 0.9375] with unit scales: the
    fp32 sums are exact, so the bf16 output equals the bf16 rounding of the
    exact product (mojo-matmul-fp8/matmul_fp8.mojo:267-270)."""
    announce("fp8 bit-exact KAT")
    m, n, k = 128, 256, 512
    ia = (np.arange(m * k, dtype=np.uint64) * 2654435761 % 16).reshape(m, k)
    ib = ((np.arange(k * n, dtype=np.uint64) + 17) * 2654435761 % 16).reshape(k, n)
    a = (ia.astype(np.float32) * 0.0625)
    b = (ib.astype(np.float32) * 0.0625)
    ac, bc = ofp8.e4m3_encode(a), ofp8.e4m3_encode(b)
    sa = np.ones((m, k // 128), np.float32)
    sb = np.ones((k // 128, (n + 127) // 128), np.float32)
    c = run(ops, as_fp8(ac), torch.from_numpy(sa), as_fp8(bc), torch.from_numpy(sb)).float().numpy()
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c, bf16_round(exact))


def test_scale_linearity(ops):
    """Doubling one row of sA doubles that row of C exactly; uniform scales
    give (plain product) x constant."""
    announce("fp8 scale linearity")
    s = shapes.FP8GemmShape("t", 64, 256, 256)
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(s)
    c0 = run(ops, a8, sa, b8, sb).float()
    sa2 = sa.clone()
    sa2[5] *= 2.0
    c1 = run(ops, a8, sa2, b8, sb).float()
    assert torch.equal(c1[5], 2.0 * c0[5])
    assert torch.equal(c1[:5], c0[:5]) and torch.equal(c1[6:], c0[6:])


def test_target_size_sampled(ops):
    """8192^3 with N(0,1) block-quantised inputs: 128 cells vs fp64 sums of dequantised operands."""
    announce("fp8 8192^3 sampled")
    s = shapes.FP8_TARGET
    a8, sa, b8, sb = inputs.fp8_gemm_inputs(s)
    c = ops.gemm_fp8_bs(a8.cuda(), sa.cuda(), b8.cuda(), sb.cuda())
    torch.cuda.synchronize()
    rng = np.random.default_rng(inputs.SAMPLE_SEED)
    rows = rng.integers(0, s.m, size=128)
    cols = rng.integers(0, s.n, size=128)
    got = c[torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()].float().cpu().numpy()
    ad = ofp8.dequantize_blockwise(ofp8.fp8_tensor_codes(a8)[rows], sa.numpy()[rows], (1, 128)).astype(np.float64)
    bcodes = ofp8.fp8_tensor_codes(b8)
    ref = np.empty(len(rows))
    for i, (r, cc) in enumerate(zip(rows, cols)):
        bcol = ofp8.e4m3_decode(bcodes[:, cc]).astype(np.float64) * np.repeat(sb.numpy()[:, cc // 128], 128)
        ref[i] = float(ad[i] @ bcol)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL
