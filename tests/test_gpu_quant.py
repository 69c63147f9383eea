"""fp8 activation quantisation on the GPU vs the CPU oracle's recipe
(oracle/fp8.py quantize_blockwise: amax/448 scale, RNE to e4m3fn, whose
codec is pinned against torch.float8_e4m3fn).  Bar: bit-exact codes and
scales (integer / byte output)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, import_submodule
from oracle import fp8 as ofp8
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu

inputs = import_submodule("inputs")
shapes = import_submodule("shapes")


def quant(ops, x):
    q, s = ops.quant_fp8_act(x.cuda())
    torch.cuda.synchronize()
    return q.view(torch.uint8).cpu().numpy(), s.cpu().numpy()


def expect(x):
    return ofp8.quantize_blockwise(x.float().numpy(), (1, 128))


@pytest.mark.parametrize("mk,dt", [((1, 128), torch.bfloat16), ((3, 384), torch.bfloat16), ((77, 1024), torch.float16),
                                   ((256, 2048), torch.bfloat16), ((1000, 640), torch.float16)])
def test_bit_exact_random(ops, mk, dt):
    m, k = mk
    announce(f"quant_fp8 {m}x{k} {dt}")
    g = torch.Generator().manual_seed(m * 7919 + k)
    x = (torch.randn((m, k), generator=g) * torch.exp(torch.randn((m, 1), generator=g) * 3)).to(dt)
    q, s = quant(ops, x)
    qe, se = expect(x)
    assert np.array_equal(s, se)
    assert np.array_equal(q, qe)


def test_edge_cases(ops):
    """Zero blocks (scale 1, code 0), a lone nonzero (-> +-448), exact e4m3
    midpoints after scaling (ties to even), values in the e4m3 subnormal
    range, and mixed signs."""
    announce("quant_fp8 edge cases")
    x = torch.zeros((6, 256), dtype=torch.float32)
    x[1, 5] = -3.0                                     # lone value: scale 3/448, code -448
    x[2, :128] = torch.linspace(-448, 448, 128)        # scale exactly 1
    # midpoints between adjacent e4m3 values with scale 1 (amax 448 at the end)
    pos = ofp8.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (pos[1:] + pos[:-1]) / 2
    x[3, :126] = torch.from_numpy(mids.astype(np.float32))
    x[3, 127] = 448.0
    x[4, 128:] = torch.from_numpy((np.arange(128) - 64) * 2.0 ** -12)  # tiny: subnormal e4m3 codes
    x[4, 200] = 448.0
    x[5] = torch.randn(256) * 1e-3
    for dt in (torch.bfloat16, torch.float16):
        xb = x.to(dt)
        q, s = quant(ops, xb)
        qe, se = expect(xb)
        assert np.array_equal(s, se) and np.array_equal(q, qe)
        assert s[0, 0] == 1.0 and s[0, 1] == 1.0 and not q[0].any()
        assert ofp8.e4m3_decode(q[1:2, 5])[0] == -448.0


def test_bit_exact_wide_range_and_near_midpoints(ops):
    """The kernel forms x/s as a reciprocal refinement (r = RN(1/s), q =
    RN(x r), q' = RN(q + (x - q s) r)) and keeps the plain division for
    blocks whose scale is below 2^-90 or above 2^100.  Both must give the
    host recipe's codes: rows over a wide exponent range (some on the
    plain-division side), and blocks whose values are bf16(t * s) for every
    e4m3 midpoint t, i.e. quotients within rounding distance of a code
    boundary under non-trivial scales, plus signed zeros."""
    announce("quant_fp8 wide range + near-midpoint blocks")
    g = torch.Generator().manual_seed(20261202)
    m, k = 1024, 4096
    x = torch.randn((m, k), generator=g) * torch.exp(torch.randn((m, 1), generator=g) * 6)
    x[::97] *= 1e-33                                   # scales < 2^-90: plain division
    pos = ofp8.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)  # 126 midpoints
    rng = np.random.default_rng(7)
    amax = torch.from_numpy(np.exp(rng.uniform(-40, 40, size=512)).astype(np.float32)).to(torch.bfloat16).float()
    blk = torch.zeros((512, 128))
    for i in range(512):
        sc = np.float32(amax[i].item()) / np.float32(448.0)
        vals = torch.from_numpy(mids * sc).to(torch.bfloat16).float()
        sign = torch.from_numpy(rng.choice([-1.0, 1.0], size=126).astype(np.float32))
        blk[i, :126] = vals * sign
        blk[i, 126] = -0.0 if i % 2 else 0.0            # signed zeros keep their sign: -0 -> code 0x80
        blk[i, 127] = amax[i]
    x[m - 512:, :128] = blk                             # 512 rows, first block each
    xb = x.to(torch.bfloat16)
    q, s = quant(ops, xb)
    qe, se = expect(xb)
    assert np.array_equal(s, se)
    bad = np.argwhere(q != qe)
    assert bad.size == 0, f"{len(bad)} code mismatches, first at {bad[:5].tolist()}"


def test_feeds_fp8_gemm(ops):
    """Device-quantised activations into the block-scaled fp8 GEMM equal the
    oracle GEMM of the same dequantised operands."""
    announce("quant_fp8 -> gemm_fp8_bs")
    m, n, k = 384, 512, 1024
    g = torch.Generator().manual_seed(5)
    a = torch.randn((m, k), generator=g).to(torch.bfloat16)
    _, _, b8, sb = inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k))
    q, s = ops.quant_fp8_act(a.cuda())
    c = ops.gemm_fp8_bs(q, s, b8.cuda(), sb.cuda())
    torch.cuda.synchronize()
    ref = ofp8.gemm_fp8_bs_ref(q.view(torch.uint8).cpu().numpy(), s.cpu().numpy(),
                               ofp8.fp8_tensor_codes(b8), sb.numpy())
    assert normwise_rel_err(c.float().cpu(), torch.from_numpy(ref)) <= 2e-2
    # and the dequantised A is close to the bf16 A it came from
    deq = ofp8.dequantize_blockwise(q.view(torch.uint8).cpu().numpy(), s.cpu().numpy(), (1, 128))
    assert np.abs(deq - a.float().numpy()).max() <= 0.07 * np.abs(a.float().numpy()).max()


def test_rejects_bad_k(ops):
    with pytest.raises(Exception):
        ops.quant_fp8_act(torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda"))


def _nan_codes_as_one(c):
    c = np.asarray(c, dtype=np.uint8).copy()
    c[(c & 0x7F) == 0x7F] = 0x7F
    return c


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_non_finite_blocks(ops, dt):
    """NaN and inf in the input, as the host recipe treats them: a block
    holding a NaN has scale 1 (inf in it clamps to +-448), a block with an
    infinite amax has scale inf (finite values -> +-0, infinities -> NaN);
    NaN codes compared as NaN whatever their sign bit."""
    announce(f"quant_fp8 non-finite {dt}")
    x = torch.randn((4, 512), generator=torch.Generator().manual_seed(8))
    x[0, 3] = float("nan")
    x[0, 200] = float("inf")
    x[1, 130] = float("-inf")
    x[1, 131] = float("nan")
    x[2, 300] = float("inf")
    x[2, 301] = float("-inf")
    x[3, 400] = -float("nan")
    x = x.to(dt)
    q, s = quant(ops, x)
    qe, se = expect(x)
    assert np.array_equal(s, se)
    assert np.array_equal(_nan_codes_as_one(q), _nan_codes_as_one(qe))
