"""Pin the fp8 oracle (CPU): the numpy e4m3 codec against torch.float8_e4m3fn,
the quantisation recipe, the bit-exact KAT and scale linearity."""
from __future__ import annotations

import numpy as np
import torch

from conftest import import_submodule
from oracle import fp8 as ofp8

quant = import_submodule("quant")


def test_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mine = ofp8.e4m3_decode_table()
    both_nan = np.isnan(codes) & np.isnan(mine)
    assert np.array_equal(codes[~both_nan], mine[~both_nan])
    assert np.array_equal(np.isnan(codes), np.isnan(mine))
    assert np.nanmax(mine) == 448.0 and np.nanmin(mine) == -448.0


def test_encode_matches_torch_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 40, 200000), rng.uniform(-448, 448, 200000),
                        rng.normal(0, 0.01, 50000)]).astype(np.float32)
    # include exact midpoints between neighbouring codes (ties to even)
    pos = ofp8.e4m3_decode_table()[:127].astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    # signed zeros and negative values that underflow to zero keep their sign
    tiny = np.array([0.0, -0.0, 1e-9, -1e-9, 2.0 ** -10, -(2.0 ** -10)], dtype=np.float32)
    x = np.concatenate([x, mids, -mids, pos.astype(np.float32), -pos.astype(np.float32), tiny])
    x = np.clip(x, -448, 448)
    t = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    mine = ofp8.e4m3_encode(x)
    assert np.array_equal(mine, t)  # codes, signed zeros included


def test_quantizers_agree():
    """The package's torch quantiser (input builder) and the oracle's numpy
    restatement produce identical codes and scales."""
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (256, 384)).astype(np.float32)
    x[:128, :128] = 0.0  # an all-zero block -> scale 1
    for block in ((1, 128), (128, 128)):
        q_t, s_t = quant.quantize_fp8_blockwise(torch.from_numpy(x), block)
        q_o, s_o = ofp8.quantize_blockwise(x, block)
        assert np.array_equal(s_t.numpy(), s_o)
        assert np.array_equal(ofp8.fp8_tensor_codes(q_t), q_o)


def test_quantization_error_bound():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (128, 256)).astype(np.float32)
    codes, s = ofp8.quantize_blockwise(x, (1, 128))
    back = ofp8.dequantize_blockwise(codes, s, (1, 128))
    # RNE to e4m3: at most half a step, i.e. 2^-4 relative for normals and
    # 2^-10 (half the subnormal step 2^-9) in units of the block scale.
    sfull = np.repeat(s, 128, axis=1)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2 ** -4 + sfull * 2 ** -10 + 1e-7)


def test_bit_exact_kat_oracle():
    """mojo-matmul-fp8/ANALYSIS.md:91-112: multiples of 1/16 sum exactly."""
    m, n, k = 16, 32, 256
    ia = (np.arange(m * k, dtype=np.uint64) * 2654435761 % 16).reshape(m, k)
    ib = ((np.arange(k * n, dtype=np.uint64) + 17) * 2654435761 % 16).reshape(k, n)
    a, b = ia.astype(np.float32) / 16, ib.astype(np.float32) / 16
    ac, bc = ofp8.e4m3_encode(a), ofp8.e4m3_encode(b)
    assert np.array_equal(ofp8.e4m3_decode(ac), a)
    c = ofp8.gemm_fp8_bs_ref(ac, np.ones((m, 2), np.float32), bc, np.ones((2, 1), np.float32))
    assert np.array_equal(c, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))


def test_scale_linearity_oracle():
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1, (8, 256)).astype(np.float32)
    b = rng.normal(0, 1, (256, 128)).astype(np.float32)
    ac, sa = ofp8.quantize_blockwise(a, (1, 128))
    bc, sb = ofp8.quantize_blockwise(b, (128, 128))
    c0 = ofp8.gemm_fp8_bs_ref(ac, sa, bc, sb)
    sa2 = sa.copy()
    sa2[3] *= 4.0
    c1 = ofp8.gemm_fp8_bs_ref(ac, sa2, bc, sb)
    assert np.allclose(c1[3], 4 * c0[3], rtol=1e-6, atol=1e-6)
    # only e4m3 quantisation noise separates it from the exact fp32 product
    assert np.abs(c0 - a @ b).max() / np.abs(a @ b).max() < 5e-2


def test_torch_dequant_reference_matches_numpy_table():
    # The bench's CPU baseline uses the torch form of the dequantised product:
    # it must give the same fp32 result as the table-driven numpy oracle
    # (identical dequantised operands, one fp32 matmul), ragged N included.
    g = torch.Generator().manual_seed(11)
    a = torch.randn((40, 384), generator=g)
    b = torch.randn((384, 200), generator=g)
    a8, sa = quant.quantize_fp8_blockwise(a, (1, 128))
    b8, sb = quant.quantize_fp8_blockwise(b, (128, 128))
    ref = ofp8.gemm_fp8_bs_ref(ofp8.fp8_tensor_codes(a8), sa.numpy(), ofp8.fp8_tensor_codes(b8), sb.numpy())
    got = ofp8.gemm_fp8_bs_ref_torch(a8, sa, b8, sb).numpy()
    assert np.array_equal(got, ref)


def _nan_codes_as_one(c):
    c = np.asarray(c, dtype=np.uint8).copy()
    c[(c & 0x7F) == 0x7F] = 0x7F
    return c


def test_non_finite_blocks_follow_the_torch_recipe():
    # A NaN in a block makes its scale 1 (NaN amax is not > 0); an infinite
    # amax makes it inf (finite values -> +-0, inf -> NaN).  The oracle must
    # agree with the package's torch quantiser, whose e4m3 cast is torch's.
    x = np.random.default_rng(5).standard_normal((4, 384)).astype(np.float32)
    x[0, 3] = np.nan
    x[0, 200] = np.inf            # block 1 of row 0: inf amax
    x[1, 130] = -np.inf
    x[1, 131] = np.nan            # NaN and inf in one block: scale 1, inf -> -448
    x[2, 300] = np.inf
    x[2, 301] = -np.inf           # inf and -inf: both NaN, the rest +-0
    codes, scales = ofp8.quantize_blockwise(x, (1, 128))
    tq, ts = quant.quantize_fp8_blockwise(torch.from_numpy(x), (1, 128))
    assert np.array_equal(scales, ts.numpy())
    assert np.array_equal(_nan_codes_as_one(codes), _nan_codes_as_one(tq.view(torch.uint8).numpy()))
    assert scales[0, 0] == 1.0 and scales[0, 1] == np.inf and scales[1, 1] == 1.0
    assert codes[1, 130] == 0xFE  # -inf / 1 clipped to -448
    assert codes[0, 3] == 0x7F and codes[0, 200] == 0x7F
