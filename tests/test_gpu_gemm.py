"""bf16 GEMM parity on the GPU: HIP kernel vs the CPU oracle (fp32 matmul of
the bf16 operands, cutile-matmul-tc-bf16/main.py:98-107).  Bound: normwise
max|got-ref|/max|ref| <= 2e-2 (bf16 output), plus the reference harness's
own sampled gate |err| <= 0.2 + 0.05|ref| (:129-135) and exact KATs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, from_bits, import_submodule, load_golden
from oracle import gemm as ogemm
from oracle.metrics import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def run(ops, a, b):
    c = ops.gemm_bf16(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    return c.cpu()


def test_golden_fixture(ops):
    announce("gemm_bf16 golden 72x136x96")
    g = load_golden("gemm_bf16_72x136x96")
    a, b = from_bits(g["a"], torch.bfloat16), from_bits(g["b"], torch.bfloat16)
    c = run(ops, a, b)
    assert normwise_rel_err(c, g["c"]) <= 1e-2


@pytest.mark.parametrize("mnk", [(1, 8, 8), (16, 16, 32), (100, 136, 72), (257, 264, 520), (512, 512, 512),
                                 (1024, 1024, 1024), (2048, 1024, 512), (4096, 8192, 256)])
def test_parity_vs_oracle(ops, mnk):
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k}")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    # bf16 output: every element within a few bf16 ulps of the fp32 result
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


@pytest.mark.parametrize("mnk,path", [((64, 64, 4096), "one tile: weight streaming"),
                                      ((256, 1024, 2048), "64 tiles: weight streaming"),
                                      ((1024, 1024, 1024), "direct-load ring, 256 tiles (BASELINE configs[0])"),
                                      ((1024, 1024, 576), "K % 128 != 0: register-staged split-K path"),
                                      ((960, 1024, 512), "M % 64 == 0, 240 tiles: direct-load ring"),
                                      ((1024, 1024, 512), "direct-load ring, 4 K tiles per group"),
                                      ((768, 1024, 640), "direct-load ring, 5 K tiles per group, 192 tiles"),
                                      ((1024, 960, 768), "direct-load ring, 6 K tiles per group, 240 tiles"),
                                      ((512, 2048, 896), "direct-load ring, 7 K tiles per group"),
                                      ((1024, 1024, 1536), "direct-load ring, 12 K tiles per group"),
                                      ((512, 1024, 4096), "128 tiles, long K: direct-load ring")])
def test_small_grid_paths(ops, mnk, path):
    """Grids of at most one 64x64 tile per CU with K >= 512: at most 64
    tiles stream the weights; more, with whole tiles and 128-deep K chunks,
    run the direct-load ring (two K groups per workgroup summed through
    LDS; K tiles per group from fewer than the ring's 4 slots in flight to
    many more), other shapes the register-staged split-K kernel."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} ({path})")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


@pytest.mark.parametrize("mnk", [(1024, 1024, 1024), (768, 1024, 640), (1024, 1024, 1536)])
def test_small_grid_strided(ops, mnk):
    """Leading dimensions beyond the row lengths (lda > K, ldb > N,
    ldc > N) on the direct-load ring; C's padding columns are left
    untouched."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} strided")
    lib = import_submodule("_lib")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    pad = 72
    a_full = torch.zeros((m, k + pad), dtype=torch.bfloat16, device="cuda")
    b_full = torch.zeros((k, n + pad), dtype=torch.bfloat16, device="cuda")
    c_full = torch.full((m, n + pad), 7.0, dtype=torch.bfloat16, device="cuda")
    a_full[:, :k] = a.cuda()
    b_full[:, :n] = b.cuda()
    lib.call("mx_gemm_bf16", a_full.data_ptr(), b_full.data_ptr(), c_full.data_ptr(), m, n, k, k + pad, n + pad,
             n + pad, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    c = c_full.cpu()
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c[:, :n], ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c[:, :n].float() - ref).abs() <= 0.2 + 0.05 * ref.abs())
    assert torch.all(c[:, n:] == 7.0)


def test_reference_distribution_sampled_gate(ops):
    """The reference harness's own check at its smoke size: U[0,1) inputs,
    200 sampled cells, |err| <= 0.2 + 0.05|ref| (cutile-matmul-tc-bf16/main.py:110-135)."""
    announce("gemm_bf16 reference-dist 512 sampled")
    s = shapes.GEMM_SMOKE
    a, b = inputs.gemm_inputs(s, dist="reference")
    c = run(ops, a, b).float().numpy()
    rng = np.random.default_rng(inputs.SAMPLE_SEED)
    rows = rng.integers(0, s.m, size=200)
    cols = rng.integers(0, s.n, size=200)
    refs = ogemm.sample_reference(a, b, rows, cols)
    got = c[rows, cols]
    assert np.all(np.abs(got - refs) <= 0.2 + 0.05 * np.abs(refs))


@pytest.mark.parametrize("k", [64, 1024])
def test_kat_constant(ops, k):
    """A=1, B=1 -> K; A=2, B=3 -> 6K (oxide-gemm-sol/bench/cublas_correctness_test.py:8-11)."""
    announce(f"gemm_bf16 KAT constant K={k}")
    m = n = 256
    for av, bv, want in ((1.0, 1.0, k), (2.0, 3.0, 6 * k)):
        a = torch.full((m, k), av, dtype=torch.bfloat16)
        b = torch.full((k, n), bv, dtype=torch.bfloat16)
        c = run(ops, a, b)
        assert torch.all(c.float() == want)


def test_kat_pattern(ops):
    """A[i,:]=(i%8+1), B[:,j]=(j%8+1) -> (i%8+1)(j%8+1)K, exactly representable."""
    announce("gemm_bf16 KAT pattern")
    m, n, k = 384, 264, 128
    a = (torch.arange(m) % 8 + 1).float()[:, None].expand(m, k).to(torch.bfloat16).contiguous()
    b = (torch.arange(n) % 8 + 1).float()[None, :].expand(k, n).to(torch.bfloat16).contiguous()
    c = run(ops, a, b).float()
    want = ((torch.arange(m) % 8 + 1)[:, None] * (torch.arange(n) % 8 + 1)[None, :] * k).float()
    assert torch.equal(c, want)


@pytest.mark.parametrize("mnk", [(4096, 4096, 32), (4096, 4096, 96), (4000, 4040, 4128), (4096, 4352, 2048),
                                 (4096, 4096, 64), (4096, 4096, 192), (4000, 4040, 4096), (4096, 4096, 1600)])
def test_direct_load_path(ops, mnk):
    """Shapes that take the large-problem kernels (>= 256 tiles of 256x256):
    with K % 64 == 0 the split-ring kernel (whole 128-byte A lines), else
    the single ring (K % 32 == 0).  A single K tile or A block, fewer K
    tiles than ring slots, ragged M and N, and K-tile counts that are not a
    multiple of either ring's period."""
    m, n, k = mnk
    announce(f"gemm_bf16 direct-load {m}x{n}x{k}")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


def test_target_size_sampled(ops):
    """8192^3 (the roofline target): 256 cells against fp64 dot products."""
    announce("gemm_bf16 8192^3 sampled")
    s = shapes.GEMM_TARGET
    a, b = inputs.gemm_inputs(s)
    c = ops.gemm_bf16(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    rng = np.random.default_rng(inputs.SAMPLE_SEED)
    rows = rng.integers(0, s.m, size=256)
    cols = rng.integers(0, s.n, size=256)
    got = c[torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()].float().cpu().numpy()
    a32, b32 = a.float().numpy(), b.float().numpy()
    ref = np.array([ogemm.ref_elem(a32, b32, r, cc) for r, cc in zip(rows, cols)])
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() / scale <= TOL


@pytest.mark.parametrize("mnk,path", [((2048, 2048, 2048), "128x128 tiles, 64 K tiles"),
                                      ((2000, 2040, 2048), "ragged M and N"),
                                      ((2560, 2560, 1024), "400 tiles: two rounds of workgroups"),
                                      ((2048, 2048, 32), "one K tile, fewer than the ring's stages"),
                                      ((2048, 2048, 160), "five K tiles: only the loop tail"),
                                      ((2048, 4096, 1056), "33 K tiles: five ring periods and a tail of three"),
                                      ((4080, 2056, 256), "ragged, 544 tiles")])
def test_direct_load_128_paths(ops, mnk, path):
    """Mid-size GEMMs (at least one 128x128 tile per CU, fewer than one
    256x256 tile per CU, K % 32 == 0) run the direct-load 16x16x32 kernel on
    128x128 tiles with a 6-stage ring.  2048^3 is a size of the reference's
    mixed-dtype harness sweep (cutile-matmul-tiled-mixed/main.py:60)."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} direct-load 128x128 ({path})")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


@pytest.mark.parametrize("mnk", [(1, 7168, 4096), (16, 4096, 7168), (32, 256, 64), (33, 1000, 192), (64, 2048, 7168),
                                 (7, 296, 640), (48, 3000, 1344), (256, 512, 4096), (130, 1024, 2048),
                                 (1000, 96, 1024), (2048, 128, 4096), (96, 512, 8192)])
def test_weight_streaming_small_m(ops, mnk):
    """M <= 64 against at least 256 columns, or at most 64 tiles of 64x64
    with K >= 512, with whole 64-deep K blocks runs the weight-streaming
    kernel: single rows, one K block (fewer than the waves), the
    two-fragment variant (M > 32) and its chunks of 64 rows (a last chunk of
    2 or 40 rows), a last column block 8 or 24 wide, block counts that do
    not divide by the wave count."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} weight streaming")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


@pytest.mark.parametrize("mnk,path", [((3072, 3072, 1024), "144 tiles of 256x256 against 576 of 128x128"),
                                      ((3000, 3064, 512), "ragged, 144 tiles"),
                                      ((3584, 3584, 2048), "196 tiles against 784")])
def test_direct_load_256_below_one_tile_per_cu(ops, mnk, path):
    """Fewer than one 256x256 tile per CU still runs the 256x256 direct-load
    kernel when 128x128 tiles would need more than 2.6 times the rounds of
    workgroups."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} direct-load 256x256 ({path})")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


@pytest.mark.parametrize("mnk,path", [((2048, 2048, 2056), "register-staged 128x128 (tiles128 >= 256, K % 32 != 0)"),
                                      ((4096, 8192, 264), "register-staged 256x256 (tiles256 >= 512, K % 32 != 0)"),
                                      ((2048, 2048, 72), "register-staged 128x128, K tail of 8")])
def test_register_staged_paths(ops, mnk, path):
    """Single GEMMs whose K is not a multiple of 32 land on the
    register-staged 128x128 and 256x256 kernels (zero-filled K tail)."""
    m, n, k = mnk
    announce(f"gemm_bf16 {m}x{n}x{k} {path}")
    a, b = inputs.gemm_inputs(shapes.GemmShape("t", m, n, k))
    c = run(ops, a, b)
    ref = ogemm.gemm_ref(a, b)
    err = normwise_rel_err(c, ref)
    assert err <= TOL, f"normwise rel err {err:.3e}"
    assert torch.all((c.float() - ref).abs() <= 0.2 + 0.05 * ref.abs())


def test_rejects_bad_arguments(ops):
    a = torch.zeros((64, 60), dtype=torch.bfloat16, device="cuda")  # K % 8 != 0
    b = torch.zeros((60, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(Exception):
        ops.gemm_bf16(a, b)


@pytest.mark.parametrize("bmnk", [(1, 64, 64, 64), (7, 100, 136, 72), (128, 32, 512, 128), (128, 32, 128, 512), (16, 5, 40, 192),
                                  (3, 300, 264, 520), (4, 1024, 1024, 256),
                                  # split-K small-M kernel: 4, 8 and 12 chunks of K, 32 x 64 and 32 x 32
                                  # tiles, ragged M and N
                                  (8, 17, 72, 256), (64, 32, 136, 768), (200, 32, 128, 512), (3, 1, 8, 512)])
def test_batched_vs_oracle(ops, bmnk):
    """Strided-batched GEMM: every item against the fp32 oracle (small-M,
    its split-K variant for 4..12 chunks of K, 64x64 and, at 4 x
    1024x1024x256, the 128x128 register-staged kernel)."""
    nb, m, n, k = bmnk
    announce(f"gemm_bf16_batched {nb}x{m}x{n}x{k}")
    g = torch.Generator().manual_seed(nb * 131 + m)
    a = (torch.rand((nb, m, k), generator=g) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand((nb, k, n), generator=g) * 2 - 1).to(torch.bfloat16)
    c = ops.gemm_bf16_batched(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    c = c.cpu()
    for i in range(nb):
        ref = ogemm.gemm_ref(a[i], b[i])
        assert normwise_rel_err(c[i], ref) <= TOL
        assert torch.all((c[i].float() - ref).abs() <= 0.2 + 0.05 * ref.abs())
