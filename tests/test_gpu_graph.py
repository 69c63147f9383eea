"""Every operator captured into a HIP graph and replayed: the library's
launches take their stream from the caller and launch kernels only (no
memset or copy nodes, no host synchronisation, workspace and outputs passed
in), so a captured call must reproduce the eager call exactly.  Each graph
is replayed three times; before every replay eager work refills the outputs
with NaN, and after it every output is compared with the eager result bit for
bit."""
from __future__ import annotations

import pytest
import torch

from conftest import announce, import_submodule

pytestmark = pytest.mark.gpu

_lib = import_submodule("_lib")
shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()])


def check_graph(name: str, launch, outs: list[torch.Tensor]) -> None:
    def clear():
        for o in outs:
            if o.dtype == torch.float8_e4m3fn:
                o.view(torch.uint8).fill_(0x7F)  # an e4m3 NaN
            else:
                o.fill_(float("nan"))

    clear()
    launch()
    torch.cuda.synchronize()
    ref = [_bits(o).clone() for o in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for r in range(3):
        clear()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, rf) in enumerate(zip(outs, ref)):
            assert torch.equal(_bits(o), rf), f"{name}: replay {r}, output {i} differs from the eager call"
    del g


def _cuda(*ts):
    return [t.cuda() for t in ts]


@pytest.mark.parametrize("mnk", [(1024, 1024, 1024), (200, 264, 520), (2048, 2048, 256), (16, 4096, 1024), (3072, 3072, 256)])
def test_gemm_bf16(ops, mnk):
    m, n, k = mnk
    announce(f"graph gemm_bf16 {m}x{n}x{k}")
    a, b = _cuda(*inputs.gemm_inputs(shapes.GemmShape("t", m, n, k)))
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    check_graph("gemm_bf16", lambda: ops.gemm_bf16(a, b, out=c), [c])


@pytest.mark.parametrize("bmnk", [(128, 32, 128, 512), (128, 32, 512, 128), (4, 100, 136, 72)])
def test_gemm_bf16_batched(ops, bmnk):
    nb, m, n, k = bmnk
    announce(f"graph gemm_bf16_batched {nb}x{m}x{n}x{k}")
    g = torch.Generator().manual_seed(nb + m + n + k)
    a = (torch.rand((nb, m, k), generator=g) * 2 - 1).to(torch.bfloat16).cuda()
    b = (torch.rand((nb, k, n), generator=g) * 2 - 1).to(torch.bfloat16).cuda()
    c = torch.empty((nb, m, n), dtype=torch.bfloat16, device="cuda")
    check_graph("gemm_bf16_batched", lambda: ops.gemm_bf16_batched(a, b, out=c), [c])


@pytest.mark.parametrize("mnk", [(512, 512, 1024), (32, 2048, 1024)])
def test_gemm_fp8(ops, mnk):
    m, n, k = mnk
    announce(f"graph gemm_fp8_bs {m}x{n}x{k}")
    a8, sa, b8, sb = _cuda(*inputs.fp8_gemm_inputs(shapes.FP8GemmShape("t", m, n, k)))
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    check_graph("gemm_fp8_bs", lambda: ops.gemm_fp8_bs(a8, sa, b8, sb, out=c), [c])


@pytest.mark.parametrize("causal", [True, False])
def test_gqa(ops, causal):
    announce(f"graph gqa B1 Hq8 Hkv2 S700 D128 causal={causal}")
    g = torch.Generator().manual_seed(7)
    q = torch.randn((1, 8, 700, 128), generator=g).to(torch.bfloat16).cuda()
    k = torch.randn((1, 2, 700, 128), generator=g).to(torch.bfloat16).cuda()
    v = torch.randn((1, 2, 700, 128), generator=g).to(torch.bfloat16).cuda()
    o = torch.empty_like(q)
    check_graph("gqa_fwd", lambda: ops.gqa_fwd(q, k, v, causal=causal, out=o), [o])


def test_mla_prefill(ops):
    announce("graph mla_prefill H4 S300 qk192 v128 causal")
    s = shapes.MLAShape("t", 1, 300, 4, 128, 64, 128, 512, True)
    q, k, v = _cuda(*inputs.mla_prefill_inputs(s, dtype=torch.bfloat16))
    o = torch.empty((1, 4, 300, 128), dtype=torch.bfloat16, device="cuda")
    check_graph("mla_prefill_fwd", lambda: ops.mla_prefill_fwd(q, k, v, causal=True, out=o), [o])


@pytest.mark.parametrize("bht", [(4, 128, 2048), (2, 16, 1)])
def test_mla_decode(ops, bht):
    B, H, T = bht
    announce(f"graph mla_decode B{B} H{H} T{T}")
    s = shapes.MLADecodeShape("t", B, H, T)
    q, kv = _cuda(*inputs.mla_inputs(s))
    ws = torch.empty(max(1, ops.mla_decode_workspace_bytes(B, H, T)), dtype=torch.uint8, device="cuda")
    o = torch.empty((B, H, 512), dtype=torch.bfloat16, device="cuda")
    check_graph("mla_decode", lambda: ops.mla_decode(q, kv, s.scale, out=o, workspace=ws), [o])


def test_mla_decode_noalloc(ops):
    """The allocation-free entry point, whose split partials live in the
    library's own device array: the graph's kernels address that array."""
    B, H, T = 4, 64, 1024
    announce(f"graph mla_decode_noalloc B{B} H{H} T{T}")
    lib = _lib.load()
    s = shapes.MLADecodeShape("t", B, H, T)
    q, kv = _cuda(*inputs.mla_inputs(s))
    o = torch.empty((B, H, 512), dtype=torch.bfloat16, device="cuda")

    def launch():
        rc = lib.mx_mla_decode_noalloc(q.data_ptr(), kv.data_ptr(), o.data_ptr(), B, H, T, 512, 64, s.scale,
                                       torch.cuda.current_stream().cuda_stream)
        assert rc == 0, _lib.strerror(rc)

    check_graph("mla_decode_noalloc", launch, [o])


def test_mla_absorbed(ops):
    announce("graph mla_decode_absorbed B4 H32 T700")
    s = shapes.MLADecodeShape("t", batch=4, n_h=32, ctx=700)
    _, kv = inputs.mla_inputs(s)
    kv = kv.cuda()
    d = {key: val.cuda() for key, val in inputs.mla_projection_inputs(s).items()}
    ws = torch.empty(ops.mla_decode_absorbed_workspace_bytes(4, 32, 700), dtype=torch.uint8, device="cuda")
    o = torch.empty((4, 32, d["w_uv"].shape[-1]), dtype=torch.bfloat16, device="cuda")
    check_graph("mla_decode_absorbed",
                lambda: ops.mla_decode_absorbed(d["q_nope"], d["q_rope"], kv, d["w_uk"], d["w_uv"], s.scale,
                                                out=o, workspace=ws), [o])


def test_gdn_decode(ops):
    announce("graph gdn_decode B3 Hk2 Hv4 dk128 dv256")
    x = {key: val.cuda() for key, val in
         inputs.gdn_inputs(shapes.GDNShape("t", batch=3, n_heads=4, d_k=128, d_v=256, n_k_heads=2)).items()}
    so = torch.empty_like(x["S_in"])
    o = torch.empty((3, 4, 256), dtype=x["v"].dtype, device="cuda")
    check_graph("gdn_decode", lambda: ops.gdn_decode(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["S_in"],
                                                     S_out=so, o=o), [o, so])


def test_kda_decode(ops):
    announce("graph kda_decode B2 H5 dk256 dv128")
    x = {key: val.cuda() for key, val in
         inputs.kda_inputs(shapes.KDAShape("t", batch=2, n_heads=5, d_k=256, d_v=128)).items()}
    so = torch.empty_like(x["S_in"])
    o = torch.empty((2, 5, 128), dtype=x["v"].dtype, device="cuda")
    check_graph("kda_decode", lambda: ops.kda_decode(x["q"], x["k"], x["v"], x["g"], x["beta"], x["S_in"],
                                                     S_out=so, o=o), [o, so])


def test_quant_fp8(ops):
    announce("graph quant_fp8_act 300x1024")
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((300, 1024), generator=g) * 4).to(torch.bfloat16).cuda()
    q = torch.empty((300, 1024), dtype=torch.float8_e4m3fn, device="cuda")
    sc = torch.empty((300, 8), dtype=torch.float32, device="cuda")
    check_graph("quant_fp8_act", lambda: ops.quant_fp8_act(x, q=q, scales=sc), [q, sc])
