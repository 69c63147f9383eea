"""The allocation-free MLA decode (mx_mla_decode_noalloc) through the C-ABI:
its output against mx_mla_decode's on the same inputs (same kernels, so
bit-identical bf16) and against the CPU oracle (normwise <= 2e-2), for two
calls in a row on one device, the second with a smaller problem, so the
second call runs over the partials the first left in the library's array."""
from __future__ import annotations

import pytest
import torch

from conftest import announce, import_submodule
from oracle import mla as omla
from oracle.metrics import normwise_rel_err

_lib = import_submodule("_lib")
shapes = import_submodule("shapes")
inputs = import_submodule("inputs")
TOL = 2e-2


def test_workspace_bound_fits_the_array():
    """The split policy keeps every workspace under the array's size (CPU)."""
    lib = _lib.load()
    cap = 128 << 20
    for B in (1, 2, 3, 8, 32, 64, 255, 1024):
        for H in (1, 16, 128, 129, 512, 2048):
            for T in (1, 64, 4096, 65536, 1 << 20):
                assert lib.mx_mla_decode_workspace(B, H, T, 512) <= cap


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(ops):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    # (B, H, T): the BASELINE shape first, then a smaller one with another split count
    for B, H, T in ((32, 128, 4096), (3, 20, 500)):
        announce(f"mla_decode_noalloc B{B} H{H} T{T}")
        s = shapes.MLADecodeShape("t", B, H, T)
        q, kv = inputs.mla_inputs(s, seed=inputs.SEED + B)
        qd, kvd = q.cuda(), kv.cuda()
        o_na = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device="cuda")
        rc = lib.mx_mla_decode_noalloc(qd.data_ptr(), kvd.data_ptr(), o_na.data_ptr(), B, H, T, 512, 64,
                                       s.scale, stream)
        assert rc == 0, _lib.strerror(rc)
        need = lib.mx_mla_decode_workspace(B, H, T, 512)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        o_ws = torch.empty((B, H, 512), dtype=torch.bfloat16, device="cuda")
        rc = lib.mx_mla_decode(qd.data_ptr(), kvd.data_ptr(), o_ws.data_ptr(), B, H, T, 512, 64, s.scale,
                               ws.data_ptr() if need else None, need, stream)
        assert rc == 0, _lib.strerror(rc)
        torch.cuda.synchronize()
        assert torch.equal(o_na.cpu().view(torch.int16), o_ws.cpu().view(torch.int16))
        ref = omla.mla_decode_ref(q, kv, s.scale, batches=list(range(min(B, 4))))
        err = normwise_rel_err(o_na.cpu()[:4], ref[:4])
        assert err <= TOL, f"normwise rel err {err:.3e}"


_FIRST_CALL_IN_CAPTURE = r'''
import importlib, math, sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import torch
from oracle import mla as omla
from oracle.metrics import normwise_rel_err
lib = importlib.import_module("cuda-oxide-bench_amd._lib").load()
shapes = importlib.import_module("cuda-oxide-bench_amd.shapes")
inputs = importlib.import_module("cuda-oxide-bench_amd.inputs")
B, H, T = 3, 20, 500
s = shapes.MLADecodeShape("t", B, H, T)
q, kv = inputs.mla_inputs(s, seed=inputs.SEED + 7)
qd, kvd = q.cuda(), kv.cuda()
o = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):  # the process's first MLA call: scratch lookup and kernel attributes inside the capture
    rc = lib.mx_mla_decode_noalloc(qd.data_ptr(), kvd.data_ptr(), o.data_ptr(), B, H, T, 512, 64, s.scale,
                                   torch.cuda.current_stream().cuda_stream)
assert rc == 0, rc
ref = omla.mla_decode_ref(q, kv, s.scale)
for r in range(3):
    o.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    err = normwise_rel_err(o.cpu(), ref)
    assert err <= 2e-2, (r, err)
    print(f"replay {r}: normwise rel err {err:.3e}", flush=True)
print("OK", flush=True)
'''


@pytest.mark.gpu
def test_noalloc_first_call_inside_graph_capture(tmp_path):
    """A fresh process whose first MLA call is mx_mla_decode_noalloc under
    HIP graph capture (the caller the entry point is for): the per-device
    scratch lookup and the kernels' LDS attributes run inside the capture,
    and every replay of the graph matches the oracle."""
    import subprocess
    import sys

    from conftest import REPO_ROOT

    announce("mla_decode_noalloc first call inside graph capture (subprocess)")
    script = tmp_path / "first_call_capture.py"
    script.write_text(_FIRST_CALL_IN_CAPTURE)
    proc = subprocess.run([sys.executable, str(script), str(REPO_ROOT)], capture_output=True, text=True,
                          timeout=240)
    print(proc.stdout[-2000:])
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-3000:]
    assert proc.stdout.strip().endswith("OK")
