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
