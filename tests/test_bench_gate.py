"""bench.py's parity gate, on the CPU: a case whose output misses its bound
against the oracle reports no numbers (the reference's rule that a kernel
failing its correctness check publishes no TFLOPS,
analysis/wave15-attention-architecture/reference/README.md:47-58).  The
"GPU output" here is the oracle's own result on a small shape, and the
mistake is planted in the reference side of the comparison."""
from __future__ import annotations

import importlib.util
import json

import pytest
import torch

from conftest import REPO_ROOT, import_submodule
from oracle import gqa as ogqa

shapes = import_submodule("shapes")
inputs = import_submodule("inputs")


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", REPO_ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _gqa_record(bench, reference):
    s = shapes.GQAShape("t", 1, 64, 4, 2, 64, True)
    q, k, v = inputs.gqa_inputs(s)
    got = ogqa.gqa_naive(q, k, v, causal=True)
    rec = {"workload": "gqa test", "unit": "TFLOPS", "mean_ms": 1.0, "wall_ms": 1.0, "flops": 1e9, "value": 1.0,
           "tflops_reference_convention": 2.0, "shape": s,
           "roofline": {"bound": "mfma", "achieved": 1.0, "peak": 2500.0, "unit": "TFLOP/s", "frac": 4e-4}}
    rec["cpu_baseline"] = bench.cpu_leg(lambda: reference(q, k, v), 1e9, "TFLOPS", "test sample", got=got)
    bench.parity_record(None, rec, lambda: pytest.fail("the CPU leg's comparison must be used"))
    return rec


def test_correct_reference_reports(bench, capsys):
    rec = _gqa_record(bench, lambda q, k, v: ogqa.gqa_naive(q, k, v, causal=True))
    assert rec["parity"]["output_normwise"] == 0.0
    assert bench.emit({"gqa": rec}, ["gqa"], 3, 1, lambda f, ms: f / ms / 1e9) == 0
    line = json.loads(capsys.readouterr().out.strip())
    assert line["value"] > 0 and line["parity"]["output_normwise"] == 0.0


def test_wrong_reference_refuses_to_report(bench, capsys):
    # planted mistake: the reference drops the causal mask
    rec = _gqa_record(bench, lambda q, k, v: ogqa.gqa_naive(q, k, v, causal=False))
    assert rec["parity"]["output_normwise"] > bench.OUT_BOUND
    assert bench.emit({"gqa": rec}, ["gqa"], 3, 1, lambda f, ms: f / ms / 1e9) == 3
    assert capsys.readouterr().out == ""


@pytest.mark.parametrize("parity,ok", [
    ({"output_normwise": 1e-3, "state_normwise": 5e-4}, True),
    ({"output_normwise": 1e-3, "state_normwise": 2e-3}, False),   # fp32 state bound 1e-3
    ({"output_normwise": 3e-2}, False),
    ({"output_normwise": float("nan")}, False),
    ({"bit_exact": True}, True),
    ({"bit_exact": False}, False),
    ({}, False),                                                  # a check that measured nothing
    (None, False),                                                # no check at all
])
def test_parity_failures(bench, parity, ok):
    rec = {} if parity is None else {"parity": parity}
    assert (bench.parity_failures({"case": rec}) == []) == ok


def test_rotation_exceeds_the_infinity_cache(bench):
    for set_bytes in (67 << 20, 135 << 20, 160 << 20, 203 << 20, 270 << 20, 1 << 30):
        r = bench.rotation_count(set_bytes)
        assert r >= 2 and (r - 1) * set_bytes >= 1.5 * bench.MALL_BYTES
        assert (r - 2) * set_bytes < 1.5 * bench.MALL_BYTES or r == 2
