"""Replay of fixture sets in the reference's inputs/ layout through the
harness cells (--inputs-dir): the committed golden sets are written out
under the reference's file names (gqa_/gdn_/kda_<name>_*.npy, f16 inputs,
f32 state and expected outputs) and each cell's correctness check runs on
them with the reference's gates."""
from __future__ import annotations

import importlib.util

import numpy as np
import pytest

from conftest import REPO_ROOT, announce, import_submodule, load_golden

pytestmark = pytest.mark.gpu
npy = import_submodule("npy")


def cell(name):
    path = REPO_ROOT / "cuda-oxide-bench_amd" / "cells" / name / "main.py"
    spec = importlib.util.spec_from_file_location(f"cell_{name.replace('-', '_')}", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def test_gqa_replay(ops, tmp_path):
    announce("fixture replay gqa_correctness")
    g = load_golden("gqa_correctness_f16")
    npy.save_fixture_set(tmp_path, "gqa", "correctness",
                         {"q": f16(g["q"]), "k": f16(g["k"]), "v": f16(g["v"]), "expected": g["o"]})
    assert cell("hip-attn-gqa").run_smoke(str(tmp_path), "correctness")


def test_gdn_replay(ops, tmp_path):
    announce("fixture replay gdn_correctness")
    g = load_golden("gdn_correctness_f16")
    # the reference stores the gates as f16 (pytorch_reference_gdn.py:220-221);
    # the golden gates come from the same f16 draw, so the f16 files are exact
    npy.save_fixture_set(tmp_path, "gdn", "correctness",
                         {"q": f16(g["q"]), "k": f16(g["k"]), "v": f16(g["v"]), "alpha": g["alpha"],
                          "beta": g["beta"], "S_in": g["S_in"], "o_expected": g["o"], "S_out_expected": g["S_out"]})
    fx = npy.load_fixture_set(tmp_path, "gdn", "correctness")
    assert fx["alpha"].dtype == np.float16
    assert cell("hip-attn-gdn").run_smoke(str(tmp_path), "correctness")


def test_kda_replay(ops, tmp_path):
    announce("fixture replay kda_correctness")
    g = load_golden("kda_correctness_f16")
    npy.save_fixture_set(tmp_path, "kda", "correctness",
                         {"q": f16(g["q"]), "k": f16(g["k"]), "v": f16(g["v"]), "g": f16(g["g"]),
                          "beta": f16(g["beta"]), "S_in": g["S_in"], "o_expected": g["o"],
                          "S_out_expected": g["S_out"]})
    assert cell("hip-attn-kda").run_smoke(str(tmp_path), "correctness")


def test_mla_prefill_replay(ops, tmp_path):
    announce("fixture replay mla_correctness_mla")
    g = load_golden("mla_prefill_correctness_f16")
    npy.save_fixture_set(tmp_path, "mla", "correctness_mla",
                         {"q": f16(g["q"]), "k": f16(g["k"]), "v": f16(g["v"]), "expected": g["o"]})
    assert cell("hip-attn-mla").run_prefill_smoke(str(tmp_path), "correctness_mla")


def test_missing_set_fails_loudly(ops, tmp_path):
    with pytest.raises(npy.NpyError):
        cell("hip-attn-gqa").run_smoke(str(tmp_path), "absent")
