"""The comparison harness (candle_fused_attn.compare): its pure helpers (doctests) and the report
renderer on the CPU; one small end-to-end run on the GPU."""
from __future__ import annotations

import doctest
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

from candle_fused_attn import compare

PKG = Path(__file__).resolve().parent.parent / "candle-fused-attn_amd"


def test_helpers_doctests():
    res = doctest.testmod(compare, verbose=False)
    assert res.attempted >= 12 and res.failed == 0


def test_decision_rule_needs_separated_rounds():
    assert compare.verdict("x", [1.0, 1.1, 1.2], "y", [1.25, 1.3]) == "x faster (x1.16)"
    assert compare.verdict("x", [1.0, 1.3], "y", [1.25, 1.4]) == "not separated"


def test_render_synthetic_report():
    wall = {"a": {"fwd": [0.1, 0.11], "train": [0.3, 0.31], "net": [0.2, 0.21]},
            "b": {"fwd": [0.2, 0.22], "train": [0.6, 0.62], "net": [0.5, 0.52]},
            "head": {"head": [0.1, 0.1]}}
    err = {p: {"rel_fro": 1e-7, "max_abs": 1e-6} for p in compare.PARTS}
    rep = {"env": {"date": "d", "shape": [2, 2, 64, 64], "causal": False, "seed": 0,
                   "timing": {}},
           "device": {"gpu": "g", "arch": "gfx950", "cus": 256, "torch": "t", "hip": "h",
                      "fp32_matmul_precision": "highest"},
           "status": {"a": "ok", "b": "ok", "c": "refused: no kernel"},
           "deterministic": {"a": True, "b": False},
           "accuracy": {"fp64_rounded_to_fp32": err, "a": err, "b": err}, "wall": wall,
           "kernels": {"a:fwd": {"ms": 0.05, "kernels": [], "irregular": []},
                       "a:train": {"ms": 0.2, "kernels": [{"name": "void k(int)", "per_call": 1.0,
                                                           "us_per_call": 150.0}],
                                   "irregular": ["void fill(int)"]},
                       "b:fwd": {"ms": 0.1, "kernels": [], "irregular": []},
                       "b:train": {"ms": 0.5, "kernels": [], "irregular": []},
                       "head:head": {"ms": 0.01, "kernels": [], "irregular": []}}}
    md = compare.render(rep, ["a", "b"])
    assert "a faster (x2.00)" in md and "refused: no kernel" in md
    assert "| a | 0.050 | 0.200 | 0.190 | fill |" in md
    assert "k ×1 150.0" in md


@pytest.mark.gpu
def test_harness_end_to_end(tmp_path):
    out = tmp_path / "cmp"
    env = dict(os.environ)
    env["PYTHONPATH"] = str(PKG) + os.pathsep + env.get("PYTHONPATH", "")
    print("harness run b2 h2 s64", flush=True)
    subprocess.run([sys.executable, "-m", "candle_fused_attn.compare", "run", "--out", str(out),
                    "--batch", "2", "--heads", "2", "--seq", "64", "--rounds", "2",
                    "--samples", "2", "--calls", "2", "--warmup", "1"],
                   check=True, env=env, timeout=300)
    rep = json.loads((out / "report.json").read_text())
    assert rep["status"]["fattn_qkv"] == "ok" and rep["status"]["fattn_general"] == "ok"
    assert rep["deterministic"]["fattn_qkv"] and rep["deterministic"]["fattn_general"]
    for name in ("fattn_qkv", "fattn_general"):
        for p in compare.PARTS:
            assert rep["accuracy"][name][p]["rel_fro"] <= 2e-6, (name, p)
    assert (out / "report.md").read_text().startswith("# fused attention vs PyTorch-ROCm")
