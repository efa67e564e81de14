"""The head-to-head harness (candle_fused_attn.compare): its statistics, decision rule, profiler
parsing and report on the CPU; one small end-to-end report on the GPU."""
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


def test_doctests():
    res = doctest.testmod(compare, verbose=False)
    assert res.attempted >= 15 and res.failed == 0


def test_latin_square_rows_cover_every_position():
    names = ["a", "b", "c", "d", "e"]
    rows = [compare.latin_row(names, r) for r in range(len(names))]
    for pos in range(len(names)):
        assert sorted(row[pos] for row in rows) == names
    for row in rows:
        assert sorted(row) == names


def test_paired_rule_is_antisymmetric_and_needs_every_round():
    a, b = [1.0, 2.0, 3.0], [1.5, 2.5, 3.5]
    assert compare.paired_rule(a, b) == -1 and compare.paired_rule(b, a) == 1
    # one round the other way round: no separation, however large the other margins
    assert compare.paired_rule([1.0, 1.0, 9.0], [5.0, 5.0, 5.0]) == 0
    with pytest.raises(ValueError):
        compare.paired_rule([1.0], [1.0, 2.0])


def test_reference64_matches_a_direct_loop():
    """The float64 recompute against a per-head loop with explicit softmax and hand-written
    gradients (dV = P^T dO, dP = dO V^T, dS = P o (dP - rowsum(dO o O)), dQ = dS K s, dK = dS^T Q s)."""
    import torch
    g = torch.Generator().manual_seed(4)
    b, s, h, d, scale = 2, 9, 2, 64, 0.3
    qkv = torch.randn(b, s, 3 * h * d, generator=g)
    dout = torch.randn(b, s, h * d, generator=g)
    for causal in (False, True):
        ref = compare.reference64(qkv, dout, h, scale, causal)
        x = qkv.double().view(b, s, 3, h, d)
        go = dout.double().view(b, s, h, d)
        for bi in range(b):
            for hi in range(h):
                q, k, v = x[bi, :, 0, hi], x[bi, :, 1, hi], x[bi, :, 2, hi]
                z = q @ k.T * scale
                if causal:
                    z = z + torch.full((s, s), float("-inf"), dtype=torch.float64).triu(1)
                p = torch.softmax(z, dim=-1)
                o = p @ v
                do = go[bi, :, hi]
                ds = p * (do @ v.T - (do * o).sum(-1, keepdim=True))
                want = {"o": o, "dq": ds @ k * scale, "dk": ds.T @ q * scale, "dv": p.T @ do}
                for part, w in want.items():
                    got = ref[part].view(b, s, h, d)[bi, :, hi]
                    assert torch.allclose(got, w, rtol=0, atol=1e-12), (causal, part)


def test_agreement_measures_a_known_perturbation():
    import torch
    ref = {p: torch.zeros(2, 3, dtype=torch.float64) for p in compare.PARTS}
    for p in compare.PARTS:
        ref[p][0, 0] = 4.0
    got = {p: ref[p].clone() for p in compare.PARTS}
    got["dk"][1, 2] = 1.0                 # ||(0, 1)|| / ||(4)|| = 0.25
    e = compare.agreement(got, ref)
    assert e["dk"] == {"rel": 0.25, "max_abs": 1.0}
    assert e["o"] == {"rel": 0.0, "max_abs": 0.0}


def test_render_from_a_synthetic_result():
    err = {p: {"rel": 3e-7, "max_abs": 2e-6} for p in compare.PARTS}
    rep = {"setup": {"device": "gpu", "b": 2, "h": 2, "s": 64, "d": 64, "seed": 0,
                     "scale": 0.125, "causal": False, "when": "now", "torch": "t", "hip": "h",
                     "matmul_precision": "highest"},
           "status": {"fattn.qkv": "ran", "sdpa.math": "ran", "sdpa.flash": "refused: fp32"},
           "what": {"fattn.qkv": "ours", "sdpa.math": "math", "sdpa.flash": "flash"},
           "rerun_equal": {"fattn.qkv": True, "sdpa.math": False},
           "agreement": {"float64 rounded to fp32": err, "fattn.qkv": err, "sdpa.math": err},
           "timing": {"rounds": 2, "reps": 3, "calls": 4, "warmup": 1,
                      "ms": {"fattn.qkv": {"fwd": [0.1, 0.11], "step": [0.3, 0.31]},
                             "sdpa.math": {"fwd": [0.2, 0.22], "step": [0.9, 0.93]}}},
           "kernel_calls": 4, "kernel_skip": 2,
           "kernels": {"fattn.qkv:step": {"ms": 0.25, "other": ["fillBuffer"], "kernels": [
               {"name": "void ns::bwd_split_kernel<64>(BwdArgs)", "per_call": 1, "us": 140.0}]},
               "sdpa.math:fwd": None}}
    md = compare.render(rep)
    assert md.startswith("# fused attention vs PyTorch-ROCm fp32 attention on gpu")
    assert "refused: fp32" in md
    assert "| fattn.qkv | sdpa.math | fattn.qkv ahead, 2.00x | fattn.qkv ahead, 3.00x |" in md
    assert "bwd_split_kernel<64> x1 140.0" in md and "| sdpa.math | fwd | n/a |" in md
    assert "| fattn.qkv | 3.00e-07 / 2.0e-06" in md


@pytest.mark.gpu
def test_report_end_to_end(tmp_path):
    out = tmp_path / "cmp"
    env = dict(os.environ)
    env["PYTHONPATH"] = str(PKG) + os.pathsep + env.get("PYTHONPATH", "")
    print("compare report b2 h2 s64", flush=True)
    subprocess.run([sys.executable, "-m", "candle_fused_attn.compare", "report", "--out",
                    str(out), "--batch", "2", "--heads", "2", "--seq", "64", "--rounds", "2",
                    "--reps", "2", "--calls", "2", "--warmup", "1"],
                   check=True, env=env, timeout=300)
    rep = json.loads((out / "report.json").read_text())
    for name in compare.MINE:
        assert rep["status"][name] == "ran" and rep["rerun_equal"][name], name
        for p in compare.PARTS:
            assert rep["agreement"][name][p]["rel"] <= 2e-6, (name, p)
    assert len(rep["timing"]["ms"]["fattn.qkv"]["step"]) == 2
    assert (out / "report.md").read_text().startswith("# fused attention vs PyTorch-ROCm")
