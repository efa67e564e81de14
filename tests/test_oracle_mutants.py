"""Shows that the checks pinning the CPU oracle reject plausible mistakes.

`restate` is a numpy restatement of the composed path (src/lib.rs:240-299). Its unmutated form
must equal the C oracle (oracle/composed.c) and pass every check. Each MUTANT plants one mistake:
  - a dropped term;
  - a missing or wrong-signed scale;
  - a transposed or wrong operand;
  - the wrong causal side;
  - a wrong log-sum-exp.
Each must fail at least one of the checks the oracle passes in tests/test_oracle.py:
  - the golden vectors (torch fp64 autograd of an independent attention, tests/golden/golden.npz);
  - central finite differences of the restatement's own forward;
  - the invariants sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i.
Mistakes are planted here, in a CPU copy, never in the product.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"

MUTANTS = ["no_D", "dq_no_scale", "dk_no_scale", "dk_transposed", "dv_not_transposed",
           "dq_uses_v", "causal_side", "score_sign", "lse_no_log", "dp_uses_k"]


def restate(q, k, v, g, scale, causal, mutant=None):
    """(o, L, dq, dk, dv) for [b, h, s, d] inputs, float64, with at most one planted mistake."""
    s = q.shape[2]
    sc = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if mutant == "score_sign":
        sc = -sc
    if causal:
        mask = np.tril(np.ones((s, s), bool), -1) if mutant == "causal_side" else \
            np.triu(np.ones((s, s), bool), 1)
        sc = np.where(mask, -np.inf, sc)
    m = sc.max(axis=-1, keepdims=True)
    e = np.exp(sc - m)
    l_ = e.sum(axis=-1, keepdims=True)
    o = np.einsum("bhij,bhjd->bhid", e / l_, v)
    lse = (m + (l_ if mutant == "lse_no_log" else np.log(l_)))[..., 0]
    p = np.exp(sc - lse[..., None])
    dv = np.einsum("bhij,bhid->bhjd", p, g) if mutant != "dv_not_transposed" else \
        np.einsum("bhij,bhjd->bhid", p, g)
    dp = np.einsum("bhid,bhjd->bhij", g, k if mutant == "dp_uses_k" else v)
    dsum = np.sum(g * o, axis=-1, keepdims=True)
    ds = p * dp if mutant == "no_D" else p * (dp - dsum)
    dq = np.einsum("bhij,bhjd->bhid", ds, v if mutant == "dq_uses_v" else k)
    dq = dq if mutant == "dq_no_scale" else dq * scale
    dk = np.einsum("bhij,bhid->bhjd", ds, q) if mutant != "dk_transposed" else \
        np.einsum("bhij,bhjd->bhid", ds, q)
    dk = dk if mutant == "dk_no_scale" else dk * scale
    return o, lse, dq, dk, dv


def check_golden(orc, mutant):
    """Every golden case within 1e-9 of the torch fp64 autograd vectors."""
    data = np.load(GOLDEN)  # allow_pickle defaults to False
    for key in sorted({k.split("/")[0] for k in data.files}):
        parts = dict((p[0], int(p[1:])) for p in key.split("_"))
        h, d, causal = parts["h"], parts["d"], bool(parts["c"])
        qkv, w = data[f"{key}/qkv"].astype(np.float64), data[f"{key}/w"].astype(np.float64)
        q, k, v = (x.astype(np.float64) for x in orc.split_heads(qkv, h))
        b, s = qkv.shape[:2]
        g = w.reshape(b, s, h, d).transpose(0, 2, 1, 3)
        o, lse, dq, dk, dv = restate(q, k, v, g, 1.0 / d ** 0.5, causal, mutant)
        grad = np.concatenate([orc.merge_heads(x) for x in (dq, dk, dv)], axis=2)
        if not (np.allclose(orc.merge_heads(o), data[f"{key}/out"], rtol=0, atol=1e-9)
                and np.allclose(lse, data[f"{key}/lse"], rtol=0, atol=1e-9)
                and np.allclose(grad, data[f"{key}/grad"], rtol=0, atol=1e-9)):
            return False
    return True


def check_finite_differences(causal, mutant):
    """The restatement's gradients against central differences of its own forward."""
    rng = np.random.default_rng(7)
    b, h, s, d = 1, 1, 5, 3
    q, k, v, w = (rng.standard_normal((b, h, s, d)) for _ in range(4))
    scale = 0.37
    _, _, dq, dk, dv = restate(q, k, v, w, scale, causal, mutant)
    eps = 1e-6
    for i, (x, gr) in enumerate(((q, dq), (k, dk), (v, dv))):
        for idx in np.ndindex(x.shape):
            args_p, args_m = [q.copy(), k.copy(), v.copy()], [q.copy(), k.copy(), v.copy()]
            args_p[i][idx] += eps
            args_m[i][idx] -= eps
            fp = np.sum(restate(*args_p, w, scale, causal, mutant)[0] * w)
            fm = np.sum(restate(*args_m, w, scale, causal, mutant)[0] * w)
            if abs((fp - fm) / (2 * eps) - gr[idx]) > 1e-7:
                return False
    return True


def check_invariants(causal, mutant):
    rng = np.random.default_rng(4)
    b, h, s, d = 1, 2, 9, 4
    q, k, v, g = (rng.standard_normal((b, h, s, d)) for _ in range(4))
    _, _, _, dk, dv = restate(q, k, v, g, 0.4, causal, mutant)
    return bool(np.allclose(dk.sum(axis=2), 0, atol=1e-12)
                and np.allclose(dv.sum(axis=2), g.sum(axis=2), atol=1e-12))


def all_checks(orc, mutant):
    return {"golden": check_golden(orc, mutant),
            **{f"finite differences causal={c}": check_finite_differences(c, mutant)
               for c in (False, True)},
            **{f"invariants causal={c}": check_invariants(c, mutant) for c in (False, True)}}


def test_restatement_equals_oracle_and_passes(orc):
    """Unmutated: the numpy restatement equals the C oracle and passes every check."""
    rng = np.random.default_rng(9)
    q, k, v, g = (rng.standard_normal((2, 3, 11, 8)) for _ in range(4))
    for causal in (False, True):
        o, lse, dq, dk, dv = restate(q, k, v, g, 0.3, causal)
        ro, rl = orc.forward(q, k, v, 0.3, causal, dtype=np.float64)
        rdq, rdk, rdv = orc.backward(q, k, v, ro, rl, g, 0.3, causal, dtype=np.float64)
        for a, r in ((o, ro), (lse, rl), (dq, rdq), (dk, rdk), (dv, rdv)):
            assert np.allclose(a, r, rtol=0, atol=1e-12)
    checks = all_checks(orc, None)
    assert all(checks.values()), checks


@pytest.mark.parametrize("mutant", MUTANTS)
def test_mutant_is_rejected(orc, mutant):
    checks = all_checks(orc, mutant)
    assert not all(checks.values()), f"{mutant} passes every check: {checks}"
    print(mutant, "rejected by", [k for k, ok in checks.items() if not ok])
