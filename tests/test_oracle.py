"""Pins the CPU oracle (oracle/composed.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a dropped term, a wrong
sign, a transposed operand, a missing scale, a wrong causal side) fails at least one of them:
  - known-answer vectors: torch float64 autograd of an independently written attention
    (tests/golden/golden.npz, made by tests/golden/make_golden.py);
  - central finite differences of the forward: every gradient formula against the forward;
  - closed forms: q = 0 gives uniform attention, s = 1 gives O = V, equal value rows give O = v
    and dQ = dK = 0;
  - invariants: sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i per (b, h); L >= row max; O in the
    convex hull of the value rows;
  - the planted-mistake test shows those invariants reject a backward with one term dropped;
    tests/test_oracle_mutants.py plants ten such mistakes in a numpy restatement and shows each
    fails at least one of these checks.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"


def golden_cases():
    data = np.load(GOLDEN)  # allow_pickle defaults to False
    keys = sorted({k.split("/")[0] for k in data.files})
    return data, keys


def parse(key):
    parts = dict((p[0], int(p[1:])) for p in key.split("_"))
    return parts["b"], parts["s"], parts["h"], parts["d"], bool(parts["c"])


def test_golden_fp64(orc):
    data, keys = golden_cases()
    assert len(keys) == 10
    for key in keys:
        b, s, h, d, causal = parse(key)
        qkv, w = data[f"{key}/qkv"], data[f"{key}/w"]
        scale = 1.0 / d ** 0.5
        out, lse = orc.qkv_forward(qkv, h, scale, causal, dtype=np.float64)
        grad = orc.qkv_backward(qkv, h, scale, causal, out, lse, w, dtype=np.float64)
        assert np.allclose(out, data[f"{key}/out"], rtol=0, atol=1e-12), key
        assert np.allclose(lse, data[f"{key}/lse"], rtol=0, atol=1e-12), key
        assert np.allclose(grad, data[f"{key}/grad"], rtol=0, atol=1e-11), key


def test_golden_fp32_band(orc):
    """The fp32 restatement within the reference's CPU band (1e-5 max-abs, tests/parity.rs:164)."""
    data, keys = golden_cases()
    for key in keys:
        b, s, h, d, causal = parse(key)
        qkv, w = data[f"{key}/qkv"], data[f"{key}/w"]
        scale = np.float32(1.0 / d ** 0.5)
        out, lse = orc.qkv_forward(qkv, h, scale, causal, dtype=np.float32)
        grad = orc.qkv_backward(qkv, h, scale, causal, out, lse, w, dtype=np.float32)
        assert orc.max_abs(out, data[f"{key}/out"]) < 1e-5, key
        assert orc.max_abs(grad, data[f"{key}/grad"]) < 1e-5, key
        assert orc.rel_fro(grad, data[f"{key}/grad"]) < 2e-6, key


@pytest.mark.parametrize("causal", [False, True])
def test_finite_differences(orc, causal):
    rng = np.random.default_rng(7)
    b, h, s, d = 1, 2, 6, 5
    q, k, v = (rng.standard_normal((b, h, s, d)) for _ in range(3))
    w = rng.standard_normal((b, h, s, d))
    scale = 0.37

    def loss(q_, k_, v_):
        o, _ = orc.forward(q_, k_, v_, scale, causal, dtype=np.float64)
        return float(np.sum(o * w))

    o, l_ = orc.forward(q, k, v, scale, causal, dtype=np.float64)
    dq, dk, dv = orc.backward(q, k, v, o, l_, w, scale, causal, dtype=np.float64)
    eps = 1e-6
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = {"q": q, "k": k, "v": v}
            args_m = dict(args_p)
            args_p[name], args_m[name] = xp, xm
            num[idx] = (loss(**{f"{n}_": a for n, a in args_p.items()})
                        - loss(**{f"{n}_": a for n, a in args_m.items()})) / (2 * eps)
        assert np.max(np.abs(num - g)) < 1e-7, name


@pytest.mark.parametrize("causal", [False, True])
def test_zero_queries_uniform(orc, causal):
    rng = np.random.default_rng(1)
    b, h, s, d = 2, 3, 11, 7
    q = np.zeros((b, h, s, d))
    k, v = rng.standard_normal((b, h, s, d)), rng.standard_normal((b, h, s, d))
    o, l_ = orc.forward(q, k, v, 0.5, causal, dtype=np.float64)
    for i in range(s):
        n = i + 1 if causal else s
        assert np.allclose(o[:, :, i], v[:, :, :n].mean(axis=2), atol=1e-13)
        assert np.allclose(l_[:, :, i], np.log(n), atol=1e-13)


def test_single_key(orc):
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((2, 2, 1, 8)) for _ in range(3))
    o, l_ = orc.forward(q, k, v, 0.25, False, dtype=np.float64)
    assert np.allclose(o, v, atol=1e-14)
    assert np.allclose(l_, 0.25 * np.sum(q * k, axis=-1), atol=1e-13)


def test_equal_value_rows(orc):
    rng = np.random.default_rng(3)
    b, h, s, d = 1, 2, 9, 6
    q, k = rng.standard_normal((b, h, s, d)), rng.standard_normal((b, h, s, d))
    v = np.broadcast_to(rng.standard_normal((b, h, 1, d)), (b, h, s, d)).copy()
    g = rng.standard_normal((b, h, s, d))
    o, l_ = orc.forward(q, k, v, 0.3, False, dtype=np.float64)
    assert np.allclose(o, v, atol=1e-13)
    dq, dk, dv = orc.backward(q, k, v, o, l_, g, 0.3, False, dtype=np.float64)
    assert np.max(np.abs(dq)) < 1e-12 and np.max(np.abs(dk)) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_invariants(orc, causal):
    rng = np.random.default_rng(4)
    b, h, s, d = 2, 2, 13, 8
    q, k, v, g = (rng.standard_normal((b, h, s, d)) for _ in range(4))
    scale = 0.4
    o, l_ = orc.forward(q, k, v, scale, causal, dtype=np.float64)
    dq, dk, dv = orc.backward(q, k, v, o, l_, g, scale, causal, dtype=np.float64)
    assert np.allclose(dk.sum(axis=2), 0, atol=1e-12)
    assert np.allclose(dv.sum(axis=2), g.sum(axis=2), atol=1e-12)
    sc = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if causal:
        sc = np.where(np.triu(np.ones((s, s), bool), 1), -np.inf, sc)
    assert np.all(l_ >= sc.max(axis=-1) - 1e-12)
    lo, hi = v.min(axis=2, keepdims=True), v.max(axis=2, keepdims=True)
    assert np.all(o >= lo - 1e-12) and np.all(o <= hi + 1e-12)


def test_planted_mistake_is_caught(orc):
    """A backward that drops D (dS = P o dP) violates sum_j dK_j = 0: the invariant test above
    would reject such an oracle."""
    rng = np.random.default_rng(5)
    b, h, s, d = 1, 1, 8, 4
    q, k, v, g = (rng.standard_normal((b, h, s, d)) for _ in range(4))
    scale = 0.5
    o, l_ = orc.forward(q, k, v, scale, False, dtype=np.float64)
    p = np.exp(np.einsum("bhid,bhjd->bhij", q, k) * scale - l_[..., None])
    dp = np.einsum("bhid,bhjd->bhij", g, v)
    dsum = np.sum(g * o, axis=-1, keepdims=True)
    ds_right = p * (dp - dsum)
    ds_wrong = p * dp
    dk_right = np.einsum("bhij,bhid->bhjd", ds_right, q) * scale
    dk_wrong = np.einsum("bhij,bhid->bhjd", ds_wrong, q) * scale
    _, dk, _ = orc.backward(q, k, v, o, l_, g, scale, False, dtype=np.float64)
    assert np.allclose(dk, dk_right, atol=1e-12)
    assert np.allclose(dk_right.sum(axis=2), 0, atol=1e-12)
    assert not np.allclose(dk_wrong.sum(axis=2), 0, atol=1e-6)


def test_fp32_vs_fp64_seeded(orc):
    """Config 1's shape through the fp32 restatement: within 2e-6 normwise of fp64."""
    rng = np.random.default_rng(11)
    q, k, v, g = (rng.standard_normal((2, 4, 128, 64)).astype(np.float32) for _ in range(4))
    for causal in (False, True):
        o64, l64 = orc.forward(q, k, v, 0.125, causal, dtype=np.float64)
        d64 = orc.backward(q, k, v, o64, l64, g, 0.125, causal, dtype=np.float64)
        o32, l32 = orc.forward(q, k, v, 0.125, causal, dtype=np.float32)
        d32 = orc.backward(q, k, v, o32, l32, g, 0.125, causal, dtype=np.float32)
        assert orc.rel_fro(o32, o64) < 2e-6
        for a, r in zip(d32, d64):
            assert orc.rel_fro(a, r) < 2e-6


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("s,causal", [(1, False), (97, False), (97, True), (200, True)])
def test_rows_equal_full_slices(orc, s, causal, dtype):
    """oracle_rows_f64 / _f32 (sampled rows without [s, s] buffers, for long sequences) give
    the full forward / backward's rows of the same precision bit for bit: O, L and dQ at query
    rows, dK and dV at key rows (first, last and random rows)."""
    rng = np.random.default_rng(s + causal)
    q, k, v, g = (rng.standard_normal((1, 1, s, 64)).astype(dtype) for _ in range(4))
    o, l_ = orc.forward(q, k, v, 0.125, causal, dtype=dtype)
    dq, dk, dv = orc.backward(q, k, v, o, l_, g, 0.125, causal, dtype=dtype)
    qi = np.unique(np.r_[0, s - 1, rng.integers(0, s, 7)])
    ki = np.unique(np.r_[0, s - 1, rng.integers(0, s, 5)])
    got = orc.rows(q[0, 0], k[0, 0], v[0, 0], g[0, 0], 0.125, causal, qi, ki, dtype=dtype)
    want = (o[0, 0][qi], l_[0, 0][qi], dq[0, 0][qi], dk[0, 0][ki], dv[0, 0][ki])
    for name, a, b in zip(("o", "l", "dq", "dk", "dv"), got, want):
        assert np.array_equal(a, b), name
    with pytest.raises(RuntimeError):
        orc.rows(q[0, 0], k[0, 0], v[0, 0], g[0, 0], 0.125, causal, [s], ki)


def test_gather_matches_strides(orc):
    rng = np.random.default_rng(6)
    storage = rng.standard_normal(4000).astype(np.float32)
    b, h, s, d = 2, 3, 5, 4
    sb, sh, ss = 600, 8, 100
    got = orc.gather(storage, 3, (b, h, s, d), (sb, sh, ss))
    want = np.empty((b, h, s, d), np.float32)
    for idx in np.ndindex(b, h, s, d):
        bi, hi, si, di = idx
        want[idx] = storage[3 + bi * sb + hi * sh + si * ss + di]
    assert np.array_equal(got, want)
    with pytest.raises(ValueError, match="outside its storage"):
        orc.gather(storage, 3, (b, h, s, d), (sb * 10, sh, ss))


def test_split_merge_heads(orc):
    x, _ = orc.closed_form_inputs(2, 5, 3, 8)
    q, k, v = orc.split_heads(x, 3)
    assert q.shape == (2, 3, 5, 8)
    assert np.array_equal(orc.merge_heads(q), x[:, :, :24])
    assert np.array_equal(orc.merge_heads(v), x[:, :, 48:])


# --- the scorer: every parity bar is an upper bound on these, so they are pinned by hand ------

def test_rel_fro_hand_computed(orc):
    """rel_fro = ||x - ref||_2 / ||ref||_2 (bench/compare.py:524-527) on cases computed by hand.
    A scorer that under-reports (squared norms, a max in place of the 2-norm, the norm of x in the
    denominator, an absolute instead of a relative figure) fails one of them."""
    ref = np.zeros(5)
    ref[0] = 3.0
    x = ref.copy()
    x[1] = 0.5
    assert orc.rel_fro(x, ref) == 0.5 / 3.0
    # ||(3, 4)|| = 5 against ||(6, 8)|| = 10, in any shape
    ref = np.array([[6.0, 0.0], [0.0, 8.0]])
    x = ref + np.array([[3.0, 0.0], [0.0, -4.0]])
    assert orc.rel_fro(x, ref) == 0.5
    assert orc.rel_fro(x.astype(np.float32), ref) == 0.5
    # the error of a uniform relative perturbation is that perturbation
    rng = np.random.default_rng(0)
    ref = rng.standard_normal((4, 7, 3))
    assert abs(orc.rel_fro(ref * (1 + 1e-3), ref) - 1e-3) < 1e-15
    assert orc.rel_fro(ref, ref) == 0.0
    # a zero reference: the absolute norm of the difference
    assert orc.rel_fro(np.array([3.0, 4.0]), np.zeros(2)) == 5.0


def test_max_abs_hand_computed(orc):
    ref = np.array([1.0, -2.0, 3.0])
    assert orc.max_abs(ref + np.array([0.25, -0.5, 0.125]), ref) == 0.5
    assert orc.max_abs(np.array([-1.0, -2.0, 3.0]), ref) == 2.0
    assert orc.max_abs(np.zeros(0), np.zeros(0)) == 0.0
