"""Python face of the CPU oracle -- TEST INFRASTRUCTURE, NOT THE PRODUCT.

Wraps liboracle.so (composed.c: the reference's composed attention, src/lib.rs:222-299,
restated in C, fp32 and fp64) with numpy, plus the reference's input recipes and its scoring
formula. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module; the operator under test never routes through it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile liboracle.so (make in this directory)."""
    res = subprocess.run(["make", "-B", "-C", str(ORACLE_DIR)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        i64, c_int = ctypes.c_int64, ctypes.c_int
        vp = ctypes.c_void_p
        for suffix, real in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
            f = getattr(L, f"oracle_forward_{suffix}")
            f.argtypes = [vp, vp, vp, i64, i64, i64, i64, real, c_int, vp, vp, c_int]
            f.restype = c_int
            f = getattr(L, f"oracle_backward_{suffix}")
            f.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, real, c_int, vp, vp, vp,
                          c_int]
            f.restype = c_int
            f = getattr(L, f"oracle_rows_{suffix}")
            f.argtypes = [vp, vp, vp, vp, i64, i64, real, c_int, vp, i64, vp, i64, vp, vp, vp,
                          vp, vp, c_int]
            f.restype = c_int
        L.oracle_gather_f32.argtypes = [vp, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp]
        L.oracle_gather_f32.restype = c_int
        _lib = L
    return _lib


def default_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return max(1, int(env))
    return max(1, min(16, os.cpu_count() or 1))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _prep(x, dtype):
    return np.ascontiguousarray(x, dtype=dtype)


def forward(q, k, v, scale: float, causal: bool, dtype=np.float32, threads: int | None = None):
    """composed_forward (src/lib.rs:241-259) on [b, h, s, d] arrays -> (O [b,h,s,d], L [b,h,s])."""
    q, k, v = (_prep(x, dtype) for x in (q, k, v))
    b, h, s, d = q.shape
    assert k.shape == q.shape and v.shape == q.shape
    o = np.empty_like(q)
    l_ = np.empty((b, h, s), dtype=dtype)
    suffix = "f32" if dtype == np.float32 else "f64"
    rc = getattr(lib(), f"oracle_forward_{suffix}")(
        _ptr(q), _ptr(k), _ptr(v), b, h, s, d, scale, int(causal), _ptr(o), _ptr(l_),
        threads or default_threads())
    if rc != 0:
        raise RuntimeError(f"oracle forward failed ({rc})")
    return o, l_


def backward(q, k, v, o, l_, d_o, scale: float, causal: bool, dtype=np.float32,
             threads: int | None = None):
    """composed_backward (src/lib.rs:271-299) -> (dQ, dK, dV), each [b, h, s, d]."""
    q, k, v, o, d_o = (_prep(x, dtype) for x in (q, k, v, o, d_o))
    l_ = _prep(l_, dtype)
    b, h, s, d = q.shape
    dq, dk, dv = (np.empty_like(q) for _ in range(3))
    suffix = "f32" if dtype == np.float32 else "f64"
    rc = getattr(lib(), f"oracle_backward_{suffix}")(
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(l_), _ptr(d_o), b, h, s, d, scale,
        int(causal), _ptr(dq), _ptr(dk), _ptr(dv), threads or default_threads())
    if rc != 0:
        raise RuntimeError(f"oracle backward failed ({rc})")
    return dq, dk, dv


def rows(q, k, v, d_o, scale: float, causal: bool, query_rows, key_rows, dtype=np.float64,
         threads: int | None = None):
    """One [s, d] slice at sampled rows, without [s, s] buffers (long sequences): (O, L, dQ)
    at `query_rows` and (dK, dV) at `key_rows`, equal bit for bit to the rows of forward /
    backward in the same precision (src/lib.rs:241-299)."""
    q, k, v, d_o = (_prep(x, dtype) for x in (q, k, v, d_o))
    s, d = q.shape
    ri = np.ascontiguousarray(query_rows, dtype=np.int64)
    ki = np.ascontiguousarray(key_rows, dtype=np.int64)
    o = np.empty((len(ri), d), dtype)
    l_ = np.empty(len(ri), dtype)
    dq = np.empty((len(ri), d), dtype)
    dk, dv = np.empty((len(ki), d), dtype), np.empty((len(ki), d), dtype)
    suffix = "f32" if dtype == np.float32 else "f64"
    rc = getattr(lib(), f"oracle_rows_{suffix}")(
        _ptr(q), _ptr(k), _ptr(v), _ptr(d_o), s, d, scale, int(causal), _ptr(ri), len(ri),
        _ptr(ki), len(ki), _ptr(o), _ptr(l_), _ptr(dq), _ptr(dk), _ptr(dv),
        threads or default_threads())
    if rc != 0:
        raise RuntimeError(f"oracle rows failed ({rc})")
    return o, l_, dq, dk, dv


def gather(storage, start: int, dims, strides):
    """gather_cpu (src/lib.rs:223-238): a strided [b, h, s, d] view of a flat f32 storage."""
    storage = _prep(storage, np.float32).reshape(-1)
    b, h, s, d = dims
    out = np.empty((b, h, s, d), dtype=np.float32)
    rc = lib().oracle_gather_f32(_ptr(storage), storage.size, start, b, h, s, d, *strides,
                                 _ptr(out))
    if rc != 0:
        raise ValueError("fused_attention: layout outside its storage")
    return out


# --- the qkv path, composed (src/lib.rs:511-523 forward, :581-588 backward) -----------------

def split_heads(qkv: np.ndarray, heads: int):
    """q, k, v [b, h, s, d] of a [b, s, 3 h d] projection (qkv_geometry, src/lib.rs:191-206)."""
    b, s, three_hd = qkv.shape
    hd = three_hd // 3
    d = hd // heads
    parts = [qkv[:, :, i * hd:(i + 1) * hd].reshape(b, s, heads, d).transpose(0, 2, 1, 3)
             for i in range(3)]
    return tuple(np.ascontiguousarray(p) for p in parts)


def merge_heads(x: np.ndarray) -> np.ndarray:
    """[b, h, s, d] -> [b, s, h d]."""
    b, h, s, d = x.shape
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3)).reshape(b, s, h * d)


def qkv_forward(qkv, heads, scale, causal, dtype=np.float32, threads=None):
    """(out [b, s, h d], L [b, h, s]) of the composed path on a qkv projection."""
    q, k, v = split_heads(np.asarray(qkv), heads)
    o, l_ = forward(q, k, v, scale, causal, dtype, threads)
    return merge_heads(o), l_


def qkv_backward(qkv, heads, scale, causal, out, l_, grad, dtype=np.float32, threads=None):
    """dqkv [b, s, 3 h d] of the composed path, given out [b, s, h d] and its gradient."""
    qkv = np.asarray(qkv)
    b, s, three_hd = qkv.shape
    d = three_hd // 3 // heads
    q, k, v = split_heads(qkv, heads)
    o = np.asarray(out).reshape(b, s, heads, d).transpose(0, 2, 1, 3)
    g = np.asarray(grad).reshape(b, s, heads, d).transpose(0, 2, 1, 3)
    dq, dk, dv = backward(q, k, v, o, l_, g, scale, causal, dtype, threads)
    return np.concatenate([merge_heads(dq), merge_heads(dk), merge_heads(dv)], axis=2)


# --- inputs and scoring ----------------------------------------------------------------------

def closed_form_inputs(b: int, s: int, h: int, d: int):
    """The reference tests' deterministic inputs (tests/parity.rs:126-138): qkv[i] =
    sin(i * 0.618034) * 1.5 and loss weights w[i] = cos(i * 0.414213), in f32 arithmetic."""
    i = np.arange(b * s * 3 * h * d, dtype=np.float32)
    x = (np.sin(i * np.float32(0.618034)) * np.float32(1.5)).astype(np.float32)
    j = np.arange(b * s * h * d, dtype=np.float32)
    w = np.cos(j * np.float32(0.414213)).astype(np.float32)
    return x.reshape(b, s, 3 * h * d), w.reshape(b, s, h * d)


def seeded_qkv_inputs(b: int, h: int, s: int, seed: int, d: int = 64):
    """The reference benchmark's inputs (bench/compare.py:496-503): a CPU torch generator
    seeded with `seed` draws qkv [b, s, 3 h d] then dout [b, s, h d], N(0, 1) fp32."""
    import torch
    g = torch.Generator().manual_seed(seed)
    hd = h * d
    qkv = torch.randn(b, s, 3 * hd, generator=g)
    dout = torch.randn(b, s, hd, generator=g)
    return qkv.numpy(), dout.numpy()


def rel_fro(x, ref) -> float:
    """Normwise relative error ||x - ref||_2 / ||ref||_2 (bench/compare.py:524-527)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref.ravel())
    num = np.linalg.norm((x - ref).ravel())
    return float(num / den) if den > 0 else float(num)


def max_abs(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(x - ref))) if x.size else 0.0
