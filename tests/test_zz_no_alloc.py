"""fattn_bwd_f32_noalloc (the backward with the library's static scratch as its workspace) against
fattn_bwd_f32 with a caller's workspace of the scratch's size, FATTN_STATIC_SCRATCH_BYTES (so the
same way of summing dQ: the whole split when it fits, else the split by chunks of (b, h) at
d <= 64, else turns): bit-identical dQ, dK, dV on two calls in a row, the second on a smaller
shape, causal and not, the first and last (b, h) pair of every call against the fp64 oracle
(normwise 2e-6, as every parity test), and the refusal of a shape whose minimum workspace exceeds
the scratch (before any launch)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from candle_fused_attn import _lib

pytestmark = pytest.mark.gpu

STATIC_SCRATCH = 64 << 20  # FATTN_STATIC_SCRATCH_BYTES (include/fattn.h)
REL_TOL = 2e-6             # normwise, vs fp64


def say(*a):
    print(*a, flush=True)


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def backward_both(b, h, s, d, causal, seed, dev):
    """(dqkv from fattn_bwd_f32_noalloc, dqkv from fattn_bwd_f32 with a workspace of the same
    kind, the kind, (qkv, dout, O)) for seeded N(0, 1) qkv and output gradient."""
    L = _lib.lib()
    rng = np.random.default_rng(seed)
    qkv = torch.from_numpy(rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)).to(dev)
    dout = torch.from_numpy(rng.standard_normal((b, s, h * d)).astype(np.float32)).to(dev)
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    scale = 1.0 / d ** 0.5
    o = torch.empty(b, s, h * d, device=dev)
    lse = torch.empty(b, h, s, device=dev)
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, scale, int(causal), st, st,
                               st, stream))
    split = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
    n = STATIC_SCRATCH
    kind = ("split" if split <= n else "split by chunks" if d <= 64
            and L.fattn_bwd_workspace_split_bytes(1, 1, s, d) <= n else "turns")
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    want = torch.full_like(qkv, float("nan"))
    _lib.check(L.fattn_bwd_f32(qp, kp, vp, P(o), P(dout), P(lse), P(want), P(ws), n, b, h, s, d,
                               scale, int(causal), st, st, st, gst, stream))
    got = torch.full_like(qkv, float("nan"))
    _lib.check(L.fattn_bwd_f32_noalloc(qp, kp, vp, P(o), P(dout), P(lse), P(got), b, h, s, d,
                                       scale, int(causal), st, st, st, gst, stream))
    torch.cuda.synchronize()
    return got, want, kind, (qkv, dout, o)


def check_against_oracle(orc, got, io, h, d, causal, pairs):
    """O and the no-alloc gradient of the (b, h) pairs `pairs` against the fp64 oracle."""
    qkv, dout, o = io
    hd, scale = h * d, 1.0 / d ** 0.5
    for p in pairs:
        bi, hi = divmod(p, h)

        def part(t, i):  # [1, 1, s, d] host array of pair p, part i
            return t[bi, :, i * hd + hi * d:i * hd + (hi + 1) * d].cpu().numpy()[None, None]

        q, k, v = (part(qkv, i) for i in range(3))
        o64, l64 = orc.forward(q, k, v, scale, causal, dtype=np.float64)
        refs = orc.backward(q, k, v, o64, l64, part(dout, 0), scale, causal, dtype=np.float64)
        errs = [orc.rel_fro(part(o, 0), o64)]
        errs += [orc.rel_fro(part(got, i), r) for i, r in enumerate(refs)]
        say(f"  pair {p}: o dq dk dv " + " ".join(f"{e:.2e}" for e in errs))
        assert max(errs) <= REL_TOL, (p, errs)


@pytest.mark.parametrize("causal", [False, True])
def test_noalloc_matches_workspace_entry(orc, cuda, causal):
    # (b, h, s, d): split fits the scratch, then a smaller split shape; the config-2 shape (its
    # split workspace exceeds the scratch: split by chunks), then a smaller one; head_dim 32 and
    # 128 (the latter past the scratch: turns).
    cases = [((4, 6, 240, 64), (2, 3, 97, 64)),
             ((64, 6, 240, 64), (8, 6, 200, 64)),
             ((2, 4, 333, 32), (1, 2, 65, 32)),
             ((2, 3, 150, 128), (1, 1, 17, 128))]
    for big, small in cases:
        for i, (b, h, s, d) in enumerate((big, small)):
            say(f"noalloc b{b} h{h} s{s} d{d} causal={causal} call {i + 1}")
            got, want, kind, io = backward_both(b, h, s, d, causal, seed=b * 1000 + s,
                                                dev=cuda)
            assert torch.isfinite(want).all()
            assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (b, h, s, d, kind)
            say(f"  {kind}: bit-identical")
            check_against_oracle(orc, got, io, h, d, causal, (0, b * h - 1))


def test_noalloc_refuses_what_does_not_fit(cuda):
    """A minimum workspace above the scratch is refused up front (FATTN_EWORKSPACE, no launch)."""
    L = _lib.lib()
    b, h, s, d = 1, 64, 1 << 18, 64   # D alone: 2^24 rows x 4 bytes = 64 MiB, plus counters
    assert L.fattn_bwd_workspace_min_bytes(b, h, s, d) > STATIC_SCRATCH
    st = _lib.arr([0, 0, 64])
    bad = ctypes.c_void_p(0x1000)
    rc = L.fattn_bwd_f32_noalloc(bad, bad, bad, bad, bad, bad, bad, b, h, s, d, 0.125, 0, st, st,
                                 st, st, None)
    assert rc == _lib.FATTN_EWORKSPACE
    assert "static scratch" in _lib.last_error()


@pytest.mark.parametrize("shape", [(64, 6, 240), (4, 6, 240)])
def test_noalloc_under_graph_capture(cuda, shape):
    """The no-alloc backward is for callers under HIP graph capture: the forward and
    fattn_bwd_f32_noalloc captured in one graph and replayed on new inputs (with eager work and
    synchronisations between replays) equal eager fattn_bwd_f32 runs with a workspace of the
    scratch's size (config 2's shape: the split by chunks, several launches captured; the smaller
    one: the whole split), bit for bit."""
    b, h, s = shape
    d = 64
    L = _lib.lib()
    qkv = torch.empty(b, s, 3 * h * d, device=cuda)
    dout = torch.empty(b, s, h * d, device=cuda)
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    got = torch.empty_like(qkv)
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    n = STATIC_SCRATCH
    kind = "split" if L.fattn_bwd_workspace_split_bytes(b, h, s, d) <= n else "split by chunks"
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)

    def captured():
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, 0.125, 0, st, st, st,
                                   stream))
        _lib.check(L.fattn_bwd_f32_noalloc(qp, kp, vp, P(o), P(dout), P(lse), P(got), b, h, s,
                                           d, 0.125, 0, st, st, st, gst, stream))

    def eager_reference():
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        want = torch.empty_like(qkv)
        _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, 0.125, 0, st, st, st,
                                   stream))
        _lib.check(L.fattn_bwd_f32(qp, kp, vp, P(o), P(dout), P(lse), P(want), P(ws), n, b, h, s,
                                   d, 0.125, 0, st, st, st, gst, stream))
        torch.cuda.synchronize()
        return want

    gen = torch.Generator().manual_seed(21)
    qkv.copy_(torch.randn(qkv.shape, generator=gen))
    dout.copy_(torch.randn(dout.shape, generator=gen))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        captured()  # warm-up (the scratch's address is looked up here, outside the capture)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured()
    for r in range(3):
        say(f"noalloc graph replay {r} shape {shape} ({kind})")
        qkv.copy_(torch.randn(qkv.shape, generator=gen))
        dout.copy_(torch.randn(dout.shape, generator=gen))
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        g = got.clone()
        want = eager_reference()
        assert torch.isfinite(want).all()
        assert torch.equal(g.view(torch.int32), want.view(torch.int32)), f"replay {r}"
