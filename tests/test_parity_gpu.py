"""GPU parity: the HIP path (through libfattn.so's C ABI) against the CPU oracle.

Mirrors the reference's tests/parity.rs: the same closed-form inputs (:126-138), the same
`run` = output and the qkv gradient of sum(out o w) (:119-123), both entry points on the same
projection (:78-88), the same shapes (:161-167, :210-221), backward twice over one graph
(:185-204), 8 bitwise reruns (:226-242) and the merge-heads layout contract (:169-183); plus the
five benchmark configurations on their seeded inputs.

The bars: normwise relative error <= 2e-6 against the fp64 oracle for O, dQ, dK, dV on the
benchmark configurations' seeded N(0, 1) inputs (the build's target), and bit-identical reruns.

On the reference tests' closed-form inputs (sin / cos sequences) the gradient is ill-conditioned:
||dQ|| is small next to the terms that cancel into it, and the reference's own algorithm in fp32
(the composed path, restated in oracle/composed.c) misses 2e-6 there by up to 20x on dQ. For
those inputs each component's bar is max(2e-6, 1.5 x that fp32 composed path's own normwise
error against fp64), and the max-abs error against fp64 is held to max(5e-6, the reference's
GPU-vs-CPU band of tests/parity.rs:218, 1.5 x the fp32 composed path's): the HIP path must be
no less accurate than the reference's arithmetic on the same inputs.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import candle_fused_attn as cfa
from candle_fused_attn import _lib

pytestmark = pytest.mark.gpu

REL_TOL = 2e-6      # normwise, vs fp64
BAND = 5e-6         # max-abs, vs the fp32 composed path (tests/parity.rs:218)


def zero_band(d):
    """The max-abs bar for a component whose fp64 value is exactly zero (dQ and dK with one key:
    dS = P (dP - D) with dP = dO . v and D = dO . o, o = v): what remains is the rounding residue
    of two d-term fp32 dot products summed in different orders (MFMA contraction, row-sum tree),
    which grows like sqrt(d). The reference's band (d 64) scaled by sqrt(d / 64)."""
    return BAND * max(1.0, (d / 64) ** 0.5)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(params=["split", "turns"])
def dq_sum(request):
    """Runs a test under each way of summing dQ over key blocks (the workspace size picks it)."""
    prev = cfa.set_dq_sum(request.param)
    yield request.param
    cfa.set_dq_sum(prev)


# --- the reference test's harness (tests/parity.rs:28-123) --------------------------------

def qkv_views(qkv, h, d):
    b, s, _ = qkv.shape
    return tuple(qkv.narrow(2, i * h * d, h * d).reshape(b, s, h, d).transpose(1, 2)
                 for i in range(3))


def attend(path, qkv, h, d, causal, scale=None):
    """path "fused": fused_attention's general node on the head views; "fused_views": the same
    call as a user makes it (the views go to the projection's node); "fused_qkv":
    fused_attention_qkv."""
    b, s, _ = qkv.shape
    scale = 1.0 / d ** 0.5 if scale is None else scale
    if path in ("fused", "fused_views"):
        q, k, v = qkv_views(qkv, h, d)
        prev = cfa.ops.set_projection_route(path == "fused_views")
        try:
            o = cfa.fused_attention(q, k, v, scale, causal)
        finally:
            cfa.ops.set_projection_route(prev)
        return o.transpose(1, 2).reshape(b, s, h * d)
    return cfa.fused_attention_qkv(qkv, h, scale, causal)


def run(path, qkv, w, h, d, causal, scale=None):
    x = qkv.detach().clone().requires_grad_(True)
    out = attend(path, x, h, d, causal, scale)
    (out * w).sum().backward()
    torch.cuda.synchronize()
    return out.detach(), x.grad.detach()


def split3(g):
    return np.split(np.asarray(g, dtype=np.float64), 3, axis=-1)


def normwise(orc, out, grad, ref_out, ref_grad):
    errs = {"o": orc.rel_fro(out, ref_out)}
    for name, a, r in zip(("dq", "dk", "dv"), split3(grad), split3(ref_grad)):
        errs[name] = orc.rel_fro(a, r)
    return errs


def check_errors(orc, out, grad, ref_out, ref_grad, tag, floor=None, d=64):
    """Normwise errors against fp64 within REL_TOL, or within 1.5x `floor` (the fp32 composed
    path's own errors on the same inputs) where that is larger. A component whose fp64 value is
    exactly zero (dQ and dK with one key: dS = dP - D cancels) has no relative error; there the
    max-abs error is held to the reference's GPU-vs-CPU band (tests/parity.rs:218), scaled with
    head_dim d by zero_band."""
    out, grad = out.cpu().numpy(), grad.cpu().numpy()
    errs = normwise(orc, out, grad, ref_out, ref_grad)
    say(f"  {tag}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    refs = dict(zip(("dq", "dk", "dv"), split3(ref_grad)), o=np.asarray(ref_out))
    gots = dict(zip(("dq", "dk", "dv"), split3(grad)), o=np.asarray(out, dtype=np.float64))
    for k, v in errs.items():
        if not np.any(refs[k]):
            dev = float(np.abs(gots[k]).max())
            assert dev <= zero_band(d), f"{tag}: {k} (exactly zero in fp64) max deviation {dev:.3e}"
            continue
        tol = max(REL_TOL, 1.5 * floor[k]) if floor else REL_TOL
        assert v <= tol, f"{tag}: {k} normwise error {v:.3e} > {tol:.3e}"
    return errs


def composed_floor(orc, x, w, h, d, causal, ref_out, ref_grad, scale=None):
    """The fp32 composed path's (the reference's algorithm in fp32) own errors vs fp64."""
    c_out, _, c_grad = oracle_qkv(orc, x, w, h, d, causal, np.float32, scale)
    floor = normwise(orc, c_out, c_grad, ref_out, ref_grad)
    cmax = max(orc.max_abs(c_out, ref_out), orc.max_abs(c_grad, ref_grad))
    say("  fp32 composed floor: " + " ".join(f"{k} {v:.2e}" for k, v in floor.items())
        + f" max-abs {cmax:.2e}")
    return floor, cmax


def check_pairs(orc, qkv, dout, out, grad, h, d, scale, causal, pairs, tag):
    """The fp64 oracle on chosen (b, h) pairs (index b h + h) of a qkv-path result, for shapes
    whose every pair would take the oracle minutes: O, dQ, dK, dV of each pair within REL_TOL
    normwise. qkv, grad [b, s, 3 h d], dout, out [b, s, h d] (device tensors)."""
    hd = h * d

    def part(t, i, bi, hi):  # pair (bi, hi) of part i as a [1, 1, s, d] host array
        lo = i * hd + hi * d
        return t[bi, :, lo:lo + d].cpu().numpy()[None, None]

    for p in pairs:
        bi, hi = divmod(p, h)
        q, k, v = (part(qkv, i, bi, hi) for i in range(3))
        o64, l64 = orc.forward(q, k, v, scale, causal, dtype=np.float64)
        refs = orc.backward(q, k, v, o64, l64, part(dout, 0, bi, hi), scale, causal,
                            dtype=np.float64)
        errs = {"o": orc.rel_fro(part(out, 0, bi, hi), o64)}
        for i, (name, ref) in enumerate(zip(("dq", "dk", "dv"), refs)):
            errs[name] = orc.rel_fro(part(grad, i, bi, hi), ref)
        say(f"  {tag} pair {p} (b {bi}, h {hi}): "
            + " ".join(f"{k_} {v_:.2e}" for k_, v_ in errs.items()))
        for k_, v_ in errs.items():
            assert v_ <= REL_TOL, f"{tag} pair {p}: {k_} normwise error {v_:.3e}"


def oracle_qkv(orc, qkv, w, h, d, causal, dtype, scale=None):
    scale = 1.0 / d ** 0.5 if scale is None else scale
    qkv = np.asarray(qkv)
    out, lse = orc.qkv_forward(qkv, h, scale, causal, dtype=dtype)
    grad = orc.qkv_backward(qkv, h, scale, causal, out, lse, np.asarray(w), dtype=dtype)
    return out, lse, grad


def bits(t):
    return t.contiguous().view(torch.int32).cpu()


# --- the saved row log-sum-exp L (src/lib.rs:258, kernels/fused_attn.cu:596) ----------------

def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _st(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def forward_qkv_c(qkv, h, scale, causal):
    """fattn_qkv_forward (the op level, FusedAttentionQkv::cuda_fwd): (O [b, s, h d], L [b, h, s])."""
    b, s, thd = qkv.shape
    out = torch.empty(b, s, thd // 3, device=qkv.device)
    lse = torch.empty(b, h, s, device=qkv.device)
    _lib.check(_lib.lib().fattn_qkv_forward(
        ctypes.c_void_p(qkv.untyped_storage().data_ptr()), qkv.storage_offset(),
        _lib.arr(qkv.shape), _lib.arr(qkv.stride()), h, scale, int(causal), _p(out), _p(lse),
        _st(qkv)))
    torch.cuda.synchronize()
    return out, lse


def forward_bhsd_c(q, k, v, scale, causal):
    """fattn_forward (the op level, FusedAttention::cuda_fwd) on [b, h, s, d] views:
    (O [b, s, h, d], L [b, h, s])."""
    b, h, s, d = q.shape
    out = torch.empty(b, s, h, d, device=q.device)
    lse = torch.empty(b, h, s, device=q.device)
    args = []
    for t in (q, k, v):
        args += [ctypes.c_void_p(t.untyped_storage().data_ptr()), t.storage_offset(),
                 _lib.arr(t.shape), _lib.arr(t.stride())]
    _lib.check(_lib.lib().fattn_forward(*args, scale, int(causal), _p(out), _p(lse), _st(q)))
    torch.cuda.synchronize()
    return out, lse


def forward_kernel_c(q, k, v, scale, causal):
    """fattn_fwd_f32_d64 (the kernel level, cuda::forward) on [b, h, s, 64] views given by their
    first element and (batch, head, seq) strides: (O [b, s, h, d], L [b, h, s])."""
    b, h, s, d = q.shape
    out = torch.empty(b, s, h, d, device=q.device)
    lse = torch.empty(b, h, s, device=q.device)
    st = [_lib.arr(t.stride()[:3]) for t in (q, k, v)]
    _lib.check(_lib.lib().fattn_fwd_f32_d64(_p(q), _p(k), _p(v), _p(out), _p(lse), b, h, s, d,
                                            scale, int(causal), *st, _st(q)))
    torch.cuda.synchronize()
    return out, lse


def check_lse(lse, ref64, ref32, tag):
    """L against the fp64 oracle's, in absolute terms (L is a log, O(1-10) here): max-abs error
    <= 2e-6 (1 + max |L|), or 1.5 x the fp32 composed path's own max-abs error where that is
    larger (the reference's arithmetic on the same inputs)."""
    got = np.asarray(lse.cpu().numpy() if torch.is_tensor(lse) else lse, dtype=np.float64)
    ref64 = np.asarray(ref64, dtype=np.float64)
    err = float(np.max(np.abs(got - ref64))) if got.size else 0.0
    floor = float(np.max(np.abs(np.asarray(ref32, np.float64) - ref64))) if got.size else 0.0
    bar = max(2e-6 * (1.0 + float(np.max(np.abs(ref64), initial=0.0))), 1.5 * floor)
    say(f"  {tag}: L max-abs {err:.2e} (fp32 composed {floor:.2e}, bar {bar:.2e})")
    assert got.shape == ref64.shape
    assert np.all(np.isfinite(got)), f"{tag}: L not finite"
    assert err <= bar, f"{tag}: L max-abs error {err:.3e} > {bar:.3e}"
    return err


def check_lse_all_levels(orc, qkv, h, d, scale, causal, tag, o_autograd=None):
    """L from the three forward entries (qkv op, general op on the head views, kernel level on
    the head views) against the oracle; their O and L are bit-identical to each other (and O to
    the autograd op's, when given)."""
    x = qkv.cpu().numpy()
    _, l64 = orc.qkv_forward(x, h, scale, causal, dtype=np.float64)
    _, l32 = orc.qkv_forward(x, h, scale, causal, dtype=np.float32)
    o1, l1 = forward_qkv_c(qkv, h, scale, causal)
    q, k, v = qkv_views(qkv, h, d)
    o2, l2 = forward_bhsd_c(q, k, v, scale, causal)
    o3, l3 = forward_kernel_c(q, k, v, scale, causal)
    check_lse(l1, l64, l32, f"{tag} qkv op")
    assert torch.equal(bits(l1), bits(l2)) and torch.equal(bits(l1), bits(l3)), f"{tag}: L"
    assert torch.equal(bits(o1), bits(o2.reshape(o1.shape)))
    assert torch.equal(bits(o1), bits(o3.reshape(o1.shape)))
    if o_autograd is not None:
        assert torch.equal(bits(o1), bits(o_autograd))
    return l1


# --- tests/parity.rs, on the GPU ------------------------------------------------------------

PARITY_SHAPES = [(2, 7, 3, 64), (2, 240, 6, 64), (1, 97, 2, 64), (1, 33, 2, 64)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", PARITY_SHAPES)
def test_matches_oracle_closed_form(orc, cuda, shape, causal):
    b, s, h, d = shape
    say(f"parity b{b} s{s} h{h} d{d} causal={causal}")
    x, w = orc.closed_form_inputs(b, s, h, d)
    ref_out, _, ref_grad = oracle_qkv(orc, x, w, h, d, causal, np.float64)
    floor, cmax = composed_floor(orc, x, w, h, d, causal, ref_out, ref_grad)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    for path in ("fused", "fused_qkv"):
        say(f"  path {path}")
        out, grad = run(path, qkv, wt, h, d, causal)
        check_errors(orc, out, grad, ref_out, ref_grad, path, floor)
        eo = orc.max_abs(out.cpu().numpy(), ref_out)
        eg = orc.max_abs(grad.cpu().numpy(), ref_grad)
        say(f"  {path}: max-abs vs fp64: out {eo:.2e} grad {eg:.2e}")
        assert max(eo, eg) <= max(BAND, 1.5 * cmax)
    check_lse_all_levels(orc, qkv, h, d, 1.0 / d ** 0.5, causal, "closed form", out)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 7, 3, 32), (1, 97, 2, 32), (2, 7, 3, 128), (1, 97, 2, 128),
                                   (1, 33, 2, 128), (1, 128, 2, 128), (2, 240, 3, 128)])
def test_closed_form_other_head_dims(orc, cuda, shape, causal):
    """The closed-form inputs at head_dim 32 and 128, under the same bars as d 64: no component
    less accurate than 1.5 x the fp32 composed path's own error against fp64 (or 2e-6). At d 128
    an earlier contraction order (32 g + t over the whole row) left dK at 1.7-2.5 x the composed
    path's error and failed here; d 64's order on each half of the row passes with margin."""
    b, s, h, d = shape
    say(f"closed form b{b} s{s} h{h} d{d} causal={causal}")
    x, w = orc.closed_form_inputs(b, s, h, d)
    ref_out, _, ref_grad = oracle_qkv(orc, x, w, h, d, causal, np.float64)
    floor, cmax = composed_floor(orc, x, w, h, d, causal, ref_out, ref_grad)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    out, grad = run("fused_qkv", qkv, wt, h, d, causal)
    check_errors(orc, out, grad, ref_out, ref_grad, f"d{d}", floor, d=d)
    eg = orc.max_abs(grad.cpu().numpy(), ref_grad)
    assert eg <= max(zero_band(d), 1.5 * cmax), f"max-abs {eg:.3e}"


def test_golden_vectors_gpu(orc, cuda):
    from test_oracle import golden_cases, parse
    data, keys = golden_cases()
    n = 0
    for key in keys:
        b, s, h, d, causal = parse(key)
        if d != 64:
            continue
        say(f"golden {key}")
        x, wn = data[f"{key}/qkv"], data[f"{key}/w"]
        ref_out, ref_grad = data[f"{key}/out"], data[f"{key}/grad"]
        floor, _ = composed_floor(orc, x, wn, h, d, causal, ref_out, ref_grad)
        qkv, w = torch.from_numpy(x).to(cuda), torch.from_numpy(wn).to(cuda)
        for path in ("fused", "fused_qkv"):
            out, grad = run(path, qkv, w, h, d, causal)
            check_errors(orc, out, grad, ref_out, ref_grad, path, floor)
        n += 1
    assert n >= 3


def test_outputs_are_merge_heads_ready(orc, cuda):
    x, _ = orc.closed_form_inputs(2, 5, 2, 64)
    qkv = torch.from_numpy(x).to(cuda)
    q, k, v = qkv_views(qkv, 2, 64)
    o = cfa.fused_attention(q, k, v, 0.3, False)
    assert tuple(o.shape) == (2, 2, 5, 64)
    assert o.transpose(1, 2).is_contiguous(), "O is physically [b, s, h, d]"
    o = cfa.fused_attention_qkv(qkv, 2, 0.3, False)
    assert tuple(o.shape) == (2, 5, 128) and o.is_contiguous() and o.dtype == torch.float32


def test_backward_twice_over_one_graph(orc, cuda):
    """The saved L is read, not consumed: two backward passes over one graph agree bitwise."""
    x, w = orc.closed_form_inputs(1, 9, 2, 64)
    qkv = torch.from_numpy(x).to(cuda).requires_grad_(True)
    wt = torch.from_numpy(w).to(cuda)
    out = attend("fused_qkv", qkv, 2, 64, False)
    loss = (out * wt).sum()
    (g1,) = torch.autograd.grad(loss, qkv, retain_graph=True)
    (g2,) = torch.autograd.grad(loss, qkv)
    assert torch.equal(bits(g1), bits(g2))


@pytest.mark.parametrize("causal", [False, True])
def test_entry_points_agree(orc, cuda, causal):
    """fused_attention on the head views and fused_attention_qkv on the projection run the same
    kernels on the same views: equal outputs and gradients."""
    b, s, h, d = 2, 240, 6, 64
    x, w = orc.closed_form_inputs(b, s, h, d)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    o1, g1 = run("fused", qkv, wt, h, d, causal)
    o2, g2 = run("fused_qkv", qkv, wt, h, d, causal)
    assert torch.equal(o1, o2) and torch.equal(g1, g2)


@pytest.mark.parametrize("path", ["fused", "fused_qkv"])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_is_deterministic(orc, cuda, causal, path, dq_sum):
    """dQ is summed over key blocks in a fixed order: reruns are bit-identical
    (tests/parity.rs:223-242, 8 reruns)."""
    b, s, h, d = 4, 240, 6, 64
    say(f"determinism {path} causal={causal} {dq_sum}")
    x, w = orc.closed_form_inputs(b, s, h, d)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    o1, g1 = run(path, qkv, wt, h, d, causal)
    b1, ob1 = bits(g1), bits(o1)
    for rerun in range(8):
        o2, g2 = run(path, qkv, wt, h, d, causal)
        assert torch.equal(bits(g2), b1), f"{path} causal {causal}: rerun {rerun} differs"
        assert torch.equal(bits(o2), ob1)


@pytest.mark.parametrize("causal", [False, True])
def test_side_streams(orc, cuda, causal, dq_sum):
    """Every launch goes on the caller's current stream (src/cuda.rs launches on candle's stream):
    two forward + backward passes on two side streams, their launches interleaved and their
    backwards in flight together (each with its own workspace), equal the same passes on the
    default stream bit for bit."""
    b, s, h, d = 4, 240, 6, 64
    say(f"side streams causal={causal} {dq_sum}")
    inputs = [tuple(torch.from_numpy(a).to(cuda) for a in orc.seeded_qkv_inputs(b, h, s, seed=sd, d=d))
              for sd in (11, 12)]
    want = [run("fused_qkv", x, w, h, d, causal, 0.125) for x, w in inputs]
    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    xs, outs = [], []
    for (x, _), st in zip(inputs, streams):
        st.wait_stream(torch.cuda.current_stream(cuda))
        with torch.cuda.stream(st):
            xg = x.detach().clone().requires_grad_(True)
            xs.append(xg)
            outs.append(cfa.fused_attention_qkv(xg, h, 0.125, causal))
    for (_, w), xg, o, st in zip(inputs, xs, outs, streams):
        with torch.cuda.stream(st):
            (o * w).sum().backward()
    torch.cuda.synchronize()
    for (o_want, g_want), xg, o in zip(want, xs, outs):
        assert torch.equal(bits(o.detach()), bits(o_want))
        assert torch.equal(bits(xg.grad), bits(g_want))


# --- edge cases ------------------------------------------------------------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_sequence_lengths(orc, cuda, causal, dq_sum):
    """Tails of every kind: single key, partial 16-query tiles, partial 64-key blocks."""
    rng = np.random.default_rng(3)
    for s in (1, 2, 15, 16, 17, 48, 63, 64, 65, 100, 129, 200):
        x = rng.standard_normal((2, s, 3 * 2 * 64)).astype(np.float32)
        w = rng.standard_normal((2, s, 2 * 64)).astype(np.float32)
        say(f"seq {s} causal={causal} {dq_sum}")
        ref_out, _, ref_grad = oracle_qkv(orc, x, w, 2, 64, causal, np.float64, 0.125)
        out, grad = run("fused_qkv", torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda),
                        2, 64, causal, 0.125)
        check_errors(orc, out, grad, ref_out, ref_grad, f"s{s}")


def test_empty_inputs(cuda):
    qkv = torch.zeros(0, 5, 384, device=cuda, requires_grad=True)
    out = cfa.fused_attention_qkv(qkv, 2, 0.125, False)
    assert tuple(out.shape) == (0, 5, 128)
    out.sum().backward()
    assert tuple(qkv.grad.shape) == (0, 5, 384)
    q = torch.zeros(2, 2, 0, 64, device=cuda)
    assert tuple(cfa.fused_attention(q, q, q, 0.125, True).shape) == (2, 2, 0, 64)


def test_misaligned_operands_are_copied(orc, cuda):
    """An operand the kernels cannot read in place is copied first (src/lib.rs:114-118)."""
    x, w = orc.closed_form_inputs(1, 33, 2, 64)
    qkv = torch.from_numpy(x).to(cuda)
    wt = torch.from_numpy(w).to(cuda)
    big = torch.zeros(qkv.numel() + 1, device=cuda)
    big[1:] = qkv.reshape(-1)
    shifted = big[1:].reshape(qkv.shape)        # storage offset 1: not float4-aligned
    assert not cfa.reads_in_place(shifted)
    o1, g1 = run("fused_qkv", qkv, wt, 2, 64, True)
    o2, g2 = run("fused_qkv", shifted, wt, 2, 64, True)
    assert torch.equal(o1, o2) and torch.equal(g1, g2)


def test_strided_gradient(orc, cuda):
    """A non-contiguous output gradient is read through its strides (or copied)."""
    x, w = orc.closed_form_inputs(2, 40, 2, 64)
    qkv = torch.from_numpy(x).to(cuda)
    w_t = torch.from_numpy(np.ascontiguousarray(np.swapaxes(w, 0, 1))).to(cuda).transpose(0, 1)
    assert not w_t.is_contiguous()
    o1, g1 = run("fused_qkv", qkv, torch.from_numpy(w).to(cuda), 2, 64, False)
    o2, g2 = run("fused_qkv", qkv, w_t, 2, 64, False)
    assert torch.equal(g1, g2)


def test_kernel_level_entry_points(orc, cuda):
    """The kernel-level C ABI (fattn_fwd_f32_d64 / fattn_bwd_f32_d64) on the qkv views gives the
    op level's results bit for bit, and the turn protocol's guard word stays 0."""
    b, s, h, d = 2, 97, 3, 64
    x, w = orc.closed_form_inputs(b, s, h, d)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    o_ref, g_ref = run("fused_qkv", qkv, wt, h, d, True)
    L = _lib.lib()
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    base = qkv.data_ptr()
    hd4 = h * d * 4
    qp, kp, vp = (ctypes.c_void_p(base + i * hd4) for i in range(3))
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    scale = 1.0 / 8.0
    rc = L.fattn_fwd_f32_d64(qp, kp, vp, ctypes.c_void_p(o.data_ptr()),
                             ctypes.c_void_p(lse.data_ptr()), b, h, s, d, scale, 1, st, st, st,
                             stream)
    _lib.check(rc)
    dqkv = torch.empty_like(qkv)
    nbytes = L.fattn_bwd_workspace_bytes(b, h, s, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    rc = L.fattn_bwd_f32_d64(qp, kp, vp, ctypes.c_void_p(o.data_ptr()),
                             ctypes.c_void_p(wt.data_ptr()), ctypes.c_void_p(lse.data_ptr()),
                             ctypes.c_void_p(dqkv.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                             nbytes, b, h, s, d, scale, 1, st, st, st, gst, stream)
    _lib.check(rc)
    status = ctypes.c_int(-1)
    _lib.check(L.fattn_bwd_status(ctypes.c_void_p(ws.data_ptr()), nbytes, b, h, s, stream,
                                  ctypes.byref(status)))
    assert status.value == 0
    assert torch.equal(o, o_ref) and torch.equal(dqkv, g_ref)
    # The three steps one by one, with either workspace size (causal: both sum dQ in key-block
    # order, so the results are identical).
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for size in (L.fattn_bwd_workspace_split_bytes, L.fattn_bwd_workspace_min_bytes):
        n = size(b, h, s, d)
        ws = torch.empty(n, dtype=torch.uint8, device=cuda)
        dqkv = torch.empty_like(qkv)
        _lib.check(L.fattn_bwd_prep_f32_d64(P(o), P(wt), gst, P(ws), n, b, h, s, d, stream))
        _lib.check(L.fattn_bwd_main_f32_d64(qp, kp, vp, P(o), P(wt), P(lse), P(dqkv), P(ws), n, b, h,
                                            s, d, scale, 1, st, st, st, gst, stream))
        _lib.check(L.fattn_bwd_dq_f32_d64(P(dqkv), P(ws), n, b, h, s, d, scale, 1, stream))
        torch.cuda.synchronize()
        assert torch.equal(dqkv, g_ref), f"steps with a {n}-byte workspace"


# --- the benchmark configurations -------------------------------

def test_config1_general_path(orc, cuda):
    """[2, 4, 128, 64] contiguous q, k, v ~ N(0, 1), dO ~ N(0, 1), scale 1/8, non-causal."""
    g = torch.Generator().manual_seed(1)
    q, k, v, do = (torch.randn(2, 4, 128, 64, generator=g) for _ in range(4))
    o64, l64 = orc.forward(q.numpy(), k.numpy(), v.numpy(), 0.125, False, dtype=np.float64)
    dq64, dk64, dv64 = orc.backward(q.numpy(), k.numpy(), v.numpy(), o64, l64, do.numpy(),
                                    0.125, False, dtype=np.float64)
    qg, kg, vg = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    o = cfa.fused_attention(qg, kg, vg, 0.125, False)
    o.backward(do.to(cuda))
    for name, a, r in (("o", o, o64), ("dq", qg.grad, dq64), ("dk", kg.grad, dk64),
                       ("dv", vg.grad, dv64)):
        e = orc.rel_fro(a.detach().cpu().numpy(), r)
        say(f"  config1 {name} {e:.2e}")
        assert e <= REL_TOL
    _, l32 = orc.forward(q.numpy(), k.numpy(), v.numpy(), 0.125, False, dtype=np.float32)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    o_op, l_op = forward_bhsd_c(qd, kd, vd, 0.125, False)
    o_k, l_k = forward_kernel_c(qd, kd, vd, 0.125, False)
    check_lse(l_op, l64, l32, "config1 general op")
    assert torch.equal(bits(l_op), bits(l_k)) and torch.equal(bits(o_op), bits(o_k))
    assert torch.equal(bits(o_op.transpose(1, 2)), bits(o.detach()))


def seeded_qkv(orc, b, h, s, seed, cuda, d=64):
    x, dout = orc.seeded_qkv_inputs(b, h, s, seed, d=d)
    return x, dout, torch.from_numpy(x).to(cuda), torch.from_numpy(dout).to(cuda)


def test_config2_target(orc, cuda):
    """qkv [64, 240, 1152] (h 6) ~ N(0, 1) seed 0 (the reference's published inputs), non-causal;
    the reference reports O 3.9e-7, dQ 4.0e-7, dK 4.6e-7, dV 4.4e-7 here."""
    x, dout, qkv, g = seeded_qkv(orc, 64, 6, 240, 0, cuda)
    ref_out, _, ref_grad = oracle_qkv(orc, x, dout, 6, 64, False, np.float64, 0.125)
    out, grad = run("fused_qkv", qkv, g, 6, 64, False, 0.125)
    errs = check_errors(orc, out, grad, ref_out, ref_grad, "config2")
    check_lse_all_levels(orc, qkv, 6, 64, 0.125, False, "config2", out)
    # The scorer reports a deliberate perturbation of the HIP output at its size: a relative
    # 1e-4 random perturbation and a uniform 1e-5 rescale, each within the output's own error.
    o = out.cpu().numpy().astype(np.float64)
    rng = np.random.default_rng(2)
    n = rng.standard_normal(o.shape)
    delta = n * (1e-4 * np.linalg.norm(ref_out) / np.linalg.norm(n))
    for name, pert, size in (("random", o + delta, 1e-4), ("rescale", o * (1 + 1e-5), 1e-5)):
        got = orc.rel_fro(pert, ref_out)
        say(f"  perturbed output ({name} {size:.0e}): scored {got:.4e}")
        assert abs(got - size) <= 2 * errs["o"] + 1e-3 * size, (name, got)


def test_config3_causal_reruns(orc, cuda, dq_sum):
    """Config 2's shape, causal, plus 10 backward reruns compared bitwise."""
    say(f"config3 {dq_sum}")
    x, dout, qkv, g = seeded_qkv(orc, 64, 6, 240, 0, cuda)
    ref_out, _, ref_grad = oracle_qkv(orc, x, dout, 6, 64, True, np.float64, 0.125)
    out, grad = run("fused_qkv", qkv, g, 6, 64, True, 0.125)
    check_errors(orc, out, grad, ref_out, ref_grad, "config3")
    if dq_sum == "split":
        check_lse_all_levels(orc, qkv, 6, 64, 0.125, True, "config3", out)
    first = bits(grad)
    for rerun in range(10):
        _, g2 = run("fused_qkv", qkv, g, 6, 64, True, 0.125)
        assert torch.equal(bits(g2), first), f"rerun {rerun} differs"


def to_heads(x, h):
    """[b, s, h d] -> [b, h, s, d]."""
    b, s, hd = x.shape
    return np.ascontiguousarray(x.reshape(b, s, h, hd // h).transpose(0, 2, 1, 3))


def check_full(orc, q, k, v, do, o, dq, dk, dv, scale, causal, tag, lse=None):
    """The fp64 oracle on every (b, h) slice: normwise errors of O, dQ, dK, dV over the whole
    tensors, L's max-abs error (when given, against the fp32 composed path's as floor), and the
    invariants sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i per (b, h)."""
    o64, l64 = orc.forward(q, k, v, scale, causal, dtype=np.float64)
    dq64, dk64, dv64 = orc.backward(q, k, v, o64, l64, do, scale, causal, dtype=np.float64)
    rel = {name: orc.rel_fro(got, ref) for name, got, ref in
           (("o", o, o64), ("dq", dq, dq64), ("dk", dk, dk64), ("dv", dv, dv64))}
    say(f"  {tag} (every slice): " + " ".join(f"{k_} {v_:.2e}" for k_, v_ in rel.items()))
    for k_, v_ in rel.items():
        assert v_ <= REL_TOL, f"{tag}: {k_} {v_:.3e}"
    if lse is not None:
        _, l32 = orc.forward(q, k, v, scale, causal, dtype=np.float32)
        check_lse(lse, l64, l32, tag)
    dk_sum = np.abs(np.asarray(dk, np.float64).sum(axis=2)).max()
    dv_err = np.abs(np.asarray(dv, np.float64).sum(axis=2)
                    - np.asarray(do, np.float64).sum(axis=2)).max()
    scale_k = np.abs(np.asarray(dk)).max() + 1e-30
    scale_v = np.abs(np.asarray(do, np.float64).sum(axis=2)).max() + 1e-30
    say(f"  {tag} invariants: |sum dK|/max|dK| {dk_sum / scale_k:.2e}, "
        f"|sum dV - sum dO|/max {dv_err / scale_v:.2e}")
    assert dk_sum / scale_k < 1e-3 and dv_err / scale_v < 1e-4


def test_config4_long_causal(orc, cuda):
    """qkv [8, 2048, 2304] (h 12) ~ N(0, 1) seed 2, causal."""
    b, h, s, d = 8, 12, 2048, 64
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 2, cuda)
    say("config4 run")
    out, grad = run("fused_qkv", qkv, g, h, d, True, 0.125)
    o_c, lse = forward_qkv_c(qkv, h, 0.125, True)
    assert torch.equal(bits(o_c), bits(out))
    q, k, v = orc.split_heads(x, h)
    do, o = to_heads(dout, h), to_heads(out.cpu().numpy(), h)
    dq, dk, dv = orc.split_heads(grad.cpu().numpy(), h)
    check_full(orc, q, k, v, do, o, dq, dk, dv, 0.125, True, "config4", lse=lse.cpu().numpy())


def test_config5_strided_views_large_logits(orc, cuda):
    """q, k, v = transpose(1, 2) of [16, 1024, 16, 64] buffers ~ N(0, 4) (std 2), read in place
    (strides [1048576, 64, 1024, 1]); dO ~ N(0, 1); scale 1/8, non-causal."""
    gen = torch.Generator().manual_seed(3)
    bufs = [torch.randn(16, 1024, 16, 64, generator=gen) * 2.0 for _ in range(3)]
    do = torch.randn(16, 16, 1024, 64, generator=gen)
    qg, kg, vg = (t.to(cuda).transpose(1, 2).requires_grad_(False) for t in bufs)
    assert all(cfa.reads_in_place(t) for t in (qg, kg, vg))
    assert qg.stride() == (1048576, 64, 1024, 1)
    leaves = [t.to(cuda).requires_grad_(True) for t in bufs]
    q, k, v = (t.transpose(1, 2) for t in leaves)
    say("config5 run")
    o = cfa.fused_attention(q, k, v, 0.125, False)
    o.backward(do.to(cuda))
    torch.cuda.synchronize()
    o_op, lse = forward_bhsd_c(qg, kg, vg, 0.125, False)
    o_k, lse_k = forward_kernel_c(qg, kg, vg, 0.125, False)
    assert torch.equal(bits(lse), bits(lse_k)) and torch.equal(bits(o_op), bits(o_k))
    assert torch.equal(bits(o_op.transpose(1, 2)), bits(o.detach()))
    qn, kn, vn = (t.transpose(1, 2).numpy() for t in bufs)
    dq, dk, dv = (t.grad.transpose(1, 2).cpu().numpy() for t in leaves)
    check_full(orc, qn, kn, vn, do.numpy(), o.detach().cpu().numpy(), dq, dk, dv, 0.125, False,
               "config5", lse=lse.cpu().numpy())


@pytest.mark.parametrize("s", [4096, 4160])
def test_long_sequences_both_walk_orders(orc, cuda, s, dq_sum):
    """Turns: non-causal key blocks walk staggered over the tiles up to 64 blocks per (b, h)
    (s 4096) and in index order beyond (s 4160); split: index order. Against fp64, and
    bit-identical reruns."""
    rng = np.random.default_rng(s)
    x = rng.standard_normal((1, s, 3 * 64)).astype(np.float32)
    w = rng.standard_normal((1, s, 64)).astype(np.float32)
    say(f"long non-causal s{s} {dq_sum}")
    ref_out, _, ref_grad = oracle_qkv(orc, x, w, 1, 64, False, np.float64, 0.125)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    out, grad = run("fused_qkv", qkv, wt, 1, 64, False, 0.125)
    check_errors(orc, out, grad, ref_out, ref_grad, f"s{s}")
    _, grad2 = run("fused_qkv", qkv, wt, 1, 64, False, 0.125)
    assert torch.equal(bits(grad), bits(grad2))


@pytest.mark.parametrize("causal", [False, True])
def test_split_and_turns_agree(orc, cuda, causal):
    """The two ways of summing dQ. Causal: both walk each key block's tiles upward and sum dQ in
    key-block order, so O and the whole gradient are bit-identical. Non-causal: turns walk the
    tiles from a staggered start (so dK and dV accumulate in another order) and sum dQ in that
    order: O is identical, the gradient agrees to rounding."""
    b, h, s = 8, 6, 240
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 0, cuda)
    res = {}
    for mode in ("split", "turns"):
        say(f"agree causal={causal} {mode}")
        prev = cfa.set_dq_sum(mode)
        try:
            res[mode] = run("fused_qkv", qkv, g, h, 64, causal, 0.125)
        finally:
            cfa.set_dq_sum(prev)
    (o1, g1), (o2, g2) = res["split"], res["turns"]
    assert torch.equal(bits(o1), bits(o2))
    if causal:
        assert torch.equal(bits(g1), bits(g2))
    else:
        for i, name in enumerate(("dQ", "dK", "dV")):
            a, b_ = g1[..., i * h * 64:(i + 1) * h * 64], g2[..., i * h * 64:(i + 1) * h * 64]
            rel = ((a - b_).norm() / b_.norm()).item()
            say(f"  {name} split vs turns: {rel:.2e}")
            assert rel <= 1e-6


@pytest.mark.parametrize("d,h,s", [(64, 9, 240), (64, 9, 100), (64, 17, 50), (32, 9, 240),
                                   (32, 17, 100), (128, 9, 240), (128, 17, 100)])
def test_dq_sums_in_step2_match_step3(orc, cuda, d, h, s):
    """Non-causal split backward: the last workgroups of step 2 sum the dQ tiles, first those of
    the (b, h)s whose last key block each XCD ran (heads 0-7, or 0-15), then the rest (the last
    head, whose last key block is dealt round robin); step 3, when run, sums what step 2 left: the
    same operations in the same order. With every head given the same q, k, v and output gradient,
    every head's O, dQ, dK and dV must be bit-identical, whichever kernel summed it; head 0 is
    checked against the fp64 oracle."""
    rng = np.random.default_rng(11 + d)
    one = rng.standard_normal((1, s, 3, 1, d)).astype(np.float32)
    x = np.ascontiguousarray(np.broadcast_to(one, (1, s, 3, h, d))).reshape(1, s, 3 * h * d)
    w1 = rng.standard_normal((1, s, 1, d)).astype(np.float32)
    w = np.ascontiguousarray(np.broadcast_to(w1, (1, s, h, d))).reshape(1, s, h * d)
    say(f"dq sums d{d} b1 h{h} s{s}")
    out, grad = run("fused_qkv", torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), h, d,
                    False, 0.125)
    o = out.reshape(1, s, h, d)
    g = grad.reshape(1, s, 3, h, d)
    for i in range(1, h):
        assert torch.equal(bits(o[:, :, i]), bits(o[:, :, 0])), f"O of head {i}"
        assert torch.equal(bits(g[:, :, :, i]), bits(g[:, :, :, 0])), f"gradient of head {i}"
    ref_out, _, ref_grad = oracle_qkv(orc, one.reshape(1, s, 3 * d), w1.reshape(1, s, d), 1, d,
                                      False, np.float64, 0.125)
    check_errors(orc, o[:, :, 0].contiguous(), g[:, :, :, 0].reshape(1, s, 3 * d), ref_out,
                 ref_grad, "head 0")
    # Which tiles step 2 summed: after step 2 alone, the done flags that hold the launch's epoch
    # (recorded in the workspace) are exactly the tiles of the (b, h)s the schedule gives the
    # summing workgroups; step 3 then sums the rest, and the gradient is the op level's.
    summed = step2_summed_tiles(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), h, d,
                                False, grad)
    from test_boundary import expected_sum_bh
    n_bh = expected_sum_bh(h, s, False)
    ntile = -(-s // 16)
    want = np.zeros((h, ntile), dtype=bool)
    want[:n_bh] = True
    say(f"  step 2 summed {int(summed.sum())} of {summed.size} tiles (schedule: {n_bh} heads)")
    assert np.array_equal(summed, want)


def test_long_noncausal_128_key_blocks(orc, cuda):
    """Non-causal d 64 from s 512 on, with at least 512 workgroups of 128 keys, step 2 runs
    128-key blocks (each wave two groups of 16 keys; half the dQ partials). At b 4 h 32 s 512:
    every (b, h) slice against the fp64 oracle, two runs bit-identical, and step 2's own dQ sums
    switched off by the test hook (step 3 sums every tile) giving the same bits."""
    from test_boundary import sum_audit
    b, h, s = 4, 32, 512
    assert sum_audit(b, h, s, 64, False)["keys"] == 128
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 21, cuda)
    say(f"128-key blocks: b{b} h{h} s{s}")
    out, grad = run("fused_qkv", qkv, g, h, 64, False, 0.125)
    ref_out, _, ref_grad = oracle_qkv(orc, x, dout, h, 64, False, np.float64, 0.125)
    check_errors(orc, out, grad, ref_out, ref_grad, "b4 h32 s512")
    out2, grad2 = run("fused_qkv", qkv, g, h, 64, False, 0.125)
    assert torch.equal(bits(out2), bits(out)) and torch.equal(bits(grad2), bits(grad))
    f = _hook("fattn_internal_step2_sums")
    prev = f(0)
    try:
        _, grad3 = run("fused_qkv", qkv, g, h, 64, False, 0.125)
    finally:
        f(prev)
    assert torch.equal(bits(grad3), bits(grad)), "step 2 sums off: different bits"
    # The general entry on the head views takes the same path: the same gradient.
    _, grad4 = run("fused", qkv, g, h, 64, False, 0.125)
    assert torch.equal(bits(grad4), bits(grad))


def test_d32_128_key_blocks(orc, cuda):
    """Non-causal d 32 with at least 1536 workgroups of 128 keys (two rounds of three per CU)
    runs 128-key blocks (bwd_split_kernel<32, 2>). At b 12 h 32 s 512: batch 0's 32 heads against
    the fp64 oracle, two runs bit-identical, and step 2's own dQ sums switched off (step 3 sums
    every tile) giving the same bits."""
    from test_boundary import sum_audit
    b, h, s, d = 12, 32, 512, 32
    assert sum_audit(b, h, s, d, False)["keys"] == 128
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 23, cuda, d=d)
    say(f"d32 128-key blocks: b{b} h{h} s{s}")
    out, grad = run("fused_qkv", qkv, g, h, d, False, 0.125)
    ref_out, _, ref_grad = oracle_qkv(orc, x[:1], dout[:1], h, d, False, np.float64, 0.125)
    check_errors(orc, out[:1], grad[:1], ref_out, ref_grad, "b12 h32 s512 d32, batch 0")
    out2, grad2 = run("fused_qkv", qkv, g, h, d, False, 0.125)
    assert torch.equal(bits(out2), bits(out)) and torch.equal(bits(grad2), bits(grad))
    sums = _hook("fattn_internal_step2_sums")
    prev = sums(0)
    try:
        _, grad3 = run("fused_qkv", qkv, g, h, d, False, 0.125)
    finally:
        sums(prev)
    assert torch.equal(bits(grad3), bits(grad)), "step 2 sums off: different bits"


def test_long_noncausal_128_key_blocks_sum_schedule(orc, cuda):
    """The 128-key path's dQ sums in step 2: b 1 h 128 s 512 with every head given the same q, k,
    v and output gradient, so that every head's O and gradient must be bit-identical whichever
    kernel summed it; after step 2 alone the done flags mark exactly the heads the schedule gives
    the summing workgroups (all 128 here); head 0 against the fp64 oracle."""
    from test_boundary import expected_sum_bh, sum_audit
    h, s, d = 128, 512, 64
    assert sum_audit(1, h, s, d, False)["keys"] == 128
    rng = np.random.default_rng(5)
    one = rng.standard_normal((1, s, 3, 1, d)).astype(np.float32)
    x = np.ascontiguousarray(np.broadcast_to(one, (1, s, 3, h, d))).reshape(1, s, 3 * h * d)
    w1 = rng.standard_normal((1, s, 1, d)).astype(np.float32)
    w = np.ascontiguousarray(np.broadcast_to(w1, (1, s, h, d))).reshape(1, s, h * d)
    out, grad = run("fused_qkv", torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), h, d,
                    False, 0.125)
    o = out.reshape(1, s, h, d)
    gr = grad.reshape(1, s, 3, h, d)
    for i in range(1, h):
        assert torch.equal(bits(o[:, :, i]), bits(o[:, :, 0])), f"O of head {i}"
        assert torch.equal(bits(gr[:, :, :, i]), bits(gr[:, :, :, 0])), f"gradient of head {i}"
    ref_out, _, ref_grad = oracle_qkv(orc, one.reshape(1, s, 3 * d), w1.reshape(1, s, d), 1, d,
                                      False, np.float64, 0.125)
    check_errors(orc, o[:, :, 0].contiguous(), gr[:, :, :, 0].reshape(1, s, 3 * d), ref_out,
                 ref_grad, "head 0")
    summed = step2_summed_tiles(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda), h, d,
                                False, grad)
    n_bh = expected_sum_bh(h, s, False, 128)
    want = np.zeros((h, -(-s // 16)), dtype=bool)
    want[:n_bh] = True
    say(f"  step 2 summed {int(summed.sum())} of {summed.size} tiles (schedule: {n_bh} heads)")
    assert n_bh == h and np.array_equal(summed, want)


@pytest.mark.parametrize("causal", [False, True])
def test_projection_views_take_the_qkv_node(orc, cuda, causal):
    """fused_attention on the head-split views of one projection runs fused_attention_qkv's node:
    its output and the projection's gradient equal both the qkv entry's and the general node's bit
    for bit, the graph holds the projection's node, and no view gradient is assembled."""
    b, h, s, d = 4, 6, 240, 64
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 7, cuda)
    res = {p: run(p, qkv, g, h, d, causal, 0.125) for p in ("fused_views", "fused_qkv", "fused")}
    for p in ("fused_qkv", "fused"):
        assert torch.equal(bits(res["fused_views"][0]), bits(res[p][0])), f"O vs {p}"
        assert torch.equal(bits(res["fused_views"][1]), bits(res[p][1])), f"gradient vs {p}"
    xx = qkv.detach().clone().requires_grad_(True)
    q, k, v = qkv_views(xx, h, d)
    out = cfa.fused_attention(q, k, v, 0.125, causal)
    names = []
    fn = out.grad_fn
    while fn is not None and len(names) < 8:
        names.append(type(fn).__name__)
        fn = fn.next_functions[0][0] if fn.next_functions else None
    say(f"  graph from the output: {names}")
    assert any("FusedAttentionQkv" in n for n in names), names
    assert not any(n == "_FusedAttentionBackward" for n in names), names


def test_projection_views_hooks_and_autograd_grad(orc, cuda):
    """Where routing the projection's views would skip what the caller attached to a view, it is
    not routed: a backward hook on k makes fused_attention take the general node, the hook runs
    and sees k's gradient, and the projection's gradient equals the routed one bit for bit. Routed,
    the views are not on the graph (torch.autograd.grad(out, [q, k, v]) finds them unused, as
    documented), while the projection's gradient is there; with routing off, autograd.grad on the
    views returns the projection gradient's three parts bit for bit."""
    b, h, s, d = 2, 3, 97, 64
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 9, cuda)
    want = run("fused_qkv", qkv, g, h, d, False, 0.125)[1].view(b, s, 3, h, d)
    gout = g.view(b, s, h, d).transpose(1, 2)

    seen = {}
    xx = qkv.detach().clone().requires_grad_(True)
    q, k, v = qkv_views(xx, h, d)
    k.register_hook(lambda grad: seen.setdefault("k", grad.detach().clone()))
    out = cfa.fused_attention(q, k, v, 0.125, False)
    fn = out.grad_fn
    while fn is not None and "FusedAttention" not in type(fn).__name__:
        fn = fn.next_functions[0][0] if fn.next_functions else None
    assert fn is not None and "Qkv" not in type(fn).__name__, "not the general node"
    out.backward(gout)
    assert "k" in seen, "the hook on k did not run"
    assert torch.equal(bits(seen["k"]), bits(want[:, :, 1].transpose(1, 2))), "k's gradient"
    assert torch.equal(bits(xx.grad.view(b, s, 3, h, d)), bits(want)), "projection gradient"

    xx = qkv.detach().clone().requires_grad_(True)
    q, k, v = qkv_views(xx, h, d)
    out = cfa.fused_attention(q, k, v, 0.125, False)
    with pytest.raises(RuntimeError):
        torch.autograd.grad(out, [q, k, v], gout)
    (gx,) = torch.autograd.grad(out, [xx], gout)
    assert torch.equal(bits(gx.view(b, s, 3, h, d)), bits(want))

    prev = cfa.set_projection_route(False)
    try:
        xx = qkv.detach().clone().requires_grad_(True)
        q, k, v = qkv_views(xx, h, d)
        out = cfa.fused_attention(q, k, v, 0.125, False)
        grads = torch.autograd.grad(out, [q, k, v], gout)
    finally:
        cfa.set_projection_route(prev)
    for i, gi in enumerate(grads):
        assert torch.equal(bits(gi.contiguous()), bits(want[:, :, i].transpose(1, 2).contiguous()))


def ws_layout(b, h, s, d):
    """Byte offsets of the backward workspace's parts (restated from fattn_api.cpp's
    workspace_layout; the library's reported sizes pin it)."""
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    tiles, nkb = b * h * (-(-s // 16)), -(-s // 64)
    lay = {"ctrl": 0, "d": 256}
    lay["turn"] = lay["d"] + up(b * h * s * 4)
    lay["part"] = lay["turn"] + up(tiles * 4)
    lay["arrive"] = lay["part"] + up(nkb * tiles * 16 * d * 4)
    lay["done"] = lay["arrive"] + up(b * h * nkb * 8)
    lay["epoch"] = lay["done"] + up(tiles * 8)
    L = _lib.lib()
    assert L.fattn_bwd_workspace_min_bytes(b, h, s, d) == lay["part"]
    assert L.fattn_bwd_workspace_split_bytes(b, h, s, d) == lay["epoch"] + 256
    return lay


def step2_summed_tiles(qkv, dout, h, d, causal, grad_want):
    """Runs the split backward kernel by kernel on the qkv views; returns the [b h, ntile] mask of
    the query tiles step 2 summed itself (done flag == the launch's epoch, read before step 3
    clears them), and checks that the three steps give `grad_want` bit for bit."""
    b, s, _ = qkv.shape
    L = _lib.lib()
    P = _p
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    stream = _st(qkv)
    o = torch.empty(b, s, h * d, device=qkv.device)
    lse = torch.empty(b, h, s, device=qkv.device)
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, 0.125, int(causal), st, st,
                               st, stream))
    lay = ws_layout(b, h, s, d)
    n = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
    ws = torch.zeros(n, dtype=torch.uint8, device=qkv.device)
    dqkv = torch.empty_like(qkv)
    _lib.check(L.fattn_bwd_prep_f32(P(o), P(dout), gst, P(ws), n, b, h, s, d, stream))
    _lib.check(L.fattn_bwd_main_f32(qp, kp, vp, P(o), P(dout), P(lse), P(dqkv), P(ws), n, b, h, s,
                                    d, 0.125, int(causal), st, st, st, gst, stream))
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    ntile = -(-s // 16)
    done = raw[lay["done"]:lay["done"] + b * h * ntile * 8].view(np.uint64).reshape(b * h, ntile)
    epoch = raw[lay["epoch"]:lay["epoch"] + 8].view(np.uint64)[0]
    assert epoch != 0
    _lib.check(L.fattn_bwd_dq_f32(P(dqkv), P(ws), n, b, h, s, d, 0.125, int(causal), stream))
    torch.cuda.synchronize()
    assert torch.equal(bits(dqkv), bits(grad_want))
    return done == epoch


def _hook(name):
    """A test hook of libfattn.so. The hooks act only when FATTN_TEST_HOOKS=1 was set before the
    library loaded (tests/conftest.py sets it): checked first, through the read-only state query."""
    L = _lib.lib()
    L.fattn_internal_hooks.argtypes = [ctypes.POINTER(ctypes.c_int64)]
    L.fattn_internal_hooks.restype = ctypes.c_int
    state = (ctypes.c_int64 * 3)()
    assert L.fattn_internal_hooks(state) == 1, "test hooks are off in this process"
    f = getattr(L, name)
    f.argtypes = [ctypes.c_int]
    f.restype = ctypes.c_int
    return f


@pytest.mark.parametrize("causal", [False, True])
def test_step2_sums_equal_step3_sums_at_scale(orc, cuda, causal):
    """Step 2's sums read the dQ partials at device scope after a device-scope arrival flag, in
    the same kernel; step 3 reads them after a kernel boundary. At config 2's shape (384 heads,
    every tile summed in step 2, so that no step 3 follows an eager backward), the backward with
    step 2's sums switched off (step 3 sums every tile) must give the same bits, on three runs;
    non-causal also with the summing workgroups of XCD x given the heads of XCD x + 3 (a test
    hook), so that every sum reads partials written on another XCD."""
    sums, shift = _hook("fattn_internal_step2_sums"), _hook("fattn_internal_sum_shift")
    x, dout, qkv, g = seeded_qkv(orc, 64, 6, 240, 5, cuda)
    res = {}
    modes = [(1, 0), (0, 0)] * 3 + ([(1, 3), (1, 3)] if not causal else [])
    for on, sh in modes:
        prev, prev_sh = sums(on), shift(sh)
        try:
            _, grad = run("fused_qkv", qkv, g, 6, 64, causal, 0.125)
        finally:
            sums(prev)
            shift(prev_sh)
        b = bits(grad)
        key = (on, sh)
        if key in res:
            assert torch.equal(b, res[key]), f"step 2 sums {key}: reruns differ"
        res[key] = b
    for key, b in res.items():
        say(f"  causal={causal}: sums/shift {key} == step 3 alone: {torch.equal(b, res[(0, 0)])}")
        assert torch.equal(b, res[(0, 0)]), key


@pytest.mark.parametrize("d", [32, 64])
def test_step2_sums_across_xcds(orc, cuda, d):
    """Every non-causal sum reading partials from another XCD (the shift hook, each of 1..7) at b 2
    h 16 s 300: the gradient equals step 3's sums bit for bit, and after step 2 alone every tile's
    done flag holds the launch's epoch (step 2 summed it)."""
    sums, shift = _hook("fattn_internal_step2_sums"), _hook("fattn_internal_sum_shift")
    h, s = 16, 300
    x, dout, qkv, g = seeded_qkv(orc, 2, h, s, 40 + d, cuda, d=d)
    prev = sums(0)
    try:
        _, want = run("fused_qkv", qkv, g, h, d, False, 0.125)
    finally:
        sums(prev)
    for sh in range(1, 8):
        prev_sh = shift(sh)
        try:
            _, grad = run("fused_qkv", qkv, g, h, d, False, 0.125)
            summed = step2_summed_tiles(qkv, g, h, d, False, want)
        finally:
            shift(prev_sh)
        say(f"  d{d} shift {sh}: equal {torch.equal(bits(grad), bits(want))}, "
            f"step 2 summed {int(summed.sum())} of {summed.size}")
        assert torch.equal(bits(grad), bits(want)), f"shift {sh}"
        assert summed.all(), f"shift {sh}"


@pytest.mark.parametrize("d,h,causal,final", [(64, 8, False, True), (64, 9, False, True),
                                              (64, 6, True, True), (64, 5, True, True),
                                              (128, 9, False, True), (128, 6, True, True),
                                              (64, 9, False, False), (128, 5, True, False)])
def test_step3_runs_only_where_needed(orc, cuda, d, h, causal, final):
    """fattn_bwd_f32 with a split workspace, eager: where step 2 sums the dQ tiles (every shape
    here) no step 3 follows, so the done flags keep the launch's epoch; with step 2's sums
    switched off by the test hook (final False) step 3 runs and leaves the flags zeroed. The
    gradient equals the kernel-level steps 1-3 bit for bit either way."""
    b, s = 1, 240
    x, dout, qkv, g = seeded_qkv(orc, b, h, s, 60 + h, cuda, d=d)
    sums = _hook("fattn_internal_step2_sums")
    prev = sums(1 if final else 0)
    try:
        _step3_case(orc, cuda, b, h, s, d, causal, final, qkv, g)
    finally:
        sums(prev)


def _step3_case(orc, cuda, b, h, s, d, causal, final, qkv, g):
    L = _lib.lib()
    P = _p
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    stream = _st(qkv)
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, 0.125, int(causal), st, st,
                               st, stream))
    lay = ws_layout(b, h, s, d)
    n = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
    ws = torch.zeros(n, dtype=torch.uint8, device=cuda)
    dqkv = torch.empty_like(qkv)
    _lib.check(L.fattn_bwd_f32(qp, kp, vp, P(o), P(g), P(lse), P(dqkv), P(ws), n, b, h, s, d,
                               0.125, int(causal), st, st, st, gst, stream))
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    ntile = -(-s // 16)
    done = raw[lay["done"]:lay["done"] + b * h * ntile * 8].view(np.uint64)
    epoch = raw[lay["epoch"]:lay["epoch"] + 8].view(np.uint64)[0]
    say(f"  h{h} causal={causal}: done flags at the epoch {int((done == epoch).sum())} of "
        f"{done.size}, zero {int((done == 0).sum())}")
    if final:
        assert epoch != 0 and (done == epoch).all(), "step 3 ran, or step 2 left tiles"
    else:
        assert (done == 0).all(), "step 3 did not clear the flags"
    _, want = run("fused_qkv", qkv, g, h, d, causal, 0.125)
    assert torch.equal(bits(dqkv), bits(want))
    if final:
        assert step2_summed_tiles(qkv, g, h, d, causal, want).all()


@pytest.mark.parametrize("d,b,h", [(32, 2, 4), (64, 2, 4), (64, 1, 6), (32, 3, 3), (128, 2, 4),
                                   (128, 1, 6)])
def test_causal_dq_sums_match_turns(orc, cuda, d, b, h):
    """Causal split backward (every key block sums the dQ tiles it completes, waiting only for the
    key blocks those tiles need; at b h 6 or 9 those run on other XCDs) against the turn
    hand-over, which sums dQ in place in the same key-block order: O and the whole gradient
    bit-identical, and within the fp64 bar."""
    s = 200
    rng = np.random.default_rng(5 + d)
    x = rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)
    w = rng.standard_normal((b, s, h * d)).astype(np.float32)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    res = {}
    for mode in ("split", "turns"):
        say(f"causal sums d{d} {mode}")
        prev = cfa.set_dq_sum(mode)
        try:
            res[mode] = run("fused_qkv", qkv, wt, h, d, True, 0.125)
        finally:
            cfa.set_dq_sum(prev)
    (o1, g1), (o2, g2) = res["split"], res["turns"]
    assert torch.equal(bits(o1), bits(o2)) and torch.equal(bits(g1), bits(g2))
    ref_out, _, ref_grad = oracle_qkv(orc, x, w, h, d, True, np.float64, 0.125)
    check_errors(orc, o1, g1, ref_out, ref_grad, f"causal d{d}", d=d)
    summed = step2_summed_tiles(qkv, wt, h, d, True, g1)
    say(f"  step 2 summed {int(summed.sum())} of {summed.size} tiles")
    assert summed.all(), "causal: step 2 sums every tile"


@pytest.mark.parametrize("causal", [False, True])
def test_graph_replays(orc, cuda, causal):
    """Forward and backward (qkv entries of the C ABI) captured in one HIP graph and replayed on
    new inputs each time: every replay equals an eager run on the same inputs bit for bit. A replay
    repeats its launch arguments, step 2's dQ-sum epoch included, so this holds only because each
    backward leaves the sums' state clear (with stale state, a replay's sums would take the
    previous replay's partials). Eager work (new inputs, an eager run on the same workspace) and
    synchronisations run between the replays."""
    b, h, s, d = 8, 6, 240, 64  # step 2 sums every dQ tile, causal too
    L = _lib.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    qkv = torch.empty(b, s, 3 * h * d, device=cuda)
    dout = torch.empty(b, s, h * d, device=cuda)
    out = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    dqkv = torch.empty_like(qkv)
    nbytes = L.fattn_bwd_workspace_bytes(b, h, s, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    shape, strides = _lib.arr(qkv.shape), _lib.arr(qkv.stride())
    gshape, gstrides = _lib.arr(dout.shape), _lib.arr(dout.stride())
    ci = 1 if causal else 0

    def step():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.fattn_qkv_forward(P(qkv), 0, shape, strides, h, 0.125, ci, P(out), P(lse),
                                       st))
        _lib.check(L.fattn_qkv_backward(P(qkv), 0, shape, strides, h, 0.125, ci, P(out), P(lse),
                                        P(dout), 0, gshape, gstrides, P(dqkv), P(ws), nbytes, st))

    gen = torch.Generator().manual_seed(7)
    qkv.copy_(torch.randn(qkv.shape, generator=gen))
    dout.copy_(torch.randn(dout.shape, generator=gen))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up on a side stream before capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for r in range(4):
        say(f"graph replay {r} causal={causal}")
        qkv.copy_(torch.randn(qkv.shape, generator=gen))
        dout.copy_(torch.randn(dout.shape, generator=gen))
        dqkv.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got_o, got_g = bits(out).clone(), bits(dqkv).clone()
        dqkv.zero_()
        step()  # eager, same inputs, same workspace
        torch.cuda.synchronize()
        assert torch.equal(got_o, bits(out)), f"replay {r}: O"
        assert torch.equal(got_g, bits(dqkv)), f"replay {r}: gradient"
    # the last replay against the fp64 oracle
    x, w = qkv.cpu().numpy(), dout.cpu().numpy()
    ref_out, _, ref_grad = oracle_qkv(orc, x, w, h, d, causal, np.float64, 0.125)
    check_errors(orc, out, dqkv, ref_out, ref_grad, "after replays")


# --- head_dim 32 and 128 (the reference's roadmap, ROADMAP.md:76-79) ------------------------

@pytest.mark.parametrize("d", [32, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dims(orc, cuda, d, causal, dq_sum):
    """The d-templated kernels against the fp64 oracle on seeded N(0, 1) inputs, tails of every
    kind (single key, partial 16-query tiles, partial 64-key blocks, several key blocks), both
    entry points bit-identical, and bit-identical reruns."""
    rng = np.random.default_rng(d + int(causal))
    scale = 1.0 / d ** 0.5
    for (b, s, h) in [(2, 1, 2), (2, 17, 3), (1, 64, 2), (2, 100, 2), (1, 240, 3), (1, 333, 2)]:
        x = rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)
        w = rng.standard_normal((b, s, h * d)).astype(np.float32)
        say(f"head_dim {d} b{b} s{s} h{h} causal={causal} {dq_sum}")
        ref_out, _, ref_grad = oracle_qkv(orc, x, w, h, d, causal, np.float64, scale)
        qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
        out, grad = run("fused_qkv", qkv, wt, h, d, causal, scale)
        check_errors(orc, out, grad, ref_out, ref_grad, f"d{d} s{s}", d=d)
        o2, g2 = run("fused", qkv, wt, h, d, causal, scale)
        assert torch.equal(bits(out), bits(o2)) and torch.equal(bits(grad), bits(g2))
        _, g3 = run("fused_qkv", qkv, wt, h, d, causal, scale)
        assert torch.equal(bits(grad), bits(g3))


@pytest.mark.parametrize("d", [32, 128])
def test_head_dims_kernel_level(orc, cuda, d):
    """The generic kernel-level entries (fattn_fwd_f32 / fattn_bwd_f32) take d 32 and 128 and
    give the op level's results bit for bit; the reference-named _d64 entries refuse them."""
    b, s, h = 2, 97, 3
    rng = np.random.default_rng(7 * d)
    x = rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)
    w = rng.standard_normal((b, s, h * d)).astype(np.float32)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    scale = 1.0 / d ** 0.5
    o_ref, g_ref = run("fused_qkv", qkv, wt, h, d, True, scale)
    L = _lib.lib()
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.fattn_fwd_f32_d64(qp, kp, vp, P(o), P(lse), b, h, s, d, scale, 1, st, st, st,
                               stream) == _lib.FATTN_EHEADDIM
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, P(o), P(lse), b, h, s, d, scale, 1, st, st, st,
                               stream))
    n = L.fattn_bwd_workspace_bytes(b, h, s, d)
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)
    dqkv = torch.empty_like(qkv)
    _lib.check(L.fattn_bwd_f32(qp, kp, vp, P(o), P(wt), P(lse), P(dqkv), P(ws), n, b, h, s, d,
                               scale, 1, st, st, st, gst, stream))
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(dqkv, g_ref)


@pytest.mark.parametrize("causal", [False, True])
def test_scale_signs(orc, cuda, causal):
    """Any finite scale, as the reference takes: negative (the forward's running max is taken on
    the scaled scores' order), zero (uniform attention) and a large one (peaked softmax)."""
    rng = np.random.default_rng(11)
    b, s, h, d = 2, 150, 2, 64
    x = rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)
    w = rng.standard_normal((b, s, h * d)).astype(np.float32)
    qkv, wt = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    for scale in (-0.125, 0.0, 0.7):
        say(f"scale {scale} causal={causal}")
        ref_out, ref_lse, ref_grad = oracle_qkv(orc, x, w, h, d, causal, np.float64, scale)
        out, grad = run("fused_qkv", qkv, wt, h, d, causal, scale)
        floor, _ = composed_floor(orc, x, w, h, d, causal, ref_out, ref_grad, scale)
        check_errors(orc, out, grad, ref_out, ref_grad, f"scale {scale}", floor)
        lse = check_lse_all_levels(orc, qkv, h, d, scale, causal, f"scale {scale}", out)
        if scale == 0.0:
            # uniform attention: L_i = ln(number of keys query i sees)
            n = np.arange(1, s + 1) if causal else np.full(s, s)
            want = np.broadcast_to(np.log(n.astype(np.float64)), (b, h, s))
            got = lse.cpu().numpy().astype(np.float64)
            assert np.max(np.abs(got - want)) <= 4e-7 * np.log(s), "L = ln n at scale 0"


# --- operand layouts at random: fused_attention on views the kernels read in place or copy -----

LAYOUTS = ("contig", "bshd", "sbhd", "padded", "misaligned", "oddrow")


def layout_of(kind, vals, rng, cuda):
    """A [b, h, s, d] leaf on the device holding `vals` (float32, C order) in one of the layouts a
    candle caller hands fused_attention: contiguous; a transposed view of [b, s, h, d] (the
    merge-heads layout); a permuted view of [s, b, h, d]; rows padded to d + 4 or d + 8 floats;
    storage offset 1 (not float4-aligned: copied); rows of d + 1 floats (not float4-aligned:
    copied). The bases are made on the device, so the views keep their strides."""
    b, h, s, d = vals.shape
    t = torch.from_numpy(vals).to(cuda)
    if kind == "contig":
        v = t.clone()
    elif kind == "bshd":
        v = t.transpose(1, 2).contiguous().transpose(1, 2)
    elif kind == "sbhd":
        v = t.permute(2, 0, 1, 3).contiguous().permute(1, 2, 0, 3)
    elif kind in ("padded", "oddrow"):
        pad = int(rng.choice([4, 8])) if kind == "padded" else 1
        base = torch.zeros(b, h, s, d + pad, device=cuda)
        base[..., :d] = t
        v = base[..., :d]
    else:
        base = torch.zeros(t.numel() + 1, device=cuda)
        base[1:] = t.reshape(-1)
        v = base[1:].view(b, h, s, d)
    assert torch.equal(v, t), kind
    assert cfa.reads_in_place(v) == (kind not in ("misaligned", "oddrow")), kind
    return v.detach().requires_grad_(True)


def check_against_oracle(orc, got, vals, scale, causal):
    """Output and gradients against the fp64 oracle at the bar of the other parity tests."""
    qn, kn, vn, wn = vals
    ref, floor = {}, {}
    for dtype, dst in ((np.float64, ref), (np.float32, floor)):
        o, l_ = orc.forward(qn, kn, vn, scale, causal, dtype)
        dq, dk, dv = orc.backward(qn, kn, vn, o, l_, wn, scale, causal, dtype)
        dst.update(o=o, dq=dq, dk=dk, dv=dv)
    for name in ("o", "dq", "dk", "dv"):
        r = np.asarray(ref[name], dtype=np.float64)
        if not np.any(r):
            dev, bar = float(np.abs(got[name]).max()), zero_band(qn.shape[-1])
            assert dev <= bar, f"{name} (exactly zero in fp64) max deviation {dev:.3e} > {bar:.1e}"
            continue
        err = orc.rel_fro(got[name], r)
        tol = max(REL_TOL, 1.5 * orc.rel_fro(floor[name], r))
        say(f"  {name}: {err:.2e} (bar {tol:.2e})")
        assert err <= tol, f"{name}: normwise error {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("seed", range(20))
def test_random_layouts(orc, cuda, seed):
    """fused_attention on q, k, v and an output gradient in layouts drawn at random (each operand
    its own), at random b, h, s (1-160), head_dim (32, 64, 128), mask and scale (either sign):
    output and the three gradients against the fp64 oracle (src/lib.rs:241-299) at the bar of the
    other parity tests -- within 2e-6 normwise or 1.5x the fp32 composed path's own error."""
    rng = np.random.default_rng(1000 + seed)
    b, h = int(rng.integers(1, 4)), int(rng.integers(1, 6))
    s, d = int(rng.integers(1, 161)), int(rng.choice([32, 64, 128]))
    causal = bool(rng.integers(0, 2))
    scale = float(rng.choice([-1.0, 1.0]) * rng.uniform(0.05, 0.3))
    kinds = [str(rng.choice(LAYOUTS)) for _ in range(4)]
    say(f"seed {seed}: b {b} h {h} s {s} d {d} causal={causal} scale {scale:.4f} layouts {kinds}")
    vals = [rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(4)]
    q, k, v, w = (layout_of(kd, x, rng, cuda) for kd, x in zip(kinds, vals))
    out = cfa.fused_attention(q, k, v, scale, causal)
    (out * w.detach()).sum().backward()
    torch.cuda.synchronize()
    got = {"o": out.detach().cpu().numpy(), "dq": q.grad.cpu().numpy(),
           "dk": k.grad.cpu().numpy(), "dv": v.grad.cpu().numpy()}
    check_against_oracle(orc, got, vals, scale, causal)


@pytest.mark.parametrize("seed", range(20))
def test_random_qkv_cases(orc, cuda, seed):
    """fused_attention_qkv at random b (1-4), h (1-8), s (1-400), head_dim (32, 64, 128), mask,
    scale (either sign) and dQ-sum mode (auto, split, turns): the output and the three slices of
    the qkv gradient against the fp64 oracle (src/lib.rs:241-299; the operator, src/lib.rs:506-580)."""
    rng = np.random.default_rng(50000 + seed)
    b, h = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    s, d = int(rng.integers(1, 401)), int(rng.choice([32, 64, 128]))
    causal = bool(rng.integers(0, 2))
    scale = float(rng.choice([-1.0, 1.0]) * rng.uniform(0.02, 0.4))
    mode = str(rng.choice(["auto", "split", "turns"]))
    say(f"seed {seed}: b {b} h {h} s {s} d {d} causal={causal} scale {scale:.4f} dq_sum {mode}")
    x = rng.standard_normal((b, s, 3 * h * d)).astype(np.float32)
    wq = rng.standard_normal((b, s, h * d)).astype(np.float32)
    prev = cfa.set_dq_sum(mode)
    try:
        xt = torch.from_numpy(x).to(cuda).requires_grad_(True)
        out = cfa.fused_attention_qkv(xt, h, scale, causal)
        out.backward(torch.from_numpy(wq).to(cuda))
        torch.cuda.synchronize()
    finally:
        cfa.set_dq_sum(prev)
    g = xt.grad.cpu().numpy().reshape(b, s, 3, h, d).transpose(2, 0, 3, 1, 4)
    got = {"o": out.detach().cpu().numpy().reshape(b, s, h, d).transpose(0, 2, 1, 3),
           "dq": g[0], "dk": g[1], "dv": g[2]}
    x5 = x.reshape(b, s, 3, h, d).transpose(2, 0, 3, 1, 4)
    vals = [np.ascontiguousarray(x5[i]) for i in range(3)]
    vals.append(np.ascontiguousarray(wq.reshape(b, s, h, d).transpose(0, 2, 1, 3)))
    check_against_oracle(orc, got, vals, scale, causal)


# --- a very long sequence: the turn hand-over past the workspace cap ------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_very_long_sequence(orc, cuda, causal):
    """One head of s 32816 (not a multiple of 64) through fused_attention_qkv: the split dQ sum
    would need more than the 4 GiB workspace cap and one (b, h) pair cannot be chunked, so the
    backward takes the turn hand-over. O, L and dQ at 48 query rows and dK, dV at 48 key rows
    (the first, the last, random ones) against the oracle's rows (oracle.rows: the composed
    formulas of src/lib.rs:241-299 without [s, s] buffers, bit-identical to the slice-wise
    oracle), at the bar of the other parity tests: within 2e-6 normwise of fp64, or 1.5x the fp32
    composed path's own error on the same rows. Both fp32 paths sum over s terms, so at this
    length that floor is what binds."""
    s, d = 32816, 64
    L = _lib.lib()
    assert L.fattn_bwd_workspace_split_bytes(1, 1, s, d) > 4 << 30
    assert L.fattn_bwd_workspace_bytes(1, 1, s, d) == L.fattn_bwd_workspace_min_bytes(1, 1, s, d)
    rng = np.random.default_rng(32816 + causal)
    x = rng.standard_normal((1, s, 3 * d)).astype(np.float32)
    w = rng.standard_normal((1, s, d)).astype(np.float32)
    say(f"s {s} causal={causal}: turn hand-over")
    qkv = torch.from_numpy(x).to(cuda)
    out, grad = run("fused_qkv", qkv, torch.from_numpy(w).to(cuda), 1, d, causal, 0.125)
    _, lse = forward_qkv_c(qkv, 1, 0.125, causal)
    _, grad2 = run("fused_qkv", qkv, torch.from_numpy(w).to(cuda), 1, d, causal, 0.125)
    assert torch.equal(bits(grad), bits(grad2)), "backward reruns differ"
    rows = np.unique(np.r_[0, s - 1, rng.integers(0, s, 46)])
    keys = np.unique(np.r_[0, s - 1, rng.integers(0, s, 46)])
    q, k, v = (x[0, :, i * d:(i + 1) * d] for i in range(3))
    ref = orc.rows(q, k, v, w[0], 0.125, causal, rows, keys, dtype=np.float64)
    f32 = orc.rows(q, k, v, w[0], 0.125, causal, rows, keys, dtype=np.float32)
    o, g = out.cpu().numpy()[0], grad.cpu().numpy()[0]
    got = (o[rows], lse.cpu().numpy()[0, 0, rows], g[rows, :d], g[keys, d:2 * d], g[keys, 2 * d:])
    check_lse(got[1], ref[1], f32[1], f"s{s}")
    for name, a, r, fl in zip(("o", "dq", "dk", "dv"), got[:1] + got[2:], ref[:1] + ref[2:],
                              f32[:1] + f32[2:]):
        assert np.all(np.isfinite(a)), name
        err, floor = orc.rel_fro(a, r), orc.rel_fro(fl, r)
        bar = max(REL_TOL, 1.5 * floor)
        say(f"  {name}: {err:.2e} (fp32 composed {floor:.2e}, bar {bar:.2e})")
        assert err <= bar, f"{name}: normwise error {err:.3e} > {bar:.3e}"


# --- many (b, h) pairs: large grids ----------------------------------------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_many_pairs(orc, cuda, causal):
    """b 256 x h 128 = 32768 (b, h) pairs of s 40 through fused_attention_qkv: a forward grid of
    32768 workgroups, and a step 2 of 32768 key blocks whose dQ sums run in the same launch
    (non-causal: summing workgroups appended to the grid and planned over the 8 XCDs; causal:
    each key block sums its own tiles). Sampled pairs (the first, the last, random ones) against
    the fp64 oracle at 2e-6, and a bit-identical rerun."""
    b, h, s, d = 256, 128, 40, 64
    gen = torch.Generator(device=cuda).manual_seed(11 + int(causal))
    qkv = torch.randn(b, s, 3 * h * d, generator=gen, device=cuda)
    dout = torch.randn(b, s, h * d, generator=gen, device=cuda)
    say(f"b {b} h {h} s {s} causal={causal}: {b * h} pairs")
    out, grad = run("fused_qkv", qkv, dout, h, d, causal, 0.125)
    _, grad2 = run("fused_qkv", qkv, dout, h, d, causal, 0.125)
    assert torch.equal(bits(grad), bits(grad2)), "backward reruns differ"
    rng = np.random.default_rng(5 + int(causal))
    pairs = sorted({0, b * h - 1, *rng.integers(0, b * h, 10).tolist()})
    check_pairs(orc, qkv, dout, out, grad, h, d, 0.125, causal, pairs,
                f"b{b} h{h} s{s} causal={causal}")


# --- the split dQ sum by chunks of (b, h) (a workspace that holds some pairs' partials) ---------

@pytest.mark.parametrize("causal,d", [(False, 64), (True, 64), (False, 32)])
def test_split_by_chunks_matches_whole(orc, cuda, causal, d):
    """fattn_bwd_f32 with a workspace that holds the split partials of only some (b, h) pairs runs
    steps 2 and 3 per chunk of pairs (causal: equal, 8 | chunk; non-causal: whole rounds of slots), where the chunks are
    large enough to beat the turn hand-over (s 4096: 12 pairs non-causal, 48 causal): the
    gradient equals the whole split's bit for bit (each pair's arithmetic and summation order are
    the same), and the guard word reads 0. Non-causal b h 24 in chunks of 16 and 8; causal b h 96
    in two of 48; d 32 (128-key blocks, three workgroups per CU) b h 48 in two of 24. A workspace
    whose chunks would be smaller takes the turn hand-over: causal, its gradient equals the
    split's bit for bit too. The first pair, one of the last chunk and the last pair are checked
    against the fp64 oracle."""
    b, h, s = (2, 12, 4096) if not causal else (6, 16, 4096)
    pairs = 16 if not causal else 48
    if d == 32:
        b, h, s, pairs = 3, 16, 4096, 24
    L = _lib.lib()
    g = torch.Generator(device=cuda).manual_seed(7)
    qkv = torch.randn(b, s, 3 * h * d, generator=g, device=cuda)
    dout = torch.randn(b, s, h * d, generator=g, device=cuda)
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    stream = _st(qkv)
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, _p(o), _p(lse), b, h, s, d, 0.125, int(causal), st, st,
                               st, stream))

    def backward(n):
        ws = torch.empty(n, dtype=torch.uint8, device=cuda)
        out = torch.full_like(qkv, float("nan"))
        _lib.check(L.fattn_bwd_f32(qp, kp, vp, _p(o), _p(dout), _p(lse), _p(out), _p(ws), n, b, h,
                                   s, d, 0.125, int(causal), st, st, st, gst, stream))
        status = ctypes.c_int(-1)
        _lib.check(L.fattn_bwd_status(_p(ws), n, b, h, s, stream, ctypes.byref(status)))
        assert status.value == 0
        del ws
        return out

    whole_n = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
    whole = backward(whole_n)
    assert torch.isfinite(whole).all()
    check_pairs(orc, qkv, dout, o, whole, h, d, 0.125, causal, (0, b * h - 3, b * h - 1),
                f"b{b} h{h} s{s} d{d} causal={causal}")
    n = L.fattn_bwd_workspace_split_bytes(1, pairs, s, d)
    assert n < whole_n
    say(f"chunks of {pairs} (b, h) causal={causal}: workspace {n >> 20} MiB of {whole_n >> 20}")
    assert torch.equal(bits(backward(n)), bits(whole)), f"chunks of {pairs}"
    if causal:
        small = L.fattn_bwd_workspace_split_bytes(1, 8, s, d)   # chunks of 8: turns instead
        say(f"workspace for 8 pairs ({small >> 20} MiB): the turn hand-over")
        assert torch.equal(bits(backward(small)), bits(whole))


@pytest.mark.parametrize("causal", [False, True])
def test_sum_give_up_raises_guard_and_writes_nan(cuda, causal):
    """A dQ sum in step 2 whose bounded wait gives up (forced from the host by a test hook: the
    sums of one (b, h) pair give up before their first poll, so every kernel still ends normally)
    leaves NaN in exactly that pair's dQ rows and raises the guard word to 3 where no step 3
    follows: a whole launch, and a backward split into chunks of pairs with the pair in the
    first chunk (the second chunk's launch must not clear what the first one raised). Every
    other element is bit-identical to a run without the hook. With step 3 to follow (the kernel-level steps), step 3 sums that pair's tiles: the
    gradient is the hookless one and the guard word reads 0."""
    b, h, s, d = (2, 12, 4096, 64) if not causal else (6, 16, 4096, 64)
    pairs = 16 if not causal else 48          # chunks: 16 + 8 non-causal, 48 + 48 causal
    victim = 3                                # a pair of the first chunk
    L = _lib.lib()
    give_up = _hook("fattn_internal_sum_give_up")
    g = torch.Generator(device=cuda).manual_seed(11)
    qkv = torch.randn(b, s, 3 * h * d, generator=g, device=cuda)
    dout = torch.randn(b, s, h * d, generator=g, device=cuda)
    st = _lib.arr([s * 3 * h * d, d, 3 * h * d])
    gst = _lib.arr([s * h * d, d, h * d])
    qp, kp, vp = (ctypes.c_void_p(qkv.data_ptr() + i * h * d * 4) for i in range(3))
    stream = _st(qkv)
    o = torch.empty(b, s, h * d, device=cuda)
    lse = torch.empty(b, h, s, device=cuda)
    _lib.check(L.fattn_fwd_f32(qp, kp, vp, _p(o), _p(lse), b, h, s, d, 0.125, int(causal), st, st,
                               st, stream))

    def status_of(ws, n):
        status = ctypes.c_int(-1)
        _lib.check(L.fattn_bwd_status(_p(ws), n, b, h, s, stream, ctypes.byref(status)))
        return status.value

    def backward(n, kernel_level=False):
        ws = torch.empty(n, dtype=torch.uint8, device=cuda)
        out = torch.full_like(qkv, float("nan"))
        if kernel_level:
            _lib.check(L.fattn_bwd_main_f32(qp, kp, vp, _p(o), _p(dout), _p(lse), _p(out), _p(ws),
                                            n, b, h, s, d, 0.125, int(causal), st, st, st, gst,
                                            stream))
            _lib.check(L.fattn_bwd_dq_f32(_p(out), _p(ws), n, b, h, s, d, 0.125, int(causal),
                                          stream))
        else:
            _lib.check(L.fattn_bwd_f32(qp, kp, vp, _p(o), _p(dout), _p(lse), _p(out), _p(ws), n,
                                       b, h, s, d, 0.125, int(causal), st, st, st, gst, stream))
        return out, status_of(ws, n)

    whole_n = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
    chunk_n = L.fattn_bwd_workspace_split_bytes(1, pairs, s, d)
    ref, st0 = backward(whole_n)
    assert st0 == 0 and torch.isfinite(ref).all()
    vb, vh = divmod(victim, h)
    mask = torch.zeros(b, s, 3, h, d, dtype=torch.bool, device=cuda)
    mask[vb, :, 0, vh] = True                 # the pair's dQ rows
    mask = mask.view_as(ref)
    prev = give_up(victim)
    try:
        for name, n, level in (("whole launch", whole_n, False), ("chunks", chunk_n, False),
                               ("kernel-level steps", whole_n, True)):
            say(f"give-up pair {victim} (b {vb}, h {vh}) causal={causal}: {name}")
            got, status = backward(n, level)
            if level:
                assert status == 0, f"{name}: guard {status}"
                assert torch.equal(bits(got), bits(ref)), f"{name}: step 3 did not sum the pair"
                continue
            assert status == 3, f"{name}: guard word {status}, expected 3"
            assert torch.isnan(got[mask]).all(), f"{name}: the pair's dQ rows are not all NaN"
            assert torch.equal(bits(got[~mask]), bits(ref[~mask])), f"{name}: other elements"
    finally:
        give_up(prev)
    again, st1 = backward(chunk_n)            # the hook off again: the next backward is clean
    assert st1 == 0 and torch.equal(bits(again), bits(ref))
