"""The C-ABI boundary without a GPU: the library loads, exports every entry point
include/fattn.h declares, and rejects bad arguments with the reference's conditions and
messages before touching any device (no compute calls here).

The rejected inputs mirror the reference's own error paths: head_dim != 64 (src/cuda.rs:85-93),
rows not 16-byte aligned (src/lib.rs:431-435, :533-538), a last dimension not 3 x heads x d
(src/lib.rs:193-197), a non-contiguous last dimension (src/lib.rs:200-205, :182-187), mismatched
q/k/v shapes (src/lib.rs:209-219), and the audit's empty-input (B2) and grid-range (B4) cases.
"""
from __future__ import annotations

import ctypes
import re

import pytest
import torch

from conftest import REPO

import candle_fused_attn as cfa
from candle_fused_attn import _lib

BAD = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails validation first
ODD = ctypes.c_void_p(0x1004)   # 4-byte aligned, not 16


def header_symbols():
    text = (REPO / "include" / "fattn.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)  # declarations only, not comments
    return sorted(set(re.findall(r"\b(fattn_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    declared = header_symbols()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(L, name), name
    assert sorted(_lib.EXPORTS) == declared
    assert "gfx950" in _lib.version()


def a3(*x):
    return _lib.arr(x)


def test_workspace_size_is_aligned_and_monotone():
    L = _lib.lib()
    n1 = L.fattn_bwd_workspace_bytes(64, 6, 240, 64)
    lo = L.fattn_bwd_workspace_min_bytes(64, 6, 240, 64)
    hi = L.fattn_bwd_workspace_split_bytes(64, 6, 240, 64)
    assert n1 % 256 == 0 and lo % 256 == 0 and hi % 256 == 0
    # minimum: control + D (64*6*240 f32) + turns (64*6*15 i32)
    assert lo >= 64 * 6 * 240 * 4 + 64 * 6 * 15 * 4 + 256
    # split: plus one 16 x d f32 partial per key block (4) and query tile (15) of each (b, h), a
    # u64 arrival slot per key block and a u64 done flag per query tile (both 256-byte multiples
    # here) and 256 bytes for the epoch of the last step 2 launch
    for d in (32, 64, 128):
        assert L.fattn_bwd_workspace_min_bytes(64, 6, 240, d) == lo
        assert (L.fattn_bwd_workspace_split_bytes(64, 6, 240, d)
                == lo + 4 * 64 * 6 * 15 * 16 * d * 4 + 64 * 6 * 4 * 8 + 64 * 6 * 15 * 8 + 256)
    assert n1 == hi  # 94 MB: below the split cap
    assert L.fattn_bwd_workspace_bytes(64, 6, 241, 64) >= n1
    assert L.fattn_bwd_workspace_bytes(-1, 6, 240, 64) == 0
    assert L.fattn_bwd_workspace_min_bytes(-1, 6, 240, 64) == 0
    assert L.fattn_bwd_workspace_bytes(64, 6, 240, 48) == 0      # head_dim not built
    # Past FATTN_SPLIT_MAX_BYTES (4 GiB), at d <= 64: the split sum of equal chunks of (b, h),
    # each chunk's state in a workspace laid out for that many pairs (split_bytes(1, chunk, ...));
    # at d 128 the minimum (the turn hand-over).
    cap = 4 << 30
    assert L.fattn_bwd_workspace_split_bytes(1, 64, 16384, 64) > cap
    # 1 GiB of partials per pair: 3 fit, but their 3 x 128 key blocks (of 128 keys) fill less than
    # one round of the 512 workgroup slots: the minimum (turns)
    assert L.fattn_bwd_workspace_split_bytes(1, 3, 16384, 64) <= cap
    assert L.fattn_bwd_workspace_split_bytes(1, 4, 16384, 64) > cap
    assert (L.fattn_bwd_workspace_bytes(1, 64, 16384, 64)
            == L.fattn_bwd_workspace_min_bytes(1, 64, 16384, 64))
    # The size takes no mask: the larger of the two rules' chunks. 256 MiB per pair, 15 fit:
    # non-causal, 64 key blocks of 128 keys per pair, so multiples of 8 pairs fill whole rounds of
    # the 512 slots: 8; causal, 15 pairs are under its minimum (four rounds of 768 slots in 64-key
    # blocks: 24 pairs): none. Chunks of 8.
    assert (L.fattn_bwd_workspace_bytes(4, 16, 8192, 64)
            == L.fattn_bwd_workspace_split_bytes(1, 8, 8192, 64))
    # 64 MiB per pair, 63 fit: non-causal, 32 key blocks of 128 keys per pair, whole rounds of 512
    # slots in multiples of 16 pairs: 48; causal, 3 equal chunks of 128 pairs: 43. So 48.
    assert (L.fattn_bwd_workspace_bytes(8, 16, 4096, 64)
            == L.fattn_bwd_workspace_split_bytes(1, 48, 4096, 64))
    assert L.fattn_bwd_workspace_split_bytes(1, 64, 4096, 64) > cap
    # d 32, 32 MiB per pair, 127 fit: non-causal, 32 key blocks of 128 keys per pair, whole rounds
    # of 768 slots in multiples of 24 pairs: 120; causal, 2 equal chunks: 64. So 120.
    assert L.fattn_bwd_workspace_split_bytes(8, 16, 4096, 32) > cap
    assert (L.fattn_bwd_workspace_bytes(8, 16, 4096, 32)
            == L.fattn_bwd_workspace_split_bytes(1, 120, 4096, 32))
    assert (L.fattn_bwd_workspace_bytes(8, 16, 4096, 128)
            == L.fattn_bwd_workspace_min_bytes(8, 16, 4096, 128))


def test_head_dim_gate_before_alignment():
    L = _lib.lib()
    st = a3(6 * 24, 6, 3 * 6 * 24 // 1)
    # qkv with head_dim 6 at a misaligned offset: the head_dim error comes first (audit B3)
    rc = L.fattn_qkv_forward(BAD, 1, a3(2, 5, 3 * 4 * 6), a3(5 * 72, 72, 1), 4, 0.3, 0, BAD,
                             BAD, None)
    assert rc == _lib.FATTN_EHEADDIM
    assert "head_dim 32, 64 or 128, got 6" in _lib.last_error()
    assert _lib.last_error().startswith("fused_attention")
    # The reference-named kernel-level entries keep its check (head_dim 64 only); the generic
    # ones take 32, 64, 128.
    rc = L.fattn_fwd_f32_d64(BAD, BAD, BAD, BAD, BAD, 1, 1, 8, 32, 0.1, 0, st, st, st, None)
    assert rc == _lib.FATTN_EHEADDIM
    assert "head_dim 64, got 32" in _lib.last_error()
    rc = L.fattn_fwd_f32(BAD, BAD, BAD, BAD, BAD, 1, 1, 8, 96, 0.1, 0, st, st, st, None)
    assert rc == _lib.FATTN_EHEADDIM
    assert "head_dim 32, 64 or 128, got 96" in _lib.last_error()
    ok = a3(8 * 32, 32, 32)
    rc = L.fattn_fwd_f32(ODD, BAD, BAD, BAD, BAD, 1, 1, 8, 32, 0.1, 0, ok, ok, ok, None)
    assert rc == _lib.FATTN_EALIGN   # past the head_dim gate: the misaligned pointer


def test_qkv_geometry_errors():
    L = _lib.lib()
    rc = L.fattn_qkv_forward(BAD, 0, a3(2, 5, 100), a3(500, 100, 1), 3, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EINVAL
    assert _lib.last_error() == ("fused_attention_qkv: last dimension 100 is not 3 x 3 heads x "
                                 "head_dim")
    rc = L.fattn_qkv_forward(BAD, 0, a3(2, 5, 384), a3(1920, 384, 1), 0, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EINVAL
    rc = L.fattn_qkv_forward(BAD, 0, a3(2, 5, 384), a3(1920, 384, 2), 2, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EINVAL
    assert "last dimension must be contiguous" in _lib.last_error()


def test_qkv_alignment_errors():
    L = _lib.lib()
    # offset 1, strides aligned
    rc = L.fattn_qkv_forward(BAD, 1, a3(2, 5, 384), a3(1920, 384, 1), 2, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EALIGN
    assert _lib.last_error() == "fused_attention_qkv: rows must be 16-byte aligned"
    # seq stride not a multiple of 4
    rc = L.fattn_qkv_forward(BAD, 0, a3(2, 5, 384), a3(1930, 386, 1), 2, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EALIGN
    # base pointer misaligned
    rc = L.fattn_qkv_forward(ODD, 0, a3(2, 5, 384), a3(1920, 384, 1), 2, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EALIGN


def test_general_path_errors():
    L = _lib.lib()
    sh, st = a3(2, 3, 5, 64), a3(960, 320, 64, 1)
    other = a3(2, 3, 6, 64)
    rc = L.fattn_forward(BAD, 0, sh, st, BAD, 0, other, st, BAD, 0, sh, st, 0.1, 0, BAD, BAD,
                         None)
    assert rc == _lib.FATTN_EINVAL
    assert "must share one [b, h, s, d] shape" in _lib.last_error()
    rc = L.fattn_forward(BAD, 0, sh, a3(960, 320, 64, 2), BAD, 0, sh, st, BAD, 0, sh, st, 0.1,
                         0, BAD, BAD, None)
    assert rc == _lib.FATTN_EINVAL
    assert "d contiguous expected" in _lib.last_error()
    rc = L.fattn_forward(BAD, 2, sh, st, BAD, 0, sh, st, BAD, 0, sh, st, 0.1, 0, BAD, BAD, None)
    assert rc == _lib.FATTN_EALIGN
    assert _lib.last_error() == "fused_attention: rows must be 16-byte aligned"
    sh48 = a3(2, 3, 5, 48)   # a head_dim the kernels are not built for
    rc = L.fattn_forward(BAD, 0, sh48, st, BAD, 0, sh48, st, BAD, 0, sh48, st, 0.1, 0, BAD,
                         BAD, None)
    assert rc == _lib.FATTN_EHEADDIM


def test_backward_argument_errors():
    L = _lib.lib()
    sh, st = a3(2, 5, 384), a3(1920, 384, 1)
    # gradient of the wrong shape
    rc = L.fattn_qkv_backward(BAD, 0, sh, st, 2, 0.1, 0, BAD, BAD, BAD, 0, a3(2, 5, 100),
                              a3(500, 100, 1), BAD, BAD, 1 << 20, None)
    assert rc == _lib.FATTN_EINVAL
    assert "rank-3 gradient" in _lib.last_error()
    # workspace too small
    rc = L.fattn_qkv_backward(BAD, 0, sh, st, 2, 0.1, 0, BAD, BAD, BAD, 0, a3(2, 5, 128),
                              a3(640, 128, 1), BAD, ctypes.c_void_p(0x10000), 16, None)
    assert rc == _lib.FATTN_EWORKSPACE
    # workspace misaligned
    rc = L.fattn_qkv_backward(BAD, 0, sh, st, 2, 0.1, 0, BAD, BAD, BAD, 0, a3(2, 5, 128),
                              a3(640, 128, 1), BAD, ctypes.c_void_p(0x10010), 1 << 20, None)
    assert rc == _lib.FATTN_EWORKSPACE
    # general path: gradient of the wrong rank/shape
    sh4, st4 = a3(2, 3, 5, 64), a3(960, 320, 64, 1)
    rc = L.fattn_backward(BAD, 0, sh4, st4, BAD, 0, sh4, st4, BAD, 0, sh4, st4, 0.1, 0, BAD,
                          BAD, BAD, 0, a3(2, 3, 5, 64), a3(960, 192, 64, 1), BAD, BAD, 1 << 20,
                          None)
    assert rc == _lib.FATTN_EINVAL
    assert "rank-4 gradient" in _lib.last_error()


def test_empty_inputs_are_a_no_op():
    """Audit B2: empty inputs give empty outputs on every entry point (no launch, no error)."""
    L = _lib.lib()
    for shape in ((0, 5, 384), (2, 0, 384)):
        rc = L.fattn_qkv_forward(None, 0, a3(*shape), a3(1920, 384, 1), 2, 0.1, 0, None, None,
                                 None)
        assert rc == 0, _lib.last_error()
        rc = L.fattn_qkv_backward(None, 0, a3(*shape), a3(1920, 384, 1), 2, 0.1, 1, None, None,
                                  None, 0, a3(shape[0], shape[1], 128), a3(640, 128, 1), None,
                                  None, 0, None)
        assert rc == 0, _lib.last_error()
    sh = a3(2, 0, 5, 64)
    st = a3(960, 320, 64, 1)
    rc = L.fattn_forward(None, 0, sh, st, None, 0, sh, st, None, 0, sh, st, 0.1, 0, None, None,
                         None)
    assert rc == 0
    rc = L.fattn_fwd_f32_d64(None, None, None, None, None, 0, 3, 7, 64, 0.1, 0, st, st, st,
                             None)
    assert rc == 0


def test_range_limits():
    """Audit B4: sizes beyond the kernels' index range are a clean error, not a launch failure."""
    L = _lib.lib()
    st = a3(0, 0, 64)
    rc = L.fattn_fwd_f32_d64(BAD, BAD, BAD, BAD, BAD, 1 << 20, 1 << 8, 1 << 8, 64, 0.1, 0, st,
                             st, st, None)
    assert rc == _lib.FATTN_ERANGE
    assert "exceeds" in _lib.last_error()
    # 65,536 batches (the reference's gridDim.z limit) is fine here: the grid is one-dimensional
    ws = L.fattn_bwd_workspace_bytes(65536, 1, 1, 64)
    assert ws > 0


def test_python_api_refuses_cpu_and_non_f32():
    """No CPU fallback: a CPU tensor or a non-f32 dtype is an error, never a silent path."""
    x = torch.zeros(2, 5, 384)
    with pytest.raises(cfa.FusedAttentionError, match="not on a HIP device"):
        cfa.fused_attention_qkv(x, 2, 0.125, False)
    q = torch.zeros(2, 2, 5, 64)
    with pytest.raises(cfa.FusedAttentionError, match="not on a HIP device"):
        cfa.fused_attention(q, q, q, 0.125, False)
    with pytest.raises(cfa.FusedAttentionError, match="f32 only"):
        cfa.fused_attention_qkv(x.double(), 2, 0.125, False)


def test_alignment_predicates():
    qkv = torch.zeros(2, 5, 3 * 2 * 64)
    assert cfa.reads_in_place(qkv)
    assert not cfa.reads_in_place(qkv[:, :, 1:])         # offset 1
    q = qkv.reshape(2, 5, 3, 2, 64)[:, :, 0].transpose(1, 2)  # head view of the projection
    assert cfa.float4_aligned(q) and cfa.reads_in_place(q)
    buf = torch.zeros(16, 1024, 16, 64)
    assert cfa.float4_aligned(buf.transpose(1, 2))       # config 5's views are read in place
    odd = torch.zeros(2, 3, 5, 66)[..., :64]
    assert cfa.float4_aligned(odd) is False              # seq stride 66 is not a multiple of 4
    assert cfa.CUDA_HEAD_DIM == 64 and cfa.HIP_HEAD_DIMS == (32, 64, 128)


def test_projection_views_predicate():
    """fused_attention routes q, k, v to the projection's op only when they are exactly its
    head-split views and every gradient would reach the projection either way."""
    b, s, h, d = 2, 5, 3, 64

    def views(qkv):
        x = qkv.view(b, s, 3, h, d)
        return [x[:, :, i].transpose(1, 2) for i in range(3)]

    qkv = torch.zeros(b, s, 3 * h * d, requires_grad=True)
    q, k, v = views(qkv)
    assert cfa.qkv_projection_of(q, k, v) is qkv
    with torch.no_grad():                                 # inference: no gradients to route
        assert cfa.qkv_projection_of(*views(qkv)) is qkv
    assert cfa.qkv_projection_of(q, v, k) is None         # parts out of order
    assert cfa.qkv_projection_of(q, k, k) is None
    other = torch.zeros(b, s, 3 * h * d)
    assert cfa.qkv_projection_of(q, k, views(other)[2]) is None       # another projection
    q2 = q.detach().requires_grad_(True)                  # a leaf of its own: keeps its gradient
    assert cfa.qkv_projection_of(q2, k, v) is None
    q3, k3, v3 = views(qkv)
    q3.retain_grad()                                      # a view that keeps its own gradient
    assert cfa.qkv_projection_of(q3, k3, v3) is None
    for i in range(3):                                    # a backward hook on any one view
        hooked = views(qkv)
        hooked[i].register_hook(lambda g: g)
        assert cfa.qkv_projection_of(*hooked) is None, f"hook on view {i}"
    wide = torch.zeros(b, s, 3 * h * d + 4)[..., : 3 * h * d]       # not a contiguous projection
    parts = [wide[..., i * h * d:(i + 1) * h * d].unflatten(-1, (h, d)).transpose(1, 2)
             for i in range(3)]
    assert cfa.qkv_projection_of(*parts) is None
    odd = torch.zeros(b, s, 3 * 3 * 48)                   # head_dim 48: not a kernel's
    x48 = odd.view(b, s, 3, 3, 48)
    assert cfa.qkv_projection_of(*[x48[:, :, i].transpose(1, 2) for i in range(3)]) is None


def test_slice_offsets_must_fit_32_bits():
    """The kernels address one (batch, head) slice with 32-bit offsets: a slice spanning more
    than 4 GiB is refused up front (no launch)."""
    L = _lib.lib()
    st = a3(0, 0, 1 << 28)   # seq stride 2^28 floats = 1 GiB per row
    ok = a3(0, 0, 64)
    rc = L.fattn_fwd_f32_d64(BAD, BAD, BAD, BAD, BAD, 1, 1, 8, 64, 0.1, 0, ok, st, ok, None)
    assert rc == _lib.FATTN_ERANGE
    assert "4 GiB" in _lib.last_error()


def test_step1_grid_uses_64_bit_thread_indices():
    """Step 1 runs b h s / 16 workgroups of 256 threads at d 64: from b h s = 2^27 rows on, a
    32-bit thread index would wrap negative (its counter clear would write before the buffer).
    The kernel indexes threads in 64 bits, so the range check admits such shapes: a call at
    2^27 rows passes it and fails only at the (missing) workspace, before any launch; past the
    int32 row limit the range check refuses."""
    L = _lib.lib()
    st = a3(0, 0, 64)
    rows = 1 << 27
    for b, h, s in ((1, 1 << 7, 1 << 20), (1 << 7, 1, 1 << 20), (1 << 10, 1 << 10, 1 << 7)):
        assert b * h * s == rows
        rc = L.fattn_bwd_prep_f32(BAD, BAD, st, None, 0, b, h, s, 64, None)
        assert rc == _lib.FATTN_EWORKSPACE, _lib.last_error()
    rc = L.fattn_bwd_prep_f32(BAD, BAD, st, None, 0, 1 << 11, 1 << 10, 1 << 10, 64, None)
    assert rc == _lib.FATTN_ERANGE
    assert "exceeds i32 indexing" in _lib.last_error()


def test_step1_is_a_no_op_where_step2_forms_d():
    """With a split-size workspace step 2 forms D = rowsum(dO o O) itself at d <= 64, and at d 128
    up to four 64-key blocks per (b, h) (s <= 256): fattn_bwd_prep_f32 then returns 0 after its
    checks, without a launch (so it runs here, with no device and pointers never dereferenced)."""
    L = _lib.lib()
    for b, h, s, d in ((2, 3, 240, 64), (2, 3, 240, 32), (2, 3, 240, 128), (1, 2, 256, 128),
                       (1, 1, 1, 128)):
        st = a3(s * h * d, d, h * d)
        n = L.fattn_bwd_workspace_split_bytes(b, h, s, d)
        rc = L.fattn_bwd_prep_f32(BAD, BAD, st, BAD, n, b, h, s, d, None)
        assert rc == 0, (b, h, s, d, _lib.last_error())


def sum_audit(b, h, s, d, causal):
    L = _lib.lib()
    f = L.fattn_internal_sum_audit
    f.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
    f.restype = ctypes.c_int
    out = (ctypes.c_int64 * 6)()
    assert f(b, h, s, d, int(causal), out) == 0
    return dict(zip(("grid", "targets", "bad", "twice", "covered", "keys"), list(out)))


def expected_keys(bh, s, d, causal):
    """Keys per split key block, from the rule's definition: 128 (two 16-key groups per wave) for
    non-causal d 64 from s 512 on when ceil(s / 128) b h >= 512 workgroups fill two per CU, and
    for non-causal d 32 when they make two rounds of three per CU (1536); else 64."""
    blocks = -(-s // 128) * bh
    if not causal and d == 64 and s >= 512 and blocks >= 512:
        return 128
    if not causal and d == 32 and blocks >= 1536:
        return 128
    return 64


def expected_sum_bh(bh, s, causal, keys=64):
    """Restated from the schedule's definition: every (b, h) has its tiles summed in step 2 while
    a (b, h) has at most 256 key blocks (the summing units read the partials at device scope, so
    where the key blocks ran does not matter)."""
    nkb = -(-s // keys)
    return 0 if nkb > 256 else bh


def expected_sum_grid(bh, s, keys=64):
    """Non-causal summing workgroups appended to step 2's grid, restated: XCD x's range of the
    (b, h)-major key blocks is [x F, (x + 1) F), F = floor(nkb b h / 8); each XCD's first mc nchunk
    workgroups take the (b, h)s whose last key block is in its range (mc: the most any range
    holds), then the (b, h)s whose last key block lies past 8 F take nchunk workgroups each, padded
    to a multiple of 8."""
    nkb, ntile = -(-s // keys), -(-s // 16)
    nchunk = -(-ntile // 3)
    f = nkb * bh // 8
    lasts = [(b_ * nkb + nkb - 1) for b_ in range(bh)]
    counts = [sum(1 for last in lasts if x * f <= last < (x + 1) * f) for x in range(8)]
    left = sum(1 for last in lasts if last >= 8 * f)
    return 8 * max(counts) * nchunk + -(-left * nchunk // 8) * 8


@pytest.mark.parametrize("causal", [False, True])
def test_step2_dq_sum_schedule(causal):
    """Step 2's dQ sums, over many shapes (the kernel's own scheduling functions, run on the
    host): a causal unit waits only for key blocks earlier in the grid; a non-causal unit of XCD x
    takes a (b, h) whose last key block runs on x (or, after those, one whose last key block is
    dealt round robin: the plan's order); no target lies past b h (the case a rounded-up per-XCD
    count once produced: nkb = 1, b h not a multiple of 8, e.g. h 17 s 50); no tile is summed
    twice; every tile of every (b, h) is summed (up to 256 key blocks per (b, h)), by the
    restated number of appended workgroups.
    Non-causal, the units are workgroups appended to the grid, ceil(ntile / 3) per (b, h) (every
    head_dim); causal, every key block's own workgroup sums its diagonal tiles (none appended; d 64
    and below: step 3 sums them at d 128)."""
    n = 0
    for s in (1, 16, 50, 64, 65, 100, 128, 200, 240, 333, 511, 512, 600, 1024, 2048):
        for bh in list(range(1, 41)) + [48, 64, 96, 128, 192, 256, 384]:
            for d in (32, 64, 128):
                a = sum_audit(1, bh, s, d, causal)
                keys = expected_keys(bh, s, d, causal)
                assert a["keys"] == keys, (s, bh, d, a)
                ntile, nkb = -(-s // 16), -(-s // keys)
                want_bh = expected_sum_bh(bh, s, causal, keys)
                assert a["bad"] == 0 and a["twice"] == 0, (s, bh, d, a)
                assert a["covered"] == want_bh * ntile, (s, bh, d, a, want_bh)
                if causal:
                    assert a["grid"] == 0 and a["targets"] == want_bh * nkb, (s, bh, d, a)
                else:
                    nchunk = -(-ntile // 3)
                    assert a["targets"] == want_bh * nchunk, (s, bh, d, a)
                    want_grid = expected_sum_grid(bh, s, keys) if want_bh else 0
                    assert a["grid"] == want_grid, (s, bh, d, a, want_grid)
                n += 1
    assert n > 1000
    # The advisor's case: b 1, h 17, s 50 (one key block per (b, h)): no target past b h; all 17
    # heads summed in step 2 (16 by the XCDs' ranges, the 17th by the round-robin rest).
    if not causal:
        a = sum_audit(1, 17, 50, 64, False)
        assert a["covered"] == 17 * 4 and a["bad"] == 0
        # The benchmark's shapes: config 2 (s 240) keeps 64-key blocks, config 5 (s 1024) 128.
        assert sum_audit(64, 6, 240, 64, False)["keys"] == 64
        assert sum_audit(16, 16, 1024, 64, False)["keys"] == 128


_HOOK_PROBE = r"""
import ctypes, json, sys
sys.path[:0] = [{repo!r}, {pkg!r}]
from candle_fused_attn import _lib
L = _lib.lib()
for name in ("fattn_internal_step2_sums", "fattn_internal_sum_shift", "fattn_internal_sum_give_up"):
    getattr(L, name).argtypes = [ctypes.c_int]
    getattr(L, name).restype = ctypes.c_int
L.fattn_internal_hooks.argtypes = [ctypes.POINTER(ctypes.c_int64)]
L.fattn_internal_hooks.restype = ctypes.c_int
audit = L.fattn_internal_sum_audit
audit.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
audit.restype = ctypes.c_int
def grid():
    out = (ctypes.c_int64 * 6)()
    assert audit(64, 6, 240, 64, 0, out) == 0
    return out[0]
rc = [L.fattn_internal_step2_sums(0), L.fattn_internal_sum_shift(3),
      L.fattn_internal_sum_give_up(5)]
err = _lib.last_error()
state = (ctypes.c_int64 * 3)()
allowed = L.fattn_internal_hooks(state)
print(json.dumps(dict(rc=rc, err=err, allowed=allowed, state=list(state), grid=grid())))
"""


@pytest.mark.parametrize("opt_in", [False, True])
def test_test_hooks_need_the_opt_in(opt_in):
    """The test hooks change how every later backward of the process runs, so they act only in a
    process that set FATTN_TEST_HOOKS=1 before the library loaded. Without it each refuses
    (FATTN_EINVAL, a message naming the variable) and changes nothing: step 2's dQ-sum schedule at
    config 2's shape keeps its appended summing workgroups, and the read-only state query shows the
    defaults (sums on, shift 0, no give-up pair). With it the same calls act."""
    import json
    import os
    import subprocess
    import sys
    env = {k: v for k, v in os.environ.items() if k != "FATTN_TEST_HOOKS"}
    if opt_in:
        env["FATTN_TEST_HOOKS"] = "1"
    code = _HOOK_PROBE.format(repo=str(REPO), pkg=str(REPO / "candle-fused-attn_amd"))
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stderr
    r = json.loads(res.stdout.strip().splitlines()[-1])
    default_grid = sum_audit(64, 6, 240, 64, False)["grid"]
    assert default_grid > 0
    if opt_in:
        assert r["rc"] == [1, 0, -1] and r["allowed"] == 1
        assert r["state"] == [0, 3, 5]
        assert r["grid"] == 0                     # sums off: nothing appended to step 2's grid
    else:
        assert r["rc"] == [_lib.FATTN_EINVAL] * 3 and r["allowed"] == 0
        assert "FATTN_TEST_HOOKS" in r["err"]
        assert r["state"] == [1, 0, -1]
        assert r["grid"] == default_grid          # the schedule is unchanged
