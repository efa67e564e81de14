"""The two public operators, mirroring the reference crate's API (src/lib.rs:90-178).

- fused_attention_qkv(qkv, heads, scale, causal): the fused [b, s, 3 h d] projection in, the
  merged [b, s, h d] output out; its backward writes ONE gradient shaped like qkv
  (src/lib.rs:96-125).
- fused_attention(q, k, v, scale, causal): [b, h, s, d] operands with any strides in, a
  [b, h, s, d] result out that is the transposed view of a contiguous [b, s, h, d] buffer, so
  merging heads is free (src/lib.rs:127-161).

Both are torch autograd Functions standing in for candle's CustomOp1 / CustomOp3: the forward
keeps the row log-sum-exp L [b, h, s] as saved state and outputs O alone; the backward reads L
(it is not consumed, so a graph can be differentiated twice, src/lib.rs:301-315). Operands are
read in place when head_dim is contiguous and the offset and other strides are multiples of 4
floats; otherwise they are copied first (src/lib.rs:110-118, :163-178, :368-380).

Every launch goes to torch's current HIP stream of the operand's device through libfattn.so;
there is no CPU path and no fallback: a CPU tensor, a non-f32 dtype or a missing library is an
error.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import FusedAttentionError, arr, check

# The reference's head dimension (src/lib.rs:91, CUDA_HEAD_DIM), and those the kernels here are
# built for.
CUDA_HEAD_DIM = 64
HIP_HEAD_DIMS = (32, 64, 128)
HIP_HEAD_DIM = CUDA_HEAD_DIM


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _storage(t: torch.Tensor):
    """(storage base pointer, element offset): a candle Layout's start_offset view."""
    return ctypes.c_void_p(t.untyped_storage().data_ptr()), int(t.storage_offset())


def _require(who: str, name: str, t: torch.Tensor, device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise FusedAttentionError(f"{who}: {name} must be a tensor")
    if t.dtype != torch.float32:
        raise FusedAttentionError(f"{who}: f32 only")
    if t.device.type != "cuda":
        raise FusedAttentionError(
            f"{who}: {name} is not on a HIP device (this operator has no CPU path)")
    if device is not None and t.device != device:
        raise FusedAttentionError(f"{who}: q, k, v must be on one device")


def _fresh(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy at offset 0 (contiguous() alone may keep a misaligned offset)."""
    return t.clone(memory_format=torch.contiguous_format)


def _qkv_aligned(t: torch.Tensor) -> bool:
    """src/lib.rs:111-113: offset and [sb, ss] multiples of 4, last stride 1."""
    if t.dim() != 3:
        return True  # the geometry check reports the rank
    sb, ss, sl = t.stride()
    return t.storage_offset() % 4 == 0 and sl == 1 and sb % 4 == 0 and ss % 4 == 0


def float4_aligned(t: torch.Tensor) -> bool:
    """src/lib.rs:163-168: a [b, h, s, d] layout whose offset and (b, h, s) strides are
    multiples of 4 floats, d contiguous."""
    if t.dim() != 4:
        return True
    sb, sh, ss, sd = t.stride()
    return (t.storage_offset() % 4 == 0 and sd == 1 and sb % 4 == 0 and sh % 4 == 0
            and ss % 4 == 0)


def float4_rows(t: torch.Tensor) -> torch.Tensor:
    """`t` itself when float4_aligned, else a contiguous copy (src/lib.rs:170-178)."""
    return t if float4_aligned(t) else _fresh(t)


def reads_in_place(t: torch.Tensor) -> bool:
    """Whether an operand is read without a copy (the audit's P5 predicate): a rank-3 qkv
    projection or a rank-4 [b, h, s, d] operand, f32, rows float4-aligned."""
    if t.dtype != torch.float32:
        return False
    if t.dim() == 3:
        return _qkv_aligned(t)
    if t.dim() == 4:
        return float4_aligned(t)
    return False


def _aligned_grad(g: torch.Tensor) -> torch.Tensor:
    """src/lib.rs:370-380: the gradient itself when its offset is a multiple of 4, its last
    stride 1 and every other stride 1 or a multiple of 4; else a contiguous copy."""
    st = g.stride()
    ok = (g.storage_offset() % 4 == 0 and (len(st) == 0 or st[-1] == 1)
          and all(s == 1 or s % 4 == 0 for s in st))
    return g if ok else _fresh(g)


_DQ_SUM_MODES = ("auto", "split", "turns")
_dq_sum = "auto"


def set_dq_sum(mode: str) -> str:
    """How the backward sums dQ over key blocks; returns the previous setting. Both ways are
    deterministic (a fixed order per query tile):
      "split": each key block writes its partials to the workspace (about 4 s^2 b h bytes) and a
               third kernel sums them -- no workgroup waits on another;
      "turns": key blocks add into dQ in place under turn counters (minimum workspace);
      "auto" (default): "split" unless its workspace exceeds the library's FATTN_SPLIT_MAX_BYTES;
               then, at head_dim <= 64, "split" by chunks of (b, h) pairs (each chunk's state in
               a workspace within that size; the same results) where the chunks fill the chip,
               else "turns".
    """
    global _dq_sum
    if mode not in _DQ_SUM_MODES:
        raise ValueError(f"set_dq_sum: mode must be one of {_DQ_SUM_MODES}, got {mode!r}")
    prev, _dq_sum = _dq_sum, mode
    return prev


def _workspace(b: int, h: int, s: int, d: int, device: torch.device) -> torch.Tensor:
    L = _lib.lib()
    size = {"auto": L.fattn_bwd_workspace_bytes, "split": L.fattn_bwd_workspace_split_bytes,
            "turns": L.fattn_bwd_workspace_min_bytes}[_dq_sum]
    nbytes = int(size(b, h, s, d))
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


class _FusedAttentionQkv(torch.autograd.Function):
    """FusedAttentionQkv (src/lib.rs:493-590) as an autograd Function."""

    @staticmethod
    def forward(ctx, qkv: torch.Tensor, heads: int, scale: float, causal: bool):
        who = "fused_attention_qkv"
        L = _lib.lib()
        if qkv.dim() != 3:
            raise FusedAttentionError(
                f"{who}: a [b, s, 3 h d] tensor expected, got shape {list(qkv.shape)}")
        b, s, three_hd = qkv.shape
        out = torch.empty((b, s, three_hd // 3), dtype=torch.float32, device=qkv.device)
        lse = torch.empty((b, max(int(heads), 0), s), dtype=torch.float32, device=qkv.device)
        base, off = _storage(qkv)
        check(L.fattn_qkv_forward(base, off, arr(qkv.shape), arr(qkv.stride()), int(heads),
                                  float(scale), int(bool(causal)), _ptr(out), _ptr(lse),
                                  _stream(qkv)))
        ctx.save_for_backward(qkv, out, lse)
        ctx.heads, ctx.scale, ctx.causal = int(heads), float(scale), bool(causal)
        return out

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        qkv, out, lse = ctx.saved_tensors
        if qkv.dtype != torch.float32:
            raise FusedAttentionError("fused_attention_qkv: f32 only")
        grad = _aligned_grad(grad)
        b, s, three_hd = qkv.shape
        dqkv = torch.empty((b, s, three_hd), dtype=torch.float32, device=qkv.device)
        ws = _workspace(b, ctx.heads, s, three_hd // 3 // max(ctx.heads, 1), qkv.device)
        base, off = _storage(qkv)
        gbase, goff = _storage(grad)
        check(_lib.lib().fattn_qkv_backward(
            base, off, arr(qkv.shape), arr(qkv.stride()), ctx.heads, ctx.scale,
            int(ctx.causal), _ptr(out), _ptr(lse), gbase, goff, arr(grad.shape),
            arr(grad.stride()), _ptr(dqkv), _ptr(ws), ws.numel(), _stream(qkv)))
        return dqkv, None, None, None


class _FusedAttention(torch.autograd.Function):
    """FusedAttention (src/lib.rs:382-491) as an autograd Function: [b, h, s, d] in, the raw
    [b, s, h, d] output out."""

    @staticmethod
    def forward(ctx, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                causal: bool):
        L = _lib.lib()
        if q.dim() != 4:
            raise FusedAttentionError(
                f"fused_attention: a [b, h, s, d] tensor expected, got shape {list(q.shape)}")
        b, h, s, d = q.shape
        out = torch.empty((b, s, h, d), dtype=torch.float32, device=q.device)
        lse = torch.empty((b, h, s), dtype=torch.float32, device=q.device)
        (qb, qo), (kb, ko), (vb, vo) = _storage(q), _storage(k), _storage(v)
        check(L.fattn_forward(qb, qo, arr(q.shape), arr(q.stride()),
                              kb, ko, arr(k.shape), arr(k.stride()),
                              vb, vo, arr(v.shape), arr(v.stride()),
                              float(scale), int(bool(causal)), _ptr(out), _ptr(lse),
                              _stream(q)))
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.scale, ctx.causal = float(scale), bool(causal)
        return out

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        q, k, v, out, lse = ctx.saved_tensors
        if q.dtype != torch.float32:
            raise FusedAttentionError("fused_attention: f32 only")
        grad = _aligned_grad(grad)
        b, h, s, d = q.shape
        dqkv = torch.empty((b, s, 3, h, d), dtype=torch.float32, device=q.device)
        ws = _workspace(b, h, s, d, q.device)
        (qb, qo), (kb, ko), (vb, vo) = _storage(q), _storage(k), _storage(v)
        gbase, goff = _storage(grad)
        check(_lib.lib().fattn_backward(
            qb, qo, arr(q.shape), arr(q.stride()), kb, ko, arr(k.shape), arr(k.stride()),
            vb, vo, arr(v.shape), arr(v.stride()), ctx.scale, int(ctx.causal), _ptr(out),
            _ptr(lse), gbase, goff, arr(grad.shape), arr(grad.stride()), _ptr(dqkv), _ptr(ws),
            ws.numel(), _stream(q)))
        # dQ, dK, dV: narrow views of the one buffer, each [b, h, s, d] (src/lib.rs:484-485).
        return (dqkv[:, :, 0].transpose(1, 2), dqkv[:, :, 1].transpose(1, 2),
                dqkv[:, :, 2].transpose(1, 2), None, None)


def fused_attention_qkv(qkv: torch.Tensor, heads: int, scale: float,
                        causal: bool) -> torch.Tensor:
    """Fused attention over a fused qkv projection: softmax(q k^T scale) v, keys after the
    query masked when `causal` (src/lib.rs:96-125).

    qkv: [batch, seq, 3 heads head_dim] f32 on a HIP device, laid out [q | k | v] along the last
    dimension; returns [batch, seq, heads head_dim], heads merged. The backward writes one
    gradient shaped like qkv.
    """
    _require("fused_attention_qkv", "qkv", qkv)
    if not _qkv_aligned(qkv):
        qkv = _fresh(qkv)
    return _FusedAttentionQkv.apply(qkv, heads, scale, causal)


_route_projection = True


def set_projection_route(on: bool) -> bool:
    """Whether fused_attention hands the head-split views of one projection to the projection's
    node (the default) or to its own general node (for tests comparing the two); returns the
    previous setting."""
    global _route_projection
    prev, _route_projection = _route_projection, bool(on)
    return prev


def qkv_projection_of(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """The contiguous [b, s, 3 h d] projection whose head-split views q, k, v are (q, k, v its
    parts at element offsets 0, h d, 2 h d, strides (s 3hd, d, 3hd, 1): the layout candle-mi
    feeds fused_attention, tests/parity.rs:38-50), or None. Only where the op on the projection
    is the same computation with the same gradients: a head_dim the kernels take, rows
    float4-aligned, and q, k, v differentiable views of it (not detached leaves, none retaining
    its own gradient, none with a backward hook registered), so every gradient reaches the
    projection either way.

    Routed, the graph runs from the output to the projection's node directly: the views' own
    nodes are not on it, so torch.autograd.grad(out, [q, k, v]) finds them unused (take the
    gradient of the projection, or turn routing off with set_projection_route(False))."""
    base = q._base
    if base is None or k._base is not base or v._base is not base or base.dim() != 3:
        return None
    if q.dim() != 4 or not base.is_contiguous() or base.dtype != torch.float32:
        return None
    b, h, s, d = q.shape
    if d not in HIP_HEAD_DIMS or tuple(base.shape) != (b, s, 3 * h * d) or not _qkv_aligned(base):
        return None
    for i, t in enumerate((q, k, v)):
        if (tuple(t.shape) != (b, h, s, d) or t.stride() != (s * 3 * h * d, d, 3 * h * d, 1)
                or t.storage_offset() - base.storage_offset() != i * h * d):
            return None
        if not torch.is_grad_enabled():
            continue  # no graph is recorded: nothing to route
        if t.requires_grad != base.requires_grad or t.retains_grad:
            return None
        if t.requires_grad and t.grad_fn is None:
            return None
        if t._backward_hooks:  # a hook on the view would never run on the projection's path
            return None
    return base


def fused_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                    causal: bool) -> torch.Tensor:
    """Fused scaled-dot-product attention: softmax(q k^T scale) v, keys after the query masked
    when `causal` (src/lib.rs:127-161).

    q, k, v: [batch, heads, seq, head_dim] f32 on one HIP device, any strides (copied first when
    the kernels cannot read them in place). Returns [batch, heads, seq, head_dim], a transposed
    view of a contiguous [batch, seq, heads, head_dim] buffer.

    When q, k, v are the head-split views of one contiguous [b, s, 3 h d] projection, the op is
    applied to the projection itself (fused_attention_qkv's node, the same kernels and bits):
    its gradient is the backward's one [b, s, 3, h, d] buffer, where three view gradients would
    make autograd copy them back into a projection-shaped tensor (at b 64, s 240, h 6, d 64: a
    70.8 MB copy and an add, 72 us of a 200 us step).
    """
    _require("fused_attention", "q", q)
    _require("fused_attention", "k", k, q.device)
    _require("fused_attention", "v", v, q.device)
    base = qkv_projection_of(q, k, v) if _route_projection else None
    if base is not None:
        b, h, s, d = q.shape
        out = _FusedAttentionQkv.apply(base, h, scale, causal)
        return out.view(b, s, h, d).transpose(1, 2)
    q, k, v = float4_rows(q), float4_rows(k), float4_rows(v)
    return _FusedAttention.apply(q, k, v, scale, causal).transpose(1, 2)
