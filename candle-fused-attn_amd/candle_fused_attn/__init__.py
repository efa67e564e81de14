"""candle_fused_attn on MI355X: fused fp32 scaled-dot-product attention, forward and
deterministic backward, head_dim 32, 64 or 128 (the reference's is 64), on hand-written gfx950
kernels (libfattn.so).

The public surface mirrors the reference crate's (src/lib.rs:90-161): `fused_attention`,
`fused_attention_qkv`, `CUDA_HEAD_DIM`.
"""
from ._lib import FusedAttentionError, LIB_PATH, version
from .ops import (
    CUDA_HEAD_DIM,
    HIP_HEAD_DIM,
    HIP_HEAD_DIMS,
    float4_aligned,
    fused_attention,
    fused_attention_qkv,
    qkv_projection_of,
    reads_in_place,
    set_dq_sum,
    set_projection_route,
)

__all__ = [
    "CUDA_HEAD_DIM",
    "HIP_HEAD_DIM",
    "HIP_HEAD_DIMS",
    "FusedAttentionError",
    "LIB_PATH",
    "float4_aligned",
    "fused_attention",
    "fused_attention_qkv",
    "qkv_projection_of",
    "reads_in_place",
    "set_dq_sum",
    "set_projection_route",
    "version",
]
