"""candle_fused_attn on MI355X: fused fp32 scaled-dot-product attention, head_dim 64, forward and
deterministic backward, on hand-written gfx950 kernels (libfattn.so).

The public surface mirrors the reference crate's (src/lib.rs:90-161): `fused_attention`,
`fused_attention_qkv`, `CUDA_HEAD_DIM`.
"""
from ._lib import FusedAttentionError, LIB_PATH, version
from .ops import (
    CUDA_HEAD_DIM,
    HIP_HEAD_DIM,
    float4_aligned,
    fused_attention,
    fused_attention_qkv,
    reads_in_place,
    set_dq_sum,
)

__all__ = [
    "CUDA_HEAD_DIM",
    "HIP_HEAD_DIM",
    "FusedAttentionError",
    "LIB_PATH",
    "float4_aligned",
    "fused_attention",
    "fused_attention_qkv",
    "reads_in_place",
    "set_dq_sum",
    "version",
]
