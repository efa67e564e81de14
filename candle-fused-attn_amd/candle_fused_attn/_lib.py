"""ctypes binding of libfattn.so (include/fattn.h).

The library is the only compute path: if it is missing or fails to load, every call raises
FusedAttentionError -- there is no CPU or composed fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  -- loaded first, so libfattn binds to torch's HIP runtime

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libfattn.so"

# Return codes (include/fattn.h).
FATTN_EINVAL = -1
FATTN_EHEADDIM = -2
FATTN_EALIGN = -3
FATTN_ERANGE = -4
FATTN_EWORKSPACE = -5

# Every entry point include/fattn.h declares.
EXPORTS = (
    "fattn_fwd_f32",
    "fattn_bwd_workspace_bytes",
    "fattn_bwd_workspace_min_bytes",
    "fattn_bwd_workspace_split_bytes",
    "fattn_bwd_prep_f32",
    "fattn_bwd_main_f32",
    "fattn_bwd_dq_f32",
    "fattn_bwd_f32",
    "fattn_bwd_f32_noalloc",
    "fattn_fwd_f32_d64",
    "fattn_bwd_prep_f32_d64",
    "fattn_bwd_main_f32_d64",
    "fattn_bwd_dq_f32_d64",
    "fattn_bwd_f32_d64",
    "fattn_qkv_forward",
    "fattn_qkv_backward",
    "fattn_forward",
    "fattn_backward",
    "fattn_last_error",
    "fattn_version",
    "fattn_bwd_status",
)


class FusedAttentionError(RuntimeError):
    """An error of the fused attention op; the message carries the reference's prefix
    (`fused_attention:` or `fused_attention_qkv:`), and `code` the C-ABI return code."""

    def __init__(self, msg: str, code: int = 0):
        super().__init__(msg)
        self.code = code


_lib = None

I64 = ctypes.c_int64
P = ctypes.c_void_p
A3 = ctypes.POINTER(ctypes.c_int64)
C_INT = ctypes.c_int
C_FLOAT = ctypes.c_float
SIZE = ctypes.c_size_t


def _declare(L: ctypes.CDLL) -> None:
    L.fattn_last_error.argtypes = []
    L.fattn_last_error.restype = ctypes.c_char_p
    L.fattn_version.argtypes = []
    L.fattn_version.restype = ctypes.c_char_p
    for name in ("fattn_bwd_workspace_bytes", "fattn_bwd_workspace_min_bytes",
                 "fattn_bwd_workspace_split_bytes"):
        getattr(L, name).argtypes = [I64, I64, I64, I64]
        getattr(L, name).restype = SIZE
    for sfx in ("", "_d64"):
        getattr(L, "fattn_fwd_f32" + sfx).argtypes = [P, P, P, P, P, I64, I64, I64, I64, C_FLOAT,
                                                      C_INT, A3, A3, A3, P]
        getattr(L, "fattn_bwd_prep_f32" + sfx).argtypes = [P, P, A3, P, SIZE, I64, I64, I64, I64,
                                                           P]
        getattr(L, "fattn_bwd_main_f32" + sfx).argtypes = [P, P, P, P, P, P, P, P, SIZE, I64,
                                                           I64, I64, I64, C_FLOAT, C_INT, A3, A3,
                                                           A3, A3, P]
        getattr(L, "fattn_bwd_dq_f32" + sfx).argtypes = [P, P, SIZE, I64, I64, I64, I64, C_FLOAT,
                                                         C_INT, P]
        getattr(L, "fattn_bwd_f32" + sfx).argtypes = [P, P, P, P, P, P, P, P, SIZE, I64, I64, I64,
                                                      I64, C_FLOAT, C_INT, A3, A3, A3, A3, P]
    L.fattn_bwd_f32_noalloc.argtypes = [P, P, P, P, P, P, P, I64, I64, I64, I64, C_FLOAT, C_INT,
                                        A3, A3, A3, A3, P]
    L.fattn_qkv_forward.argtypes = [P, I64, A3, A3, I64, C_FLOAT, C_INT, P, P, P]
    L.fattn_qkv_backward.argtypes = [P, I64, A3, A3, I64, C_FLOAT, C_INT, P, P, P, I64, A3, A3,
                                     P, P, SIZE, P]
    L.fattn_forward.argtypes = [P, I64, A3, A3, P, I64, A3, A3, P, I64, A3, A3, C_FLOAT, C_INT,
                                P, P, P]
    L.fattn_backward.argtypes = [P, I64, A3, A3, P, I64, A3, A3, P, I64, A3, A3, C_FLOAT, C_INT,
                                 P, P, P, I64, A3, A3, P, P, SIZE, P]
    L.fattn_bwd_status.argtypes = [P, SIZE, I64, I64, I64, P, ctypes.POINTER(C_INT)]
    for name in EXPORTS:
        if name not in ("fattn_last_error", "fattn_version") and "workspace" not in name:
            getattr(L, name).restype = C_INT


def lib() -> ctypes.CDLL:
    """The loaded libfattn.so; raises FusedAttentionError if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FusedAttentionError(
                f"fused_attention: {LIB_PATH} is not built (run __graft_entry__.build() or "
                "python candle-fused-attn_amd/build.py); there is no fallback path")
        try:
            L = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise FusedAttentionError(f"fused_attention: cannot load {LIB_PATH}: {e}") from e
        _declare(L)
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().fattn_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != 0:
        raise FusedAttentionError(last_error() or f"fused_attention: error {rc}", rc)


def arr(values) -> ctypes.Array:
    vals = [int(x) for x in values]
    return (ctypes.c_int64 * len(vals))(*vals)


def version() -> str:
    return lib().fattn_version().decode()
